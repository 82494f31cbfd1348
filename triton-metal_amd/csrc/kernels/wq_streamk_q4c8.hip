// Long-K W-only streaming kernels (wq_streamk.h): int4, 8 chunks per wave (K <= 8192).
#include "wq_streamk.h"

TM_STREAMK_S(4, 1, 8)
TM_STREAMK_S(4, 2, 8)
TM_STREAMK_M(4, 8)
