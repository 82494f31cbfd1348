// Long-K W-only streaming kernels (wq_streamk.h): int8, 16 chunks per wave (K <= 8192).
#include "wq_streamk.h"

TM_STREAMK_S(8, 1, 16)
TM_STREAMK_S(8, 2, 16)
TM_STREAMK_M(8, 16)
