// Long-K W-only streaming kernels (wq_streamk.h): int4, 16 chunks per wave (K <= 16384).
#include "wq_streamk.h"

TM_STREAMK_S(4, 1, 16)
TM_STREAMK_S(4, 2, 16)
TM_STREAMK_M(4, 16)
