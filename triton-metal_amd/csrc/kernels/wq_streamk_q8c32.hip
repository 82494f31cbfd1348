// Long-K W-only streaming kernels (wq_streamk.h): int8, 32 chunks per wave (K <= 16384).
#include "wq_streamk.h"

TM_STREAMK_S(8, 1, 32)
TM_STREAMK_S(8, 2, 32)
TM_STREAMK_M(8, 32)
// split-K: K above 16384 in slices of at most 16384
TM_STREAMK_KS(8, 32)
TM_STREAMK_KM(8, 32)
