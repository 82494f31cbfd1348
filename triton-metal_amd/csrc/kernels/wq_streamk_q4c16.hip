// Long-K W-only streaming kernels (wq_streamk.h): int4, 16 chunks per wave (K <= 16384).
#include "wq_streamk.h"

TM_STREAMK_S(4, 1, 16)
TM_STREAMK_S(4, 2, 16)
TM_STREAMK_M(4, 16)
// split-K, 17 <= M <= 64: K above 16384 in slices of at most 16384
TM_STREAMK_KM(4, 16)
