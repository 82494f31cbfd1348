// Long-K W-only streaming kernels (wq_streamk.h): int4, 32 chunks per wave
// (K <= 32768), single pass only (the multi-pass form would hold 128 weight
// registers per lane and spill).
#include "wq_streamk.h"

TM_STREAMK_S(4, 1, 32)
TM_STREAMK_S(4, 2, 32)
// split-K, M <= 16: K above 32768 in slices of at most 32768
TM_STREAMK_KS(4, 32)
