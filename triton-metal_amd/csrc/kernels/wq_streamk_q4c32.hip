// Long-K W-only streaming kernels (wq_streamk.h): int4, 32 chunks per wave
// (K <= 32768), single pass only (the multi-pass form would hold 128 weight
// registers per lane and spill).
#include "wq_streamk.h"

TM_STREAMK_S(4, 1, 32)
TM_STREAMK_S(4, 2, 32)
