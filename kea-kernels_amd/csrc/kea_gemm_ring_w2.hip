// LDS-ring GEMM kernel instances for 2-bit ternary weights.
#define KEA_RING_WBITS 2
#include "kea_gemm_ring_inst.h"
