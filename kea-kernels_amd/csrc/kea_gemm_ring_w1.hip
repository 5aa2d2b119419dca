// LDS-ring GEMM kernel instances for 1-bit sign weights.
#define KEA_RING_WBITS 1
#include "kea_gemm_ring_inst.h"
