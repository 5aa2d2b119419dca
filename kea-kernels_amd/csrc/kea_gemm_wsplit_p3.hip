// Wave-split GEMM kernel instances for 3 activation parts.
#define KEA_WSPLIT_P 3
#include "kea_gemm_wsplit_inst.h"
