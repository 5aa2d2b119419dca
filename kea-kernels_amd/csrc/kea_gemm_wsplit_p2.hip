// Wave-split GEMM kernel instances for 2 activation parts.
#define KEA_WSPLIT_P 2
#include "kea_gemm_wsplit_inst.h"
