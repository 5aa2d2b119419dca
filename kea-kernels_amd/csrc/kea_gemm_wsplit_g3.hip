// Wave-split GEMM kernel instances with per-group weight scales for 3 activation parts.
#define KEA_WSPLIT_P 3
#include "kea_gemm_wsplit_group_inst.h"
