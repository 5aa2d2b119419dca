// Wave-split GEMM kernel instances with per-group weight scales for 2 activation parts.
#define KEA_WSPLIT_P 2
#include "kea_gemm_wsplit_group_inst.h"
