// Wave-split GEMM kernel instances with per-group weight scales for 1 activation part.
#define KEA_WSPLIT_P 1
#include "kea_gemm_wsplit_group_inst.h"
