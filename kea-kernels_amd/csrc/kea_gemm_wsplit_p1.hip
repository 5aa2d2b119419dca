// Wave-split GEMM kernel instances for 1 activation part.
#define KEA_WSPLIT_P 1
#include "kea_gemm_wsplit_inst.h"
