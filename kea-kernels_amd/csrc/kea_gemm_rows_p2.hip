#define KEA_ROWS_P 2
#include "kea_gemm_rows_inst.h"
