#define KEA_ROWS_P 1
#include "kea_gemm_rows_inst.h"
