#define KEA_ROWS_P 3
#include "kea_gemm_rows_inst.h"
