// The row-quantizing GEMM (kea_gemm_rows_inst.h): kernel instance lookup, shared with the host code of kea_gemm.hip
// (argument validation and the launch).
#pragma once

#include <hip/hip_runtime.h>

#include "kea_gemm_wsplit.h"

namespace kea {

using RowsFn = void (*)(const float *, const uint32_t *, const void *, int, int, int, int, int, Params);

// Dynamic LDS of a launch: the wave partial tiles (as the wave-split kernel) and each wave's int8 code staging rows
// (16 rows of s * 64 bytes, padded by 16).
inline int rows_lds_bytes(int parts, const WsplitTile &t, int s) {
    return wsplit_lds_bytes(parts, t) + t.nw * 16 * (s * 64 + 16);
}

// The kernel instance for a KEA_ROWS_* mode on wave-split tile index `tile` with `s` k-steps per wave (K = nw * s * 64),
// or nullptr where none exists (modes other than KEA_ROWS_PLAIN need K = 1024 on four waves; registers must fit).
// Defined per activation part count.
RowsFn rows_pick_p1(int wbits, int mode, int tile, int s);
RowsFn rows_pick_p2(int wbits, int mode, int tile, int s);
RowsFn rows_pick_p3(int wbits, int mode, int tile, int s);

}  // namespace kea
