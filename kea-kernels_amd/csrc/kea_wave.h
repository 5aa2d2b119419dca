// Wave64 reductions without LDS round trips.
//
// wave_sum is the xor butterfly with offsets 1, 2, 4, 8, 16, 32 (every lane adds its partner l ^ off at each step),
// so every lane ends with the same, fixed-order total that a CPU restatement reproduces. The first four steps run
// on DPP lane permutes: quad_perm [1,0,3,2] and [2,3,0,1] are exactly l ^ 1 and l ^ 2; after them the four lanes of a
// quad hold the same value, so row_half_mirror (l -> 7 - l within 8 lanes) reads the same value as l ^ 4, and after
// that row_mirror (l -> 15 - l within 16) the same as l ^ 8. The 16 lanes of a row then agree, and the last two steps
// are (r0 + r1) + (r2 + r3) over the four row values read with readlane. wave_max is the same tree with fmaxf.
#pragma once

#include <hip/hip_runtime.h>

namespace kea {

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_value(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ __forceinline__ float wave_sum(float v) {
    v = v + dpp<0xB1>(v);   // quad_perm [1,0,3,2]: l ^ 1
    v = v + dpp<0x4E>(v);   // quad_perm [2,3,0,1]: l ^ 2
    v = v + dpp<0x141>(v);  // row_half_mirror: the value of l ^ 4
    v = v + dpp<0x140>(v);  // row_mirror: the value of l ^ 8
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

}  // namespace kea
