// The key-split attention's workspace and the merge of its two halves, shared by the attention kernels
// (kea_encoder.hip) and the merging quantizer (kea_quantize.hip), so that both compute the same bits.
#pragma once

#include <hip/hip_runtime.h>

namespace kea {

// Workspace: the unnormalised partial outputs O_s = sum_j exp(s_ij - m_s) v_j of the two key halves s = 0, 1, then
// the rows' softmax statistics (m_s, l_s = sum_j exp(s_ij - m_s)) per head.
//   o  [2][rows][heads * 128] floats, ml [2][rows][heads][2] floats; rows = batch * T.
struct SplitWs {
    float *o;
    float *ml;
};
// The split applies to sequences of at most 128 frames with an even number of 16-key tiles, and only where the
// unsplit grid (heads x tiles x batch workgroups) leaves at least half of the 256 CUs idle.
inline bool attention_splits(long long batch, long long t, int heads) {
    const long long nkt = (t + 15) / 16;
    return t <= 128 && nkt % 2 == 0 && heads * nkt * batch * 2 <= 256;
}
inline __host__ __device__ long long split_ws_floats(long long rows, int heads) {
    return 2 * rows * heads * 128 + 2 * rows * heads * 2;
}
inline __host__ __device__ SplitWs split_ws(void *base, long long rows, int heads) {
    float *o = (float *)base;
    return SplitWs{o, o + 2 * rows * heads * 128};
}

// out = (O0 exp(m0 - m) + O1 exp(m1 - m)) / (l0 exp(m0 - m) + l1 exp(m1 - m)), m = max(m0, m1), for four
// consecutive features of one (row, head).
__device__ __forceinline__ void merge_halves(const float4 o0, const float4 o1, const float2 ml0, const float2 ml1,
                                             float *out4) {
    const float m = fmaxf(ml0.x, ml1.x);
    const float a0 = expf(ml0.x - m), a1 = expf(ml1.x - m);
    const float inv = 1.0f / (ml0.y * a0 + ml1.y * a1);
    out4[0] = (o0.x * a0 + o1.x * a1) * inv;
    out4[1] = (o0.y * a0 + o1.y * a1) * inv;
    out4[2] = (o0.z * a0 + o1.z * a1) * inv;
    out4[3] = (o0.w * a0 + o1.w * a1) * inv;
}

// The merged features k .. k + 3 (k % 4 == 0) of row `row` (head k / 128).
__device__ __forceinline__ void merged4(const SplitWs ws, long long rows, int heads, long long row, int k,
                                        float *out4) {
    const long long hd = (long long)heads * 128;
    const int h = k >> 7;
    const float4 o0 = *(const float4 *)(ws.o + row * hd + k);
    const float4 o1 = *(const float4 *)(ws.o + (rows + row) * hd + k);
    const float2 ml0 = *(const float2 *)(ws.ml + (row * heads + h) * 2);
    const float2 ml1 = *(const float2 *)(ws.ml + ((rows + row) * heads + h) * 2);
    merge_halves(o0, o1, ml0, ml1, out4);
}

}  // namespace kea
