// The building blocks of the wave-split GEMM (kea_gemm_wsplit_inst.h): the weight loads, the MFMA sequence, the exact
// LDS reduction over the waves and the epilogue dispatch of one 16x16 block. Every function is force-inlined over compile-time shapes, so the arrays stay in registers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kea_gemm_common.h"

namespace kea {

// The aligned 32-bit word holding element i of an f32 or f16 vector (f16: the half is selected at conversion time by
// raw_to_f32 with the same v and i). The word lies inside the 4-byte block of an in-bounds element, so it never
// reaches past a page the vector touches.
__device__ __forceinline__ uint32_t load_raw(const void *v, bool f16, uint32_t i) {
    const char *a = (const char *)v + (f16 ? 2u * i : 4u * i);
    return *(const uint32_t *)__builtin_align_down(a, 4);  // keeps the pointer's (global) address space
}
__device__ __forceinline__ float raw_to_f32(uint32_t raw, bool f16, const void *v, uint32_t i) {
    const uint32_t hi = (uint32_t)(((uintptr_t)v >> 1) + i) & 1u;  // f16: which half of the word
    const float h = (float)__builtin_bit_cast(_Float16, (uint16_t)(raw >> (hi * 16)));
    return f16 ? h : __builtin_bit_cast(float, raw);
}

// The wave's weight words: WPW native words per lane for each of the NT n-tiles from the tile at column n0, starting
// at word j0 (J words per lane per n-tile). RAGGED = false: complete quads of words (or one word per wave), loaded
// with 64- or 128-bit vector loads; otherwise general per-word addressing (a short last quad has lane stride < 4,
// words past J load any valid word, whose activations are zero).
template <int NT, int WPW, bool RAGGED>
__device__ __forceinline__ void wsplit_load_w(const uint32_t *w, int n0, int NTILES, int J, int j0, uint32_t lane16,
                                              uint32_t (&wv)[NT][WPW]) {
#pragma unroll
    for (int jn = 0; jn < NT; ++jn) {
        // wave-uniform base of the n-tile's words, plus a 32-bit per-lane byte offset (SGPR-base loads)
        const int t = min((n0 >> 4) + jn, NTILES - 1);
        const char *tb = (const char *)(w + (long long)t * J * 64);
        if constexpr (WPW == 1 || RAGGED) {
#pragma unroll
            for (int u = 0; u < WPW; ++u) {
                const int j = min(j0 + u, J - 1), jq = j & ~3;
                const int wq = min(4, J - jq);
                wv[jn][u] = *(const uint32_t *)(tb + jq * 256 + (j & 3) * 4 + lane16 / 4 * (uint32_t)wq);
            }
        } else if constexpr (WPW == 2) {
            const uint2 v = *(const uint2 *)(tb + (j0 >> 2) * 1024 + ((j0 >> 1) & 1) * 8 + lane16);
            wv[jn][0] = v.x; wv[jn][1] = v.y;
        } else {
#pragma unroll
            for (int g = 0; g < WPW / 4; ++g) {
                const uint4 v = *(const uint4 *)(tb + ((j0 >> 2) + g) * 1024 + lane16);
                wv[jn][4 * g] = v.x; wv[jn][4 * g + 1] = v.y; wv[jn][4 * g + 2] = v.z; wv[jn][4 * g + 3] = v.w;
            }
        }
    }
}

// 1-bit weights, bit-plane layout: the wave's S 16-byte units (one per k-step from the wave's first k-step s0) of the
// 128-row group holding the tile (n0 / 128; every tile lies inside one group: BN divides 128). RAGGED: k-steps past
// the matrix load its last unit (their activations are zero).
template <int S, bool RAGGED>
__device__ __forceinline__ void wsplit_load_planes(const uint32_t *w, int n0, int ksteps, int s0, int lane,
                                                   uint4 (&wu)[S]) {
    // wave-uniform base of the group's units, plus a 32-bit per-lane byte offset (SGPR-base loads)
    const char *gb = (const char *)(w + (long long)(n0 >> 7) * ksteps * 256);
#pragma unroll
    for (int t = 0; t < S; ++t) {
        const int st = RAGGED ? min(s0 + t, ksteps - 1) : s0 + t;
        wu[t] = *(const uint4 *)(gb + ((uint32_t)st * 64u + (uint32_t)lane) * 16u);
    }
}

// 1-bit bit-plane MFMAs over the wave's S k-steps: n-tile jn of the tile is plane p0 + jn of the group, whose operand
// is the unit masked with 0x01010101 << plane (int8 values 0 / 2^plane, plane 7: -128; one AND per 4 weights),
// accumulated in acc[c][i][jn]; acc[c][i][NT] accumulates the activation row sums (an all-ones operand). The exact
// signed sums follow after the reduction (wsplit_planes_fix).
template <int P, int RM, int NT, int S>
__device__ __forceinline__ void wsplit_mfma_planes(const uint4 (&wu)[S], const v4i (&af)[P][RM][S], int p0,
                                                   v4i (&acc)[P][RM][NT + 1]) {
#pragma unroll
    for (int c = 0; c < P; ++c)
#pragma unroll
        for (int i = 0; i < RM; ++i)
#pragma unroll
            for (int jn = 0; jn <= NT; ++jn) acc[c][i][jn] = (v4i){0, 0, 0, 0};
    const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
#pragma unroll
    for (int t = 0; t < S; ++t) {
#pragma unroll
        for (int jn = 0; jn < NT; ++jn) {
            const uint32_t mask = 0x01010101u << (p0 + jn);  // wave-uniform
            v4i bf;
            bf[0] = (int)(wu[t].x & mask); bf[1] = (int)(wu[t].y & mask);
            bf[2] = (int)(wu[t].z & mask); bf[3] = (int)(wu[t].w & mask);
#pragma unroll
            for (int c = 0; c < P; ++c)
#pragma unroll
                for (int i = 0; i < RM; ++i)
                    acc[c][i][jn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf, af[c][i][t], acc[c][i][jn], 0, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < P; ++c)
#pragma unroll
            for (int i = 0; i < RM; ++i)
                acc[c][i][NT] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ones, af[c][i][t], acc[c][i][NT], 0, 0, 0);
    }
}

// The exact signed sums of a bit-plane block from its masked sums a (= 2^plane * sum q * bit; plane 7: -128 * ...)
// and the row sum o of the same activations: sum q * w = o - 2 * sum q * bit (bit 1 = weight -1). Exact: a is a
// multiple of 2^plane, and the shifts divide it exactly.
template <int P>
__device__ __forceinline__ void wsplit_planes_fix(int plane, const int (&o)[P], int (&a)[P][4]) {
    if (plane == 7) {  // wave-uniform: the plane's int8 value is -128, so the masked sum is -128 * sum q * bit
#pragma unroll
        for (int c = 0; c < P; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) a[c][r] = o[c] + 2 * (a[c][r] >> 7);
    } else {
#pragma unroll
        for (int c = 0; c < P; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) a[c][r] = o[c] - 2 * (a[c][r] >> plane);
    }
}

// Straight-line MFMAs over the wave's S k-steps: each weight word is expanded once (1 bit: v_and + v_perm per 4
// weights, two k-steps per word; 2 bits: one k-step per word) and feeds the RM row blocks x P parts of
// v_mfma_i32_16x16x64_i8 with the weights as the A operand.
template <int WBITS, int P, int RM, int NT, int S, int WPW>
__device__ __forceinline__ void wsplit_mfma(const uint32_t (&wv)[NT][WPW], const v4i (&af)[P][RM][S],
                                            v4i (&acc)[P][RM][NT]) {
    constexpr int KSW = WBITS == 1 ? 2 : 1;
#pragma unroll
    for (int c = 0; c < P; ++c)
#pragma unroll
        for (int i = 0; i < RM; ++i)
#pragma unroll
            for (int jn = 0; jn < NT; ++jn) acc[c][i][jn] = (v4i){0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < S; ++t) {
        const int u = t / KSW, h = t % KSW;
#pragma unroll
        for (int jn = 0; jn < NT; ++jn) {
            const uint32_t w32 = wv[jn][u];
            v4i bf;
            if constexpr (WBITS == 1) {
                if (h == 0) {
                    bf[0] = b1_expand<0>(w32); bf[1] = b1_expand<1>(w32); bf[2] = b1_expand<2>(w32); bf[3] = b1_expand<3>(w32);
                } else {
                    bf[0] = b1_expand<4>(w32); bf[1] = b1_expand<5>(w32); bf[2] = b1_expand<6>(w32); bf[3] = b1_expand<7>(w32);
                }
            } else {
                const uint32_t w4 = w32 >> 4;
                bf[0] = t2_lo(w32); bf[1] = t2_hi(w32); bf[2] = t2_lo(w4); bf[3] = t2_hi(w4);
            }
#pragma unroll
            for (int c = 0; c < P; ++c)
#pragma unroll
                for (int i = 0; i < RM; ++i)
                    acc[c][i][jn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf, af[c][i][t], acc[c][i][jn], 0, 0, 0);
        }
    }
}

// Writes the wave's partial tile to its LDS slice: the NT blocks [P][RM][NT][64 lanes][4] int32, then (bit-planes,
// ROWS) the row-sum block compacted to one int32 per lane, [P][RM][64] (its 4 components are equal: every row of the
// all-ones operand is the same); a barrier must follow.
template <int P, int RM, int NT, bool ROWS, int NA>
__device__ __forceinline__ void wsplit_share(int32_t *mine, int lane, const v4i (&acc)[P][RM][NA]) {
#pragma unroll
    for (int c = 0; c < P; ++c)
#pragma unroll
        for (int i = 0; i < RM; ++i) {
#pragma unroll
            for (int jn = 0; jn < NT; ++jn) *(v4i *)(mine + ((c * RM + i) * NT + jn) * 256 + lane * 4) = acc[c][i][jn];
            if constexpr (ROWS) mine[P * RM * NT * 256 + (c * RM + i) * 64 + lane] = acc[c][i][NT][0];
        }
}

// The exact sum over the NW wave partials (slices PART int32 apart) of block (i, jn) for this lane's 4 outputs, in
// wave order.
template <int P, int RM, int NT, int NW, int PART>
__device__ __forceinline__ void wsplit_block_sum(const int32_t *red, int i, int jn, int lane, int (&a)[P][4]) {
#pragma unroll
    for (int c = 0; c < P; ++c) {
        const int32_t *src = red + ((c * RM + i) * NT + jn) * 256 + lane * 4;
        v4i sum = *(const v4i *)src;
#pragma unroll
        for (int v = 1; v < NW; ++v) sum += *(const v4i *)(src + v * PART);
#pragma unroll
        for (int r = 0; r < 4; ++r) a[c][r] = sum[r];
    }
}

// The exact sum over the NW wave partials of the compacted row sums of row block i (bit-planes), in wave order.
template <int P, int RM, int NT, int NW, int PART>
__device__ __forceinline__ void wsplit_rows_sum(const int32_t *red, int i, int lane, int (&o)[P]) {
#pragma unroll
    for (int c = 0; c < P; ++c) {
        const int32_t *src = red + P * RM * NT * 256 + (c * RM + i) * 64 + lane;
        int sum = src[0];
#pragma unroll
        for (int v = 1; v < NW; ++v) sum += src[v * PART];
        o[c] = sum;
    }
}

// The epilogue of row m, columns nb .. nb + 3 of the block at (mt, nt) of an M x N output: for a whole block of a
// plain output (`plain`: no residual or raw accumulators; e.bias holds kNoBias without a bias) one vector store, from
// a copy specialised on the dtype and on the SiLU flag or the GLU pairs, so no SiLU or residual is evaluated only to
// be discarded; else the general epilogue.
template <int P>
__device__ __forceinline__ void wsplit_epilogue(const Params &p, bool plain, int M, int N, int m, int mt, int nt,
                                                int nb, const int (&a)[P][4], const EpiOperands &e) {
    if (plain && mt + 16 <= M && nt + 16 <= N) {
        const bool silu = (p.flags & KEA_FLAG_SILU) != 0;
        uint16_t *y16 = (uint16_t *)p.y + (long long)m * p.ldy;
        float *y32 = (float *)p.y + (long long)m * p.ldy;
        if (p.flags & KEA_FLAG_GLU) {  // the library refuses GLU with the SiLU
            if (p.y_dtype == KEA_F16) epilogue4_full<P, KEA_F16, false, false, 0, true>(p, y16, nb, a, e);
            else if (p.y_dtype == KEA_BF16) epilogue4_full<P, KEA_BF16, false, false, 0, true>(p, y16, nb, a, e);
            else epilogue4_full<P, KEA_F32, false, false, 0, true>(p, y32, nb, a, e);
        } else if (p.y_dtype == KEA_F16) {
            if (silu) epilogue4_full<P, KEA_F16, false, false, 1>(p, y16, nb, a, e);
            else epilogue4_full<P, KEA_F16, false, false, 0>(p, y16, nb, a, e);
        } else if (p.y_dtype == KEA_BF16) {
            if (silu) epilogue4_full<P, KEA_BF16, false, false, 1>(p, y16, nb, a, e);
            else epilogue4_full<P, KEA_BF16, false, false, 0>(p, y16, nb, a, e);
        } else {
            if (silu) epilogue4_full<P, KEA_F32, false, false, 1>(p, y32, nb, a, e);
            else epilogue4_full<P, KEA_F32, false, false, 0>(p, y32, nb, a, e);
        }
    } else {
        epilogue4<P>(p, m, nb, a, e);
    }
}

}  // namespace kea
