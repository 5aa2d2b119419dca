// Instances of the row-quantizing GEMM kernel for one activation part count (KEA_ROWS_P), included by
// kea_gemm_rows_p1.hip .. _p3.hip so the part counts compile in parallel.
//
// The wave-split GEMM (kea_gemm_wsplit_inst.h) with the activation quantizer in front of it in the same launch: a
// workgroup reads the FP32 rows of its 16-row tile over the whole of K, optionally puts them through one or two
// LayerNorms, quantizes them into P residual int8 parts in registers and runs the MFMAs, reduction and epilogue of
// the wave-split kernel on them. The codes and scales are bitwise those of kea_quantize / kea_norm_quantize /
// kea_attention_merge_quantize on the same rows (f32 scales), so the output is bitwise that of the two-launch path.
//
// Every workgroup of a row tile quantizes the same rows again (the N / BN column tiles each read the FP32 rows):
// this trades L2 reads for a launch, which pays where launches dominate (small M).
//
// Layout: wave w of NW holds the S k-steps [w S, (w + 1) S) of every row of the tile; lane l holds row l % 16 and
// the 16 consecutive k at 64 t + 16 (l / 16) of step t, which is exactly the int8 operand layout of
// v_mfma_i32_16x16x64_i8 that the codes are packed into. Row statistics are reduced over the 4 lanes of a row with
// two lane exchanges and over the waves through LDS.
//
// LayerNorm sums (the only reductions that are not exact) follow the quantizer's fixed order, which for K = 1024
// (4 waves x 4 k-steps here) maps onto this layout: the quantizer's thread th of wave w holds k = 256 w + 4 (th % 64)
// + j, i.e. step t = (th % 64) / 16, lane group (th % 16) / 4 and 4-element chunk th % 4 of wave w here. Its xor
// butterfly over th (offsets 1 and 2: chunks inside a lane; 4 and 8: lane groups, lanes l ^ 16 and l ^ 32; 16 and 32:
// steps) and the wave totals in wave order are reproduced term by term.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kea_gemm_rows.h"
#include "kea_gemm_wsplit_body.h"
#include "kea_merge.h"
#include "kea_rowq.h"

#ifndef KEA_ROWS_P
#error "define KEA_ROWS_P (1, 2 or 3) before including kea_gemm_rows_inst.h"
#endif

namespace {

using namespace kea;

// The total over this wave's quarter of the row (K = 1024, S = 4) in the quantizer's butterfly order: per lane
// chunk sums (((0 + a) + b) + c) + d, the chunk pairs, the lane groups (l ^ 16, then l ^ 32), then the step pairs.
// SQUARE: the terms are the squares of the values.
template <bool SQUARE>
__device__ __forceinline__ float quarter_sum(const float (&z)[4][16]) {
    float u[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        float c4[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) s = s + (SQUARE ? z[t][4 * c + j] * z[t][4 * c + j] : z[t][4 * c + j]);
            c4[c] = s;
        }
        u[t] = (c4[0] + c4[1]) + (c4[2] + c4[3]);
        u[t] = u[t] + __shfl_xor(u[t], 16);
        u[t] = u[t] + __shfl_xor(u[t], 32);
    }
    return (u[0] + u[1]) + (u[2] + u[3]);
}

// The row total of per-wave values: slot[wave][row] written by lane group 0, one barrier, then the NW values of the
// lane's row summed (or maxed) in wave order. Each reduction of a launch uses its own slot (no barrier before reuse).
template <int NW, bool MAX>
__device__ __forceinline__ float across_waves(float v, float (*slot)[16], int lane, int wave) {
    if ((lane >> 4) == 0) slot[wave][lane & 15] = v;
    __syncthreads();
    float r = slot[0][lane & 15];
#pragma unroll
    for (int w = 1; w < NW; ++w) r = MAX ? fmaxf(r, slot[w][lane & 15]) : r + slot[w][lane & 15];
    return r;
}

// LayerNorm of the lane's values (K = 1024: S = 4, NW = 4) with the quantizer's arithmetic: mean, then the sum of
// squared deviations, inv = 1 / sqrt(var + eps), z = z * inv * w + b. lw / lb: the weights and biases at the lane's k.
template <int NW>
__device__ __forceinline__ void layer_norm_rows(float (&z)[4][16], const float (&lw)[4][16], const float (&lb)[4][16],
                                                float eps, int K, float (*slot0)[16], float (*slot1)[16], int lane,
                                                int wave) {
    const float mean = across_waves<NW, false>(quarter_sum<false>(z), slot0, lane, wave) / (float)K;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) z[t][e] = z[t][e] - mean;
    const float var = across_waves<NW, false>(quarter_sum<true>(z), slot1, lane, wave) / (float)K;
    const float inv = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) z[t][e] = z[t][e] * inv * lw[t][e] + lb[t][e];
}

// 16 consecutive floats at src (16-byte aligned) into v.
__device__ __forceinline__ void load16(const float *src, float (&v)[16]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 f = *(const float4 *)(src + 4 * q);
        v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
    }
}

// The kernel: grid (ceil(N / BN), ceil(M / 16)), NW wave64s, K = NW * S * 64 exactly (the host checks). x: the FP32
// rows [M][ldx], or for KEA_ROWS_MERGE the key-split attention workspace of M rows and p.heads heads (K = heads *
// 128). meta: bit 1 wscale is f16, bit 2 bias is f16. The operands of the first loads are preloaded scalar arguments.
template <int MODE, int WBITS, int P, int NT, int NW, int S>
__global__ void __launch_bounds__(NW * 64) rows_kernel(const float *x, const uint32_t *w, const void *ws, int M,
                                                       int N, int K, int ldx, int meta, Params p) {
    static_assert(WBITS == 2 || S % 2 == 0, "1-bit waves take whole words (two k-steps each)");
    constexpr bool NORM = MODE == KEA_ROWS_NORM || MODE == KEA_ROWS_NORM2;
    static_assert(!NORM || (NW == 4 && S == 4), "LayerNorm rows follow the quantizer's order for K = 1024");
    constexpr int KSW = WBITS == 1 ? 2 : 1, WPW = S / KSW;
    constexpr int BN = NT * 16, UB = (NT + NW - 1) / NW, PART = P * NT * 256;
    extern __shared__ __attribute__((aligned(16))) int32_t red[];  // [NW][P][NT][64 lanes][4]
    __shared__ float stat[4 + P][NW][16];                           // per-wave row statistics, one slot each

    const void *const bias = p.bias;
    const int J = WBITS == 1 ? (K + 127) >> 7 : (K + 63) >> 6, NTILES = (N + 15) >> 4;
    const bool ws16 = (meta >> 1) & 1, b16 = (meta >> 2) & 1;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * 16;
    const int s0 = wave * S;
    const int row = min(m0 + (lane & 15), M - 1);  // rows past M repeat row M - 1 and are never stored
    const int kl = s0 * 64 + (lane >> 4) * 16;     // the lane's first k; step t adds 64 t

    // ---- loads: weights, FP32 rows (and LayerNorm parameters), epilogue scales ----
    uint32_t wv[NT][WPW];
    wsplit_load_w<NT, WPW, false>(w, n0, NTILES, J, s0 / KSW, (uint32_t)lane * 16u, wv);
    float z[S][16];
    if constexpr (MODE == KEA_ROWS_MERGE) {
        const int heads = p.heads;
        const SplitWs sw = split_ws((void *)x, M, heads);
        const long long hd = (long long)heads * 128;
#pragma unroll
        for (int t = 0; t < S; ++t) {
            const int k = kl + 64 * t, h = k >> 7;  // 16 consecutive k lie in one head
            const float2 ml0 = *(const float2 *)(sw.ml + ((long long)row * heads + h) * 2);
            const float2 ml1 = *(const float2 *)(sw.ml + ((long long)(M + row) * heads + h) * 2);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 o0 = *(const float4 *)(sw.o + (long long)row * hd + k + 4 * q);
                const float4 o1 = *(const float4 *)(sw.o + (long long)(M + row) * hd + k + 4 * q);
                merge_halves(o0, o1, ml0, ml1, &z[t][4 * q]);
            }
        }
    } else {
        const float *src = x + (long long)row * ldx + kl;
#pragma unroll
        for (int t = 0; t < S; ++t) load16(src + 64 * t, z[t]);
    }
    float lw[NORM ? S : 1][16], lb[NORM ? S : 1][16];
    if constexpr (NORM) {
#pragma unroll
        for (int t = 0; t < S; ++t) {
            load16(p.nw0 + kl + 64 * t, lw[t]);
            load16(p.nb0 + kl + 64 * t, lb[t]);
        }
    }
    uint32_t ra[UB][4], rb[UB][4];
#pragma unroll
    for (int u = 0; u < UB; ++u) {
        const int jn = min(wave + NW * u, NT - 1);
        const int nb = n0 + jn * 16 + (lane >> 4) * 4;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            ra[u][r] = load_raw(ws, ws16, min(nb + r, N - 1));
            rb[u][r] = bias ? load_raw(bias, b16, min(nb + r, N - 1)) : 0u;
        }
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);

    // ---- the quantizer on the rows in registers ----
    if constexpr (NORM) {
        layer_norm_rows<NW>(z, lw, lb, p.eps0, K, stat[0], stat[1], lane, wave);
        if constexpr (MODE == KEA_ROWS_NORM2) {
            // LayerNorm0(x) is stored once per row, by the workgroups of the first column tile
            if (blockIdx.x == 0 && m0 + (lane & 15) < M) {
                float *dst = p.x_out + (long long)row * p.ld_out + kl;
#pragma unroll
                for (int t = 0; t < S; ++t)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        *(float4 *)(dst + 64 * t + 4 * q) =
                            make_float4(z[t][4 * q], z[t][4 * q + 1], z[t][4 * q + 2], z[t][4 * q + 3]);
            }
#pragma unroll
            for (int t = 0; t < S; ++t) {
                load16(p.nw1 + kl + 64 * t, lw[t]);
                load16(p.nb1 + kl + 64 * t, lb[t]);
            }
            layer_norm_rows<NW>(z, lw, lb, p.eps1, K, stat[2], stat[3], lane, wave);
        }
    }
    v4i af[P][1][S];
    float sc[P];
#pragma unroll
    for (int c = 0; c < P; ++c) {
        float amax = 0.f;
#pragma unroll
        for (int t = 0; t < S; ++t)
#pragma unroll
            for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(z[t][e]));
        amax = fmaxf(amax, __shfl_xor(amax, 16));
        amax = fmaxf(amax, __shfl_xor(amax, 32));
        amax = across_waves<NW, true>(amax, stat[4 + c], lane, wave);
        const float s = fmaxf(amax / 127.0f, 1.0e-30f), inv = 1.0f / s;
        sc[c] = s;
#pragma unroll
        for (int t = 0; t < S; ++t)
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                uint32_t packed = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) packed |= quantize_code(z[t][4 * d + j], s, inv) << (8 * j);
                af[c][0][t][d] = (int)packed;
            }
    }

    // ---- MFMAs, exact reduction over the waves, epilogue ----
    v4i acc[P][1][NT];
    wsplit_mfma<WBITS, P, 1, NT, S, WPW>(wv, af, acc);
    wsplit_share<P, 1, NT>(red + wave * PART, lane, acc);
    __syncthreads();
    const bool plain = p.y && !p.acc && !p.res && !(p.flags & KEA_FLAG_GLU) && p.y_vec;
#pragma unroll
    for (int u = 0; u < UB; ++u) {
        const int jn = wave + NW * u;
        if (jn >= NT) break;  // wave-uniform
        int a[P][4];
        wsplit_block_sum<P, 1, NT, NW>(red, 0, jn, lane, a);
        const int m = m0 + (lane & 15), nt = n0 + jn * 16, nb = nt + (lane >> 4) * 4;
        if (m >= M || nb >= N) continue;
        EpiOperands e;
#pragma unroll
        for (int c = 0; c < 3; ++c) e.s[c] = c < P ? sc[c] : 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int n = min(nb + r, N - 1);
            e.alpha[r] = raw_to_f32(ra[u][r], ws16, ws, (uint32_t)n);
            e.bias[r] = bias ? raw_to_f32(rb[u][r], b16, bias, (uint32_t)n) : kNoBias;
        }
        load_residual(p, m, nb, e.res);
        wsplit_epilogue<P>(p, plain, M, N, m, m0, nt, nb, a, e);
    }
}

// Instances exist only where the registers fit: the FP32 rows (16 per k-step; twice that while the two attention
// halves are merged), the LayerNorm parameters while they are live, the codes, weight words and accumulators, within
// 256 per wave (NW = 4) or 224 (NW = 8, two waves per SIMD).
template <int MODE, int WBITS, int NT, int NW, int S>
RowsFn pick_fit() {
    constexpr bool NORM = MODE == KEA_ROWS_NORM || MODE == KEA_ROWS_NORM2;
    constexpr int P = KEA_ROWS_P;
    constexpr int words = WBITS == 1 ? S / 2 : S;
    constexpr int load_phase = S * 16 * (NORM ? 3 : MODE == KEA_ROWS_MERGE ? 2 : 1) + NT * words;
    constexpr int code_phase = S * 16 + P * S * 4 + NT * words + P * NT * 4;
    constexpr int regs = load_phase > code_phase ? load_phase : code_phase;
    if constexpr ((!NORM || (NW == 4 && S == 4)) && regs <= (NW == 4 ? 256 : 224))
        return rows_kernel<MODE, WBITS, P, NT, NW, S>;
    else
        return nullptr;
}

template <int MODE, int WBITS>
RowsFn pick_tile(int tile, int s) {
    // the wave-split tiles with 16-row blocks (kea_gemm_wsplit.h): 0 16x128 k/4, 2 16x64 k/4, 3 16x128 k/8,
    // 5 16x32 k/4, 7 16x64 k/8
    switch (tile) {
        case 0: return s == 4 ? pick_fit<MODE, WBITS, 8, 4, 4>() : nullptr;
        case 2: return s == 4 ? pick_fit<MODE, WBITS, 4, 4, 4>() : nullptr;
        case 5: return s == 4 ? pick_fit<MODE, WBITS, 2, 4, 4>() : nullptr;
        case 3: return s == 8 ? pick_fit<MODE, WBITS, 8, 8, 8>() : nullptr;
        case 7: return s == 8 ? pick_fit<MODE, WBITS, 4, 8, 8>() : s == 4 ? pick_fit<MODE, WBITS, 4, 8, 4>() : nullptr;
        default: return nullptr;
    }
}

template <int WBITS>
RowsFn pick_mode(int mode, int tile, int s) {
    switch (mode) {
        case KEA_ROWS_PLAIN: return pick_tile<KEA_ROWS_PLAIN, WBITS>(tile, s);
        case KEA_ROWS_NORM: return pick_tile<KEA_ROWS_NORM, WBITS>(tile, s);
        case KEA_ROWS_NORM2: return pick_tile<KEA_ROWS_NORM2, WBITS>(tile, s);
        case KEA_ROWS_MERGE: return pick_tile<KEA_ROWS_MERGE, WBITS>(tile, s);
        default: return nullptr;
    }
}

}  // namespace

namespace kea {

#if KEA_ROWS_P == 1
RowsFn rows_pick_p1(int wbits, int mode, int tile, int s) {
#elif KEA_ROWS_P == 2
RowsFn rows_pick_p2(int wbits, int mode, int tile, int s) {
#else
RowsFn rows_pick_p3(int wbits, int mode, int tile, int s) {
#endif
    return wbits == 1 ? pick_mode<1>(mode, tile, s) : pick_mode<2>(mode, tile, s);
}

}  // namespace kea
