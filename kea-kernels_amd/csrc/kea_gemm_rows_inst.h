// Instances of the row-quantizing GEMM kernel for one activation part count (KEA_ROWS_P), included by
// kea_gemm_rows_p1.hip .. _p3.hip so the part counts compile in parallel.
//
// The wave-split GEMM (kea_gemm_wsplit_inst.h) with the activation quantizer in front of it in the same launch: a
// workgroup reads the FP32 rows of its 16-row tile over the whole of K, optionally puts them through one or two
// LayerNorms, quantizes them into P residual int8 parts and runs the MFMAs, reduction and epilogue of the wave-split
// kernel on them. The codes and scales are bitwise those of kea_quantize / kea_norm_quantize /
// kea_attention_merge_quantize on the same rows (f32 scales), so the output is bitwise that of the two-launch path.
//
// Every workgroup of a row tile quantizes the same rows again (the N / BN column tiles each read the FP32 rows):
// this trades L2 reads for a launch, which pays where launches dominate (small M).
//
// Layout: wave w of NW holds the k range [w S 64, (w + 1) S 64) of the tile's 16 rows. Rows are read coalesced, as
// the quantizer reads them: lane l holds the 4 consecutive floats at k = w S 64 + 256 c + 4 l (c < S / 4) of every
// row, so one load instruction covers 1 KiB of one row. For K = 1024 (4 waves of 4 k-steps) lane l of wave w holds
// exactly the elements of the quantizer's thread 64 w + l, so the LayerNorm sums are the quantizer's own: each lane's
// (((0 + a) + b) + c) + d, kea::wave_sum over the wave, then the wave totals in wave order. Row maxima are exact in
// any order. The int8 codes go to the MFMA operand layout (lane l: row l % 16, the 16 k at 64 t + 16 (l / 16) of step
// t) through a per-wave LDS staging area.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kea_gemm_rows.h"
#include "kea_gemm_wsplit_body.h"
#include "kea_merge.h"
#include "kea_rowq.h"
#include "kea_wave.h"

#ifndef KEA_ROWS_P
#error "define KEA_ROWS_P (1, 2 or 3) before including kea_gemm_rows_inst.h"
#endif

namespace {

using namespace kea;

// The row totals (sums, or maxima with MAX) of the 16 rows from this lane's values v[r]: kea::wave_sum / wave_max
// over the wave, then the NW wave totals of each row in wave order through LDS (slot[wave][row]; each reduction of a
// launch uses its own slot, so no barrier precedes a slot's first write). out[r] is the same in every lane.
template <int NW, bool MAX>
__device__ __forceinline__ void row_totals(const float (&v)[16], float (*slot)[16], int lane, int wave,
                                           float (&out)[16]) {
    float mine = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float t = MAX ? wave_max(v[r]) : wave_sum(v[r]);
        mine = lane == r ? t : mine;
    }
    if (lane < 16) slot[wave][lane] = mine;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        float a = slot[0][r];
#pragma unroll
        for (int w = 1; w < NW; ++w) a = MAX ? fmaxf(a, slot[w][r]) : a + slot[w][r];
        out[r] = a;
    }
}

// LayerNorm of the 16 rows (K = 1024: one 4-float chunk per lane and row) with the quantizer's arithmetic: mean,
// then the sum of squared deviations, inv = 1 / sqrt(var + eps), z = z * inv * w + b. lw / lb: the weights and
// biases at the lane's 4 k.
template <int NW>
__device__ __forceinline__ void layer_norm_rows(float (&z)[16][1][4], const float (&lw)[1][4], const float (&lb)[1][4],
                                                float eps, int K, float (*slot0)[16], float (*slot1)[16], int lane,
                                                int wave) {
    float part[16], tot[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) part[r] = (((0.f + z[r][0][0]) + z[r][0][1]) + z[r][0][2]) + z[r][0][3];
    row_totals<NW, false>(part, slot0, lane, wave, tot);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float mean = tot[r] / (float)K;
#pragma unroll
        for (int j = 0; j < 4; ++j) z[r][0][j] = z[r][0][j] - mean;
        part[r] = (((0.f + z[r][0][0] * z[r][0][0]) + z[r][0][1] * z[r][0][1]) + z[r][0][2] * z[r][0][2]) +
                  z[r][0][3] * z[r][0][3];
    }
    row_totals<NW, false>(part, slot1, lane, wave, tot);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float inv = 1.0f / sqrtf(tot[r] / (float)K + eps);
#pragma unroll
        for (int j = 0; j < 4; ++j) z[r][0][j] = z[r][0][j] * inv * lw[0][j] + lb[0][j];
    }
}

__device__ __forceinline__ void set4(float (&d)[4], const float4 v) {
    d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
}

// The kernel: grid (ceil(N / BN), ceil(M / 16)), NW wave64s, K = NW * S * 64 exactly (the host checks). x: the FP32
// rows [M][ldx], or for KEA_ROWS_MERGE the key-split attention workspace of M rows and p.heads heads (K = heads *
// 128). meta: bit 1 wscale is f16, bit 2 bias is f16. The operands of the first loads are preloaded scalar arguments.
// Dynamic LDS: the partial tiles [NW][P][NT][64][4] int32, then the code staging [NW][16][RS] bytes.
template <int MODE, int WBITS, int P, int NT, int NW, int S>
__global__ void __launch_bounds__(NW * 64) rows_kernel(const float *x, const uint32_t *w, const void *ws, int M,
                                                       int N, int K, int ldx, int meta, Params p) {
    static_assert(WBITS == 2 || S % 2 == 0, "1-bit waves take whole words (two k-steps each)");
    static_assert(S % 4 == 0, "a wave's k range is whole 256-float chunks per row");
    constexpr bool NORM = MODE == KEA_ROWS_NORM || MODE == KEA_ROWS_NORM2;
    static_assert(!NORM || (NW == 4 && S == 4), "LayerNorm rows follow the quantizer's order for K = 1024");
    constexpr int KSW = WBITS == 1 ? 2 : 1, WPW = S / KSW;
    constexpr int C = S / 4;                       // 4-float chunks per lane and row
    constexpr int RS = S * 64 + 16;                // staging bytes per row (16-byte pad: conflict-free reads)
    constexpr int BN = NT * 16, UB = (NT + NW - 1) / NW, PART = P * NT * 256;
    extern __shared__ __attribute__((aligned(16))) int32_t red[];
    __shared__ float stat[4 + P][NW][16];          // per-wave row statistics, one slot per reduction

    const void *const bias = p.bias;
    const int J = WBITS == 1 ? (K + 127) >> 7 : (K + 63) >> 6, NTILES = (N + 15) >> 4;
    const bool ws16 = (meta >> 1) & 1, b16 = (meta >> 2) & 1;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * 16;
    const int s0 = wave * S;
    const int kq = s0 * 64 + 4 * lane;             // the lane's first k; chunk c adds 256 c

    // ---- loads: weights, FP32 rows (and LayerNorm parameters), epilogue scales ----
    uint32_t wv[NT][WPW];
    wsplit_load_w<NT, WPW, false>(w, n0, NTILES, J, s0 / KSW, (uint32_t)lane * 16u, wv);
    float z[16][C][4];
    if constexpr (MODE == KEA_ROWS_MERGE) {
        const int heads = p.heads;
        const SplitWs sw = split_ws((void *)x, M, heads);
        const long long hd = (long long)heads * 128;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const long long row = min(m0 + r, M - 1);  // rows past M repeat row M - 1 and are never stored
#pragma unroll
            for (int c = 0; c < C; ++c) {
                const int k = kq + 256 * c, h = k >> 7;
                const float4 o0 = *(const float4 *)(sw.o + row * hd + k);
                const float4 o1 = *(const float4 *)(sw.o + (M + row) * hd + k);
                const float2 ml0 = *(const float2 *)(sw.ml + (row * heads + h) * 2);
                const float2 ml1 = *(const float2 *)(sw.ml + ((M + row) * heads + h) * 2);
                merge_halves(o0, o1, ml0, ml1, z[r][c]);
            }
        }
    } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float *src = x + (long long)min(m0 + r, M - 1) * ldx + kq;
#pragma unroll
            for (int c = 0; c < C; ++c) set4(z[r][c], *(const float4 *)(src + 256 * c));
        }
    }
    float lw[NORM ? C : 1][4], lb[NORM ? C : 1][4];
    if constexpr (NORM) {
        set4(lw[0], *(const float4 *)(p.nw0 + kq));
        set4(lb[0], *(const float4 *)(p.nb0 + kq));
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
            if (blockIdx.x == 0) {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (m0 + r < M)
                        *(float4 *)(p.x_out + (long long)(m0 + r) * p.ld_out + kq) =
                            make_float4(z[r][0][0], z[r][0][1], z[r][0][2], z[r][0][3]);
            }
            set4(lw[0], *(const float4 *)(p.nw1 + kq));
            set4(lb[0], *(const float4 *)(p.nb1 + kq));
            layer_norm_rows<NW>(z, lw, lb, p.eps1, K, stat[2], stat[3], lane, wave);
        }
    }
    // codes: packed in the load layout, staged through this wave's LDS rows, read back in the MFMA operand layout
    char *stage = (char *)(red + NW * PART) + wave * 16 * RS;
    v4i af[P][1][S];
    float sc[P];
#pragma unroll
    for (int c = 0; c < P; ++c) {
        float amax[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float a = 0.f;
#pragma unroll
            for (int cc = 0; cc < C; ++cc)
#pragma unroll
                for (int j = 0; j < 4; ++j) a = fmaxf(a, fabsf(z[r][cc][j]));
            amax[r] = a;
        }
        row_totals<NW, true>(amax, stat[4 + c], lane, wave, amax);
        float mine = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float s = fmaxf(amax[r] / 127.0f, 1.0e-30f), inv = 1.0f / s;
            mine = (lane & 15) == r ? s : mine;
#pragma unroll
            for (int cc = 0; cc < C; ++cc) {
                uint32_t packed = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) packed |= quantize_code(z[r][cc][j], s, inv) << (8 * j);
                *(uint32_t *)(stage + r * RS + 256 * cc + 4 * lane) = packed;
            }
        }
        sc[c] = mine;
        __builtin_amdgcn_wave_barrier();  // the wave's staging writes precede its reads (LDS runs a wave in order)
#pragma unroll
        for (int t = 0; t < S; ++t) af[c][0][t] = *(const v4i *)(stage + (lane & 15) * RS + 64 * t + 16 * (lane >> 4));
        __builtin_amdgcn_wave_barrier();  // ... and the next part's writes follow these reads
    }

    // ---- MFMAs, exact reduction over the waves, epilogue ----
    v4i acc[P][1][NT];
    wsplit_mfma<WBITS, P, 1, NT, S, WPW>(wv, af, acc);
    wsplit_share<P, 1, NT>(red + wave * PART, lane, acc);
    __syncthreads();
    const bool plain = p.y && !p.acc && !p.res && p.y_vec;
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
// halves are merged), the codes, weight words and accumulators, within 256 per wave (NW = 4) or 224 (NW = 8, two
// waves per SIMD).
template <int MODE, int WBITS, int NT, int NW, int S>
RowsFn pick_fit() {
    constexpr bool NORM = MODE == KEA_ROWS_NORM || MODE == KEA_ROWS_NORM2;
    constexpr int P = KEA_ROWS_P;
    constexpr int words = WBITS == 1 ? S / 2 : S;
    constexpr int load_phase = S * 16 * (MODE == KEA_ROWS_MERGE ? 2 : 1) + NT * words;
    constexpr int code_phase = S * 16 + P * S * 4 + NT * words + P * NT * 4;
    constexpr int regs = load_phase > code_phase ? load_phase : code_phase;
    constexpr int lds = NW * P * NT * 1024 + NW * 16 * (S * 64 + 16);
    if constexpr ((!NORM || (NW == 4 && S == 4)) && regs <= (NW == 4 ? 256 : 224) && lds <= 160 * 1024)
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
