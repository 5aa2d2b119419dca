// Instances of the wave-split GEMM with per-group weight scales for one activation part count (KEA_WSPLIT_P),
// included by kea_gemm_wsplit_g1.hip .. _g3.hip so the part counts compile in parallel.
//
// Per-group weight scales (ws_group = 64 * GQ k, alpha [N][G]) change the epilogue into a fold over the groups in
// group order: r = 0; for g: r = fma(comb_P(acc_g), alpha[n][g], r); then r + bias, the optional SiLU and residual
// (the library's per-group rule, restated by the oracle's epilogue; the per-part combination is the reference's
// comb<P>, kk/binary/kernels_parts.py:28-39). The fold is one FP32 chain per output, so it cannot be split over waves;
// the int32 group sums can.
//
// One workgroup of NW wave64s owns a 16 x BN output tile (BN = 16 * NT) and the whole K range: NW * S k-steps of 64,
// S consecutive ones per wave, each wave's range made of whole groups (S % GQ == 0). Each wave loads every operand it
// needs at once (as the per-channel wave-split kernel), runs the MFMAs of one group at a time into fresh accumulators
// and writes each group's exact int32 block sums to that group's LDS slot. The tile's alpha block is staged into LDS
// as f32 [group][column] while the operand loads are in flight. After one barrier every block of the tile is folded
// by every thread of the workgroup, one to four consecutive outputs each: per group, their sums (one LDS vector read
// per part) and alpha (one more) give one fma per output, in group order; the sum of the group sums is the full-K
// accumulator for acc_out.
//
// The host runs these instances only when one workgroup covers K exactly with whole quads of weight words (K % 64 == 0,
// K = NW * S * 64, J % 4 == 0 when a wave reads more than one word): every load is an unmasked vector load. Other
// shapes take the LDS-ring kernel's per-group tiles.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "kea_gemm_wsplit.h"
#include "kea_gemm_wsplit_body.h"

#ifndef KEA_WSPLIT_P
#error "define KEA_WSPLIT_P (1, 2 or 3) before including kea_gemm_wsplit_group_inst.h"
#endif

namespace {

using namespace kea;

// The MFMAs of the wave's S k-steps, one group of GQ k-steps at a time: each group's int32 sums of the NT blocks and P
// parts go to that group's slot ([P][NT][64 lanes][4] int32) at `slots` + group * SLOT.
template <int WBITS, int P, int NT, int S, int WPW, int GQ>
__device__ __forceinline__ void group_mfma(const uint32_t (&wv)[NT][WPW], const v4i (&af)[P][1][S], int32_t *slots,
                                           int lane) {
    constexpr int KSW = WBITS == 1 ? 2 : 1;
    constexpr int SLOT = P * NT * 256;
#pragma unroll
    for (int gl = 0; gl < S / GQ; ++gl) {
        v4i acc[P][NT];
#pragma unroll
        for (int c = 0; c < P; ++c)
#pragma unroll
            for (int jn = 0; jn < NT; ++jn) acc[c][jn] = (v4i){0, 0, 0, 0};
#pragma unroll
        for (int tt = 0; tt < GQ; ++tt) {
            const int t = gl * GQ + tt, u = t / KSW, h = t % KSW;
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
                    acc[c][jn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf, af[c][0][t], acc[c][jn], 0, 0, 0);
            }
        }
        int32_t *slot = slots + gl * SLOT;
#pragma unroll
        for (int c = 0; c < P; ++c)
#pragma unroll
            for (int jn = 0; jn < NT; ++jn) *(v4i *)(slot + (c * NT + jn) * 256 + lane * 4) = acc[c][jn];
    }
}

template <int WBITS, int P, int NT, int NW, int S, int GQ>
__global__ void __launch_bounds__(NW * 64) wsplit_group_kernel(const int8_t *q, const uint32_t *w, const void *qs,
                                                               const void *ws, int M, int N, int K, int ldq, int meta,
                                                               int part_stride, Params p) {
    static_assert(WBITS == 2 || S % 2 == 0, "1-bit waves take whole words (two k-steps each)");
    static_assert(S % GQ == 0, "a wave's K range is whole groups");
    constexpr int KSW = WBITS == 1 ? 2 : 1;
    constexpr int WPW = S / KSW;
    constexpr int BN = NT * 16;
    constexpr int GW = S / GQ;                 // groups per wave
    constexpr int GWG = NW * GW;               // groups per workgroup (all of K)
    constexpr int SLOT = P * NT * 256;         // int32 of one group's sums
    constexpr int APAD = BN + 4;               // f32 per staged alpha row (16-byte rows, rotated banks)
    extern __shared__ __attribute__((aligned(16))) int32_t lds[];  // [GWG][SLOT] int32 [, alpha f32 [GWG][APAD]]
    float *alpha = (float *)(lds + GWG * SLOT);

    const void *const bias = p.bias;
    const long long qs_stride = p.qs_stride;
    const int J = WBITS == 1 ? (K + 127) >> 7 : (K + 63) >> 6, NTILES = (N + 15) >> 4;
    const bool qs16 = meta & 1, ws16 = (meta >> 1) & 1, b16 = (meta >> 2) & 1;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * 16;
    const int s0 = wave * S;

    // ---- loads: weights, activations, all issued before the first wait ----
    const uint32_t lane16 = (uint32_t)lane * 16u;
    uint32_t wv[NT][WPW];
    wsplit_load_w<NT, WPW, false>(w, n0, NTILES, J, s0 / KSW, lane16, wv);
    v4i af[P][1][S];
    {
        const int kl = (lane >> 4) * 16;
        const int m = min(m0 + (lane & 15), M - 1);
        const uint32_t row = (uint32_t)m * (uint32_t)ldq;
#pragma unroll
        for (int c = 0; c < P; ++c) {
            const int8_t *part = q + (long long)c * part_stride;
#pragma unroll
            for (int t = 0; t < S; ++t)
                af[c][0][t] = *(const v4i *)(part + (long long)s0 * 64 + t * 64 + (row + (uint32_t)kl));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // The fold is spread over every thread of the workgroup: thread t finishes the OPT consecutive outputs
    // o = t * OPT + j (OPT = 1, 2 or 4) of the tile's 16 x BN, numbered in the LDS order of the group sums (block,
    // lane, component): its group sums are one 4-, 8- or 16-byte LDS read per part and group, and the reads of a wave
    // are contiguous. Output o is row (o % 256) / 4 % 16 of the tile, column 16 * (o / 256) + 4 * ((o % 256) / 64) +
    // o % 4; the OPT outputs of a thread share the row and lie in consecutive columns. Their row scales, bias and
    // residual values are loaded now.
    constexpr int OUTS = 16 * BN;
    constexpr int OPT = wsplit_group_opt(NT, NW);
    static_assert(OUTS <= NW * 64 * OPT, "every output has a thread");
    const int o0 = (int)threadIdx.x * OPT;
    const bool fold = o0 < OUTS;  // threads past the tile's outputs only help with the MFMAs
    const int oo = fold ? o0 : 0, ol = (oo & 255) >> 2;
    const int orow = ol & 15, ocol = 16 * (oo >> 8) + 4 * (ol >> 4) + (oo & 3);
    uint32_t rs[3], rb[OPT];
    float rr[OPT];
    {
        const int m = min(m0 + orow, M - 1);
#pragma unroll
        for (int c = 0; c < 3; ++c) rs[c] = c < P ? load_raw(qs, qs16, (uint32_t)(c * qs_stride + m)) : 0u;
#pragma unroll
        for (int j = 0; j < OPT; ++j) {
            const int n = min(n0 + ocol + j, N - 1);
            rb[j] = bias ? load_raw(bias, b16, (uint32_t)n) : 0u;
            rr[j] = p.res ? p.res[(long long)m * p.ldr + n] : 0.f;
        }
    }
    // alpha: with few values per thread (AREG) each thread's own column's G values as raw words in registers (f16: two
    // groups a word). Meta bit 3 (rows 16-byte aligned, whole 16-byte units): the tile's block of alpha, BN rows of
    // [N][G] and so one contiguous range, is loaded once with one 16-byte load per thread of the first BN * G * esz / 16
    // (units past row N - 1 clamped to the last unit in the array: their columns are never stored), staged in LDS
    // through the barrier, and each thread then reads its column's row from LDS (16 threads share a column: one global
    // load of each byte instead of sixteen). Otherwise each thread loads its row element by element. Without AREG the
    // tile's block [GWG groups][BN columns], clamped into [N][G] (the clamped values are never stored), is staged in
    // LDS as f32, consecutive threads taking consecutive groups of one column.
    const int G = p.groups;  // == GWG (checked by the host)
    constexpr bool AREG = wsplit_group_alpha_regs(P, NT, NW, S, GQ);
    static_assert(!AREG || OPT == 1, "register-held alpha serves one output a thread");
    constexpr int AW = AREG ? GWG : 1;
    uint32_t araw[OPT][AW];
    constexpr int AL = AREG ? 1 : (GWG * BN + NW * 64 - 1) / (NW * 64);
    float av[AL];
    static_assert(!AREG || BN * GWG * 4 <= NW * 64 * 16, "one 16-byte unit of the alpha block per thread at most");
    const bool avec = (meta >> 3) & 1;
    const int arow = GWG * (ws16 ? 2 : 4);  // bytes of one alpha row
    uint4 ast = make_uint4(0u, 0u, 0u, 0u);
    if constexpr (AREG) {
        if (avec) {
            if ((int)threadIdx.x * 16 < BN * arow)
                ast = *(const uint4 *)((const char *)ws + (long long)n0 * arow +
                                       min((int)threadIdx.x * 16, (N - n0) * arow - 16));
        } else {
            const int n = min(n0 + ocol, N - 1);
            if (ws16) {
                const uint16_t *row = (const uint16_t *)ws + (long long)n * G;
#pragma unroll
                for (int g = 0; g < GWG; g += 2)
                    araw[0][g / 2] = (uint32_t)row[g] | ((uint32_t)row[min(g + 1, GWG - 1)] << 16);
            } else {
                const uint32_t *row = (const uint32_t *)ws + (long long)n * G;
#pragma unroll
                for (int g = 0; g < GWG; ++g) araw[0][g] = row[g];
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < AL; ++i) {
            const int idx = (int)threadIdx.x + i * NW * 64;
            const int col = idx / GWG, g = idx - (idx / GWG) * GWG;
            const int n = min(n0 + col, N - 1), gg = min(g, G - 1);
            av[i] = (idx < GWG * BN) ? load_scalar(ws, ws16 ? KEA_F16 : KEA_F32, (long long)n * G + gg) : 0.f;
        }
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);

    // ---- MFMAs, one group at a time, each group's sums to its LDS slot ----
    group_mfma<WBITS, P, NT, S, WPW, GQ>(wv, af, lds + wave * GW * SLOT, lane);
    uint8_t *astage = (uint8_t *)(lds + GWG * SLOT);  // AREG: the staged alpha block, raw [BN][G] bytes
    if constexpr (AREG) {
        if (avec && (int)threadIdx.x * 16 < BN * arow) *(uint4 *)(astage + threadIdx.x * 16) = ast;
    }
    if constexpr (!AREG) {
#pragma unroll
        for (int i = 0; i < AL; ++i) {
            const int idx = (int)threadIdx.x + i * NW * 64;
            const int col = idx / GWG, g = idx - (idx / GWG) * GWG;
            if (idx < GWG * BN) alpha[g * APAD + col] = av[i];
        }
    }
    __syncthreads();
    if constexpr (AREG) {
        if (avec) {
            // one loop per dtype, so every register index is a compile-time constant
            const uint4 *src = (const uint4 *)(astage + ocol * arow);
            if (ws16) {
#pragma unroll
                for (int i = 0; i < GWG / 8; ++i) {
                    const uint4 v = src[i];
                    araw[0][4 * i] = v.x; araw[0][4 * i + 1] = v.y; araw[0][4 * i + 2] = v.z; araw[0][4 * i + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < GWG / 4; ++i) {
                    const uint4 v = src[i];
                    araw[0][4 * i] = v.x; araw[0][4 * i + 1] = v.y; araw[0][4 * i + 2] = v.z; araw[0][4 * i + 3] = v.w;
                }
            }
        }
    }

    // ---- fold: every group of K in order (the host runs these instances with G == GWG: all of K is this
    // workgroup's), one FP32 chain per output ----
    float sc[3];
#pragma unroll
    for (int c = 0; c < 3; ++c)
        sc[c] = c < P ? raw_to_f32(rs[c], qs16, qs, (uint32_t)(c * qs_stride + min(m0 + orow, M - 1))) : 0.f;
    float racc[OPT];
    int at[P][OPT];
#pragma unroll
    for (int j = 0; j < OPT; ++j) {
        racc[j] = 0.f;
#pragma unroll
        for (int c = 0; c < P; ++c) at[c][j] = 0;
    }
    using IV = int __attribute__((ext_vector_type(OPT)));
    using FV = float __attribute__((ext_vector_type(OPT)));
    // the fold, in copies specialised on acc_out (the full-K sums only when they are wanted: no dead adds in the chains)
    // and on the dtype of register-held alpha (every register index a compile-time constant, no per-group branch).
    // f16 alpha enters each fma as its f16 half: the conversion is exact and the compiler folds it into the fma
    // (v_fma_mix_f32), so no separate conversion is spent on it. The group sums are read from LDS in chunks of CH groups
    // (at most 64 registers), every read of a chunk issued before the first use, so the LDS latency is paid once per
    // chunk rather than once per group.
    constexpr int CH = (64 / (P * OPT)) < GWG ? (64 / (P * OPT) > 0 ? 64 / (P * OPT) : 1) : GWG;
    auto fold_groups = [&](auto with_acc, auto f16_tag) {
        constexpr bool F16A = decltype(f16_tag)::value;
#pragma unroll
        for (int g0 = 0; g0 < GWG; g0 += CH) {
            IV a[CH][P];
#pragma unroll
            for (int i = 0; i < CH; ++i)
#pragma unroll
                for (int c = 0; c < P; ++c)
                    if (g0 + i < GWG) a[i][c] = *(const IV *)(lds + (g0 + i) * SLOT + c * OUTS + oo);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < CH; ++i) {
                const int g = g0 + i;
                if (g >= GWG) break;
                FV al;
                if constexpr (AREG && F16A)
                    al[0] = (float)__builtin_bit_cast(_Float16, (uint16_t)(araw[0][g / 2] >> (16 * (g & 1))));
                else if constexpr (AREG)
                    al[0] = __builtin_bit_cast(float, araw[0][g]);
                else
                    al = *(const FV *)(alpha + g * APAD + ocol);
#pragma unroll
                for (int j = 0; j < OPT; ++j) {
                    int ar[3] = {a[i][0][j], P > 1 ? a[i][1 % P][j] : 0, P > 2 ? a[i][2 % P][j] : 0};
                    racc[j] = __builtin_fmaf(combine<P>(ar, sc, p.flags), al[j], racc[j]);
                    if constexpr (decltype(with_acc)::value) {
#pragma unroll
                        for (int c = 0; c < P; ++c) at[c][j] += a[i][c][j];
                    }
                }
            }
        }
    };
    if (AREG && ws16) {
        if (p.acc) fold_groups(std::true_type{}, std::true_type{});
        else fold_groups(std::false_type{}, std::true_type{});
    } else {
        if (p.acc) fold_groups(std::true_type{}, std::false_type{});
        else fold_groups(std::false_type{}, std::false_type{});
    }
    // ---- epilogue of each output: r + bias, SiLU, residual, store; acc_out = the sum of the group sums ----
    const int m = m0 + orow;
    if (!fold || m >= M) return;
#pragma unroll
    for (int j = 0; j < OPT; ++j) {
        const int n = n0 + ocol + j;
        if (n >= N) break;
        if (p.y) {
            float x = racc[j];
            if (bias) x = x + raw_to_f32(rb[j], b16, bias, (uint32_t)n);
            if (p.flags & KEA_FLAG_SILU) x = kea::silu_epilogue(x);
            if (p.res) x = rr[j] + x * p.res_factor;
            const long long off = (long long)m * p.ldy + n;
            if (p.y_dtype == KEA_F32) ((float *)p.y)[off] = x;
            else ((uint16_t *)p.y)[off] = p.y_dtype == KEA_F16 ? to_f16_bits(x) : to_bf16_bits(x);
        }
        if (p.acc) {
#pragma unroll
            for (int c = 0; c < P; ++c) p.acc[((long long)c * M + m) * p.acc_ld + n] = at[c][j];
        }
    }
}

// Instances exist for register and LDS budgets that fit (kea::wsplit_group_fits, checked by the host first).
template <int WBITS, int P, int NT, int NW, int S, int GQ>
WsplitFn group_fit() {
    constexpr int words = WBITS == 1 ? S / 2 : S;
    constexpr int regs = P * S * 4 + NT * words + P * NT * 4;
    constexpr int lds = wsplit_group_lds(P, NT, NW, S, GQ);
    if constexpr (S % GQ == 0 && (WBITS == 2 || S % 2 == 0) && regs <= wsplit_reg_budget(NW) && lds <= 160 * 1024)
        return wsplit_group_kernel<WBITS, P, NT, NW, S, GQ>;
    else
        return nullptr;
}

template <int WBITS, int P, int NT, int NW, int GQ>
WsplitFn group_pick_s(int s) {
    switch (s) {
        case 2: return group_fit<WBITS, P, NT, NW, 2, GQ>();
        case 4: return group_fit<WBITS, P, NT, NW, 4, GQ>();
        case 8: return group_fit<WBITS, P, NT, NW, 8, GQ>();
        case 16: return group_fit<WBITS, P, NT, NW, 16, GQ>();
        default: return nullptr;
    }
}

template <int WBITS, int P, int NT, int NW>
WsplitFn group_pick_gq(int gq, int s) {
    switch (gq) {
        case 1: return group_pick_s<WBITS, P, NT, NW, 1>(s);
        case 2: return group_pick_s<WBITS, P, NT, NW, 2>(s);
        case 4: return group_pick_s<WBITS, P, NT, NW, 4>(s);
        default: return nullptr;
    }
}

// The instance for kWsplitTiles[tile] if it is a 16-row tile of at most four n-tiles (nullptr otherwise).
template <int WBITS, int P, int T = 0>
WsplitFn group_pick_tile(int tile, int gq, int s) {
    if constexpr (T < kNumWsplitTiles) {
        constexpr WsplitTile t = kWsplitTiles[T];
        if (tile == T) {
            if constexpr (t.rm == 1 && t.nt <= 4) return group_pick_gq<WBITS, P, t.nt, t.nw>(gq, s);
            else return nullptr;
        }
        return group_pick_tile<WBITS, P, T + 1>(tile, gq, s);
    } else {
        return nullptr;
    }
}

}  // namespace

namespace kea {

#if KEA_WSPLIT_P == 1
WsplitFn wsplit_group_pick_p1(int wbits, int tile, int gq, int s) {
#elif KEA_WSPLIT_P == 2
WsplitFn wsplit_group_pick_p2(int wbits, int tile, int gq, int s) {
#else
WsplitFn wsplit_group_pick_p3(int wbits, int tile, int gq, int s) {
#endif
    return wbits == 1 ? group_pick_tile<1, KEA_WSPLIT_P>(tile, gq, s) : group_pick_tile<2, KEA_WSPLIT_P>(tile, gq, s);
}

}  // namespace kea
