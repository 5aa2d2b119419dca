// Instances of the wave-split GEMM kernel for one activation part count (KEA_WSPLIT_P), included by
// kea_gemm_wsplit_p1.hip .. _p3.hip so the part counts compile in parallel.
//
// Wave-split low-bit GEMM for small M on MI355X (gfx950): the same contract and epilogue as the LDS-ring kernel of
// kea_gemm.hip (kk/binary/kernels.py:134-565, kk/ternary/fused_kernels.py:53-120), organised for launches whose time
// is set by memory latency rather than by matrix-core throughput.
//
// One workgroup owns a BM x BN output tile (BM = 16 * RM rows, BN = 16 * NT columns) and a range of NW * S k-steps of
// 64; wave w of its NW waves takes the S consecutive k-steps [w * S, (w + 1) * S) of that range. Each wave:
//   * issues every load it needs at once, before any wait: its activation fragments (one 16-byte load per lane per
//     k-step, the MFMA operand layout of 16 rows x 64 k), its weights and the epilogue's scales (raw words whose
//     conversion waits until the epilogue: a lane's 4 per-channel scales, and bias values, with one range-checked
//     16-byte buffer load each). Weights are native words (one 32-bit word per lane per n-tile and
//     word: 2 k-steps at 1 bit, 1 at 2 bits; four consecutive words with one 128-bit load) or, for the 1-bit
//     instances that kea::wsplit_planes selects, the bit-plane part of the layout (one 16-byte unit per lane per
//     k-step holds the k-step's weights of all 8 n-tiles of a 128-row group);
//   * feeds the RM row blocks x P parts of v_mfma_i32_16x16x64_i8, with the weights as the A operand (a lane ends
//     with 4 consecutive columns of a row). Words are expanded once (1 bit: v_and_b32 + v_perm_b32 per 4 weights;
//     2 bits: two v_perm_b32 per 8); bit-planes: n-tile j's operand is the unit masked with 0x01010101 << plane (one
//     v_and_b32 per 4 weights; int8 values 0 / 2^plane), plus one MFMA per k-step on an all-ones operand for the
//     activation row sums;
//   * writes its int32 partial tile to LDS. After one barrier the tile's 16x16 blocks are shared out over the waves,
//     each block summed over the NW partials in wave order (integer addition: exact) and finished by the epilogue
//     (bit-planes: the signed sums first, row sum - 2 * masked sum / 2^plane, exact).
// Activations at k >= the end of the K range are zeroed at load, so the (valid, never garbage) weight words there
// contribute nothing; rows past M are clamped to row M - 1 and columns past N to the last n-tile, and neither is
// stored. SLICED: blockIdx.z is a K slice of steps_per_slice k-steps whose exact int32 sums go to the slices
// [S][P][M][N] instead of the epilogue (the finish kernel adds them in slice order).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "kea_gemm_wsplit.h"
#include "kea_gemm_wsplit_body.h"

#ifndef KEA_WSPLIT_P
#error "define KEA_WSPLIT_P (1, 2 or 3) before including kea_gemm_wsplit_inst.h"
#endif

namespace {

using namespace kea;

// RAGGED = false: the host guarantees that every wave's K range is whole (K % 64 == 0, the workgroup's range a
// multiple of NW * S k-steps) and that its weight words lie in complete quads (J % 4 == 0 or one word per wave), so
// every load is an unmasked vector load. RAGGED = true: loads from clamped addresses, masked to zero at k >= kend
// (per byte, so K % 16 != 0 is covered).
// The operands the loads need come first, as scalar arguments, so the dispatch can preload them into SGPRs
// (-amdgpu-kernarg-preload-count): no kernel-argument round trip stands before the first load. meta: bit 0 qs is
// f16, bit 1 wscale is f16, bit 2 bias is f16. The rest (epilogue, slices) is read from `p`.
template <int WBITS, int P, int RM, int NT, int NW, int S, bool SLICED, bool RAGGED>
__global__ void __launch_bounds__(NW * 64) wsplit_kernel(const int8_t *q, const uint32_t *w, const void *qs,
                                                         const void *ws, int M, int N, int K, int ldq, int meta,
                                                         int part_stride, Params p) {
    constexpr bool PL = wsplit_planes(WBITS, P, RM, NT);  // 1-bit weights from the bit-plane part
    static_assert(!PL || 128 % (NT * 16) == 0, "bit-plane tiles lie inside one 128-row group");
    static_assert(WBITS == 2 || PL || S % 2 == 0, "1-bit waves take whole words (two k-steps each)");
    constexpr int KSW = WBITS == 1 && !PL ? 2 : 1; // k-steps per native word
    constexpr int WPW = S / KSW;                  // words per lane per n-tile for one wave
    constexpr int BM = RM * 16, BN = NT * 16;
    constexpr int NB = RM * NT;                   // 16x16 blocks of the tile
    constexpr int NBK = wsplit_blocks(PL, NT);    // accumulator blocks per part and row block (bit-planes: + row sums)
    constexpr int UB = (NB + NW - 1) / NW;        // blocks one wave finishes
    constexpr int PART = wsplit_part(PL, P, RM, NT);  // int32 of one wave's partial tile in LDS
    extern __shared__ __attribute__((aligned(16))) int32_t red[];  // [NW][PART]: blocks, then compacted row sums

    const void *const bias = p.bias;
    const long long qs_stride = p.qs_stride;
    const int J = WBITS == 1 ? (K + 127) >> 7 : (K + 63) >> 6, NTILES = (N + 15) >> 4;
    const int sps = SLICED ? p.steps_per_slice : 0;
    const bool qs16 = meta & 1, ws16 = (meta >> 1) & 1, b16 = (meta >> 2) & 1;

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int ksteps = (K + 63) >> 6;
    const int sa = SLICED ? (int)blockIdx.z * sps : 0;
    const int sb = SLICED ? min(ksteps, sa + sps) : ksteps;
    const int s0 = sa + wave * S;                 // this wave's first k-step
    const int kend = min(K, sb * 64);

    // ---- loads: weights, activations, epilogue scales, all issued before the first wait ----
    const uint32_t lane16 = (uint32_t)lane * 16u;  // < 1024
    // bit-planes: the units of the tile's group (w points at the layout's bit-plane part); otherwise words
    uint4 wu[PL ? S : 1];
    uint32_t wv[PL ? 1 : NT][PL ? 1 : WPW];
    if constexpr (PL) wsplit_load_planes<S, RAGGED>(w, n0, ksteps, s0, lane, wu);
    else wsplit_load_w<NT, WPW, RAGGED>(w, n0, NTILES, J, s0 / KSW, lane16, wv);
    v4i af[P][RM][S];
    {
        const int kl = (lane >> 4) * 16;          // this lane's 16 bytes of each k-step
#pragma unroll
        for (int c = 0; c < P; ++c)
#pragma unroll
            for (int i = 0; i < RM; ++i) {
                // wave-uniform base plus a 32-bit per-lane offset (q spans less than 2 GiB)
                const int m = min(m0 + i * 16 + (lane & 15), M - 1);
                const int8_t *part = q + (long long)c * part_stride;
                const uint32_t row = (uint32_t)m * (uint32_t)ldq;
#pragma unroll
                for (int t = 0; t < S; ++t) {
                    const int k = (s0 + t) * 64 + kl;
                    if constexpr (!RAGGED) {
                        af[c][i][t] = *(const v4i *)(part + (long long)s0 * 64 + t * 64 + (row + (uint32_t)kl));
                    } else {
                        // k < kend <= K <= ldq with ldq % 16 == 0: the 16 bytes lie in the row; else load the row start
                        v4i v = *(const v4i *)(part + (row + (uint32_t)(k < kend ? k : 0)));
#pragma unroll
                        for (int d = 0; d < 4; ++d) {
                            const int valid = kend - (k + 4 * d);  // bytes at k >= kend must not contribute
                            const uint32_t keep =
                                valid >= 4 ? 0xFFFFFFFFu : (valid <= 0 ? 0u : (1u << (8 * valid)) - 1u);
                            v[d] = (int)((uint32_t)v[d] & keep);
                        }
                        af[c][i][t] = v;
                    }
                }
            }
    }
    // the operand loads go out before anything that needs a kernel argument outside the preloaded ones
    __builtin_amdgcn_sched_barrier(0);
    // epilogue scales of the blocks this wave finishes: raw words now, converted in the epilogue; and their residual
    // values, which would otherwise be a memory round trip after the reduction (the residual may be y itself: each
    // element is read here and written later by this same lane, so in-place updates stay exact)
    uint32_t rs[UB][3];
    v4u ra[UB], rb[UB];
    float rr[UB][4];
    const ColVec wsv = col_vec(ws, ws16, N), bv = col_vec(bias, b16, N);
    if constexpr (!SLICED) {
#pragma unroll
        for (int u = 0; u < UB; ++u) {
            const int b = min(wave + NW * u, NB - 1);
            const int i = b / NT, jn = b - (b / NT) * NT;
            const int m = min(m0 + i * 16 + (lane & 15), M - 1);
#pragma unroll
            for (int c = 0; c < 3; ++c) rs[u][c] = c < P ? load_raw(qs, qs16, (uint32_t)(c * qs_stride + m)) : 0u;
            // a block's 4 scales (and bias values) with one range-checked 16-byte load
            const int nb = n0 + jn * 16 + (lane >> 4) * 4;
            ra[u] = col_load4(wsv, ws16, nb);
            rb[u] = bias ? col_load4(bv, b16, nb) : (v4u){0u, 0u, 0u, 0u};
            if (p.res) load_residual(p, m, nb, rr[u]);
        }
    }
    // Every load above is issued before the first instruction that waits. The memory clobber keeps the compiler from
    // sinking the scale loads to their use in the epilogue, where their latency would stand alone.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    // The epilogue's kernel arguments are pinned into scalar registers now, while the operand loads are in flight:
    // read where they are used, each would be a kernel-argument round trip on the epilogue's critical path.
    if constexpr (!SLICED)
        asm volatile("" ::"s"(p.M), "s"(p.N), "s"(p.res), "s"(p.ldr), "s"(p.res_factor), "s"(p.y), "s"(p.ldy),
                     "s"(p.flags), "s"(p.y_dtype), "s"(p.y_vec), "s"(p.acc));

    // ---- MFMAs: straight-line code over the wave's S k-steps ----
    v4i acc[P][RM][NBK];
    if constexpr (PL) wsplit_mfma_planes<P, RM, NT, S>(wu, af, (n0 >> 4) & 7, acc);
    else wsplit_mfma<WBITS, P, RM, NT, S, WPW>(wv, af, acc);

    // ---- exact reduction over the waves through LDS ----
    wsplit_share<P, RM, NT, PL>(red + wave * PART, lane, acc);
    __syncthreads();

    // ---- epilogue: block b = wave + NW * u of the tile ----
    const bool plain = !SLICED && p.y && !p.acc && !p.res && p.y_vec;
#pragma unroll
    for (int u = 0; u < UB; ++u) {
        const int b = wave + NW * u;
        if (b >= NB) break;  // wave-uniform
        const int i = b / NT, jn = b - (b / NT) * NT;
        int a[P][4];
        wsplit_block_sum<P, RM, NT, NW, PART>(red, i, jn, lane, a);
        if constexpr (PL) {  // the signed sums from the masked sums and the activation row sums
            int o[P];
            wsplit_rows_sum<P, RM, NT, NW, PART>(red, i, lane, o);
            wsplit_planes_fix<P>(((n0 >> 4) + jn) & 7, o, a);
        }
        const int mt = m0 + i * 16, m = mt + (lane & 15);
        const int nt = n0 + jn * 16, nb = nt + (lane >> 4) * 4;
        if (m >= M || nb >= N) continue;
        if constexpr (SLICED) {
#pragma unroll
            for (int c = 0; c < P; ++c)
                store_int4(p.slices + (((long long)blockIdx.z * P + c) * M + m) * N + nb, p.slice_vec, nb, N, a[c]);
        } else {
            EpiOperands e;
#pragma unroll
            for (int c = 0; c < 3; ++c)
                e.s[c] = c < P ? raw_to_f32(rs[u][c], qs16, qs, (uint32_t)(c * qs_stride + m)) : 0.f;
            col_to_f32(ra[u], ws16, wsv.delta, e.alpha);
            if (bias) {
                col_to_f32(rb[u], b16, bv.delta, e.bias);
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) e.bias[r] = kNoBias;
            }
            if (p.res) {
#pragma unroll
                for (int r = 0; r < 4; ++r) e.res[r] = rr[u][r];
            }
            wsplit_epilogue<P>(p, plain, M, N, m, mt, nt, nb, a, e);
        }
    }
}

// Instances exist only for register budgets that fit (kea::wsplit_fits, checked by the host before any launch).
template <int WBITS, int P, int RM, int NT, int NW, int S, bool SLICED, bool RAGGED>
WsplitFn pick_fit() {
    if constexpr (wsplit_regs(WBITS, P, RM, NT, S) <= wsplit_reg_budget(NW) &&
                  wsplit_lds(WBITS, P, RM, NT, NW) <= 160 * 1024)
        return wsplit_kernel<WBITS, P, RM, NT, NW, S, SLICED, RAGGED>;
    else
        return nullptr;
}

template <int WBITS, int P, int RM, int NT, int NW, bool SLICED, bool RAGGED>
WsplitFn pick_s(int s) {
    switch (s) {
        case 2: return pick_fit<WBITS, P, RM, NT, NW, 2, SLICED, RAGGED>();
        case 4: return pick_fit<WBITS, P, RM, NT, NW, 4, SLICED, RAGGED>();
        case 8: return pick_fit<WBITS, P, RM, NT, NW, 8, SLICED, RAGGED>();
        default: return pick_fit<WBITS, P, RM, NT, NW, 16, SLICED, RAGGED>();
    }
}

// The instance for kWsplitTiles[tile] (nullptr for an unknown index), one case per table entry.
template <int WBITS, int P, bool SLICED, bool RAGGED, int T = 0>
WsplitFn pick_tile(int tile, int s) {
    if constexpr (T < kNumWsplitTiles) {
        constexpr WsplitTile t = kWsplitTiles[T];
        if (tile == T) return pick_s<WBITS, P, t.rm, t.nt, t.nw, SLICED, RAGGED>(s);
        return pick_tile<WBITS, P, SLICED, RAGGED, T + 1>(tile, s);
    } else {
        return nullptr;
    }
}

template <int WBITS, int P>
WsplitFn pick_flags(int tile, int s, bool sliced, bool ragged) {
    if (sliced) return ragged ? pick_tile<WBITS, P, true, true>(tile, s) : pick_tile<WBITS, P, true, false>(tile, s);
    return ragged ? pick_tile<WBITS, P, false, true>(tile, s) : pick_tile<WBITS, P, false, false>(tile, s);
}

}  // namespace

namespace kea {

#if KEA_WSPLIT_P == 1
WsplitFn wsplit_pick_p1(int wbits, int tile, int s, bool sliced, bool ragged) {
#elif KEA_WSPLIT_P == 2
WsplitFn wsplit_pick_p2(int wbits, int tile, int s, bool sliced, bool ragged) {
#else
WsplitFn wsplit_pick_p3(int wbits, int tile, int s, bool sliced, bool ragged) {
#endif
    return wbits == 1 ? pick_flags<1, KEA_WSPLIT_P>(tile, s, sliced, ragged)
                      : pick_flags<2, KEA_WSPLIT_P>(tile, s, sliced, ragged);
}

}  // namespace kea
