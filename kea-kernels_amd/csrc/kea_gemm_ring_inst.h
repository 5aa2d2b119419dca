// Instances of the LDS-ring GEMM kernel for one weight width (KEA_RING_WBITS), included by kea_gemm_ring_w1.hip and
// kea_gemm_ring_w2.hip so the two widths compile in parallel.
#pragma once

#include "kea_gemm_ring.h"

#ifndef KEA_RING_WBITS
#error "define KEA_RING_WBITS (1 or 2) before including kea_gemm_ring_inst.h"
#endif

namespace {

using namespace kea;

// Waits until at most N vector-memory operations of this wavefront are outstanding (gfx9 s_waitcnt encoding:
// vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt left at their "no wait" maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier without the release/acquire fences of __syncthreads(): those make the compiler wait for every
// in-flight global->LDS copy (vmcnt(0)), which would drain the ring. The kernel's explicit vmcnt waits already
// guarantee that the copies a stage needs have landed; the empty asm statements keep the compiler from moving LDS
// accesses across the barrier.
__device__ __forceinline__ void stage_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

typedef __attribute__((address_space(1))) const void *gptr_t;
typedef __attribute__((address_space(3))) void *lptr_t;

__device__ __forceinline__ void dma16(const void *g, void *lds_wave_base) {
    __builtin_amdgcn_global_load_lds((gptr_t)g, (lptr_t)lds_wave_base, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void *g, void *lds_wave_base) {
    __builtin_amdgcn_global_load_lds((gptr_t)g, (lptr_t)lds_wave_base, 4, 0, 0);
}

// One workgroup: BM = WM*RM*16 activation rows x BN = WN*RN*16 output columns, WM x WN wavefronts; a wavefront owns
// RM x RN 16x16 tiles for each of the P parts. SLICED: blockIdx.z is a K slice writing int32 partials.
//
// K is streamed in stages of SW native words (SW*128 k for 1-bit, SW*64 k for 2-bit) through a ring of NS LDS
// buffers. Every byte arrives by direct global->LDS copies (global_load_lds: 16 bytes per lane for activations, 4 per
// lane for weight words), issued NS-1 stages ahead and tracked with vmcnt, so up to (NS-1)*SW words of K are in
// flight per workgroup and no VGPR holds staging data. Each wavefront issues the same number of copies per stage
// (out-of-range sources are clamped to a valid address and their bytes are never used), which keeps the vmcnt
// arithmetic exact. Activation rows are stored as 16-byte units with an XOR swizzle so that the 16 rows read by one
// MFMA operand fetch land in distinct LDS bank groups. KTAIL kernels serve K % 16 != 0 (byte-precise K masking).
//
// GQ > 0: per-group weight scales, one group per GQ k-steps of 64 (ws_group = 64 * GQ). The tile's block of alpha
// ([N][G] in memory) is staged once into LDS as f32 [group][column] (zero rows past the last group), and after the
// last k-step of each group every lane folds that group's exact int32 sums into an FP32 running value:
// r = fma(comb_P(acc - acc_at_previous_group_end), alpha[n][g], r). Group ends are fixed positions of the unrolled
// stage, so the folding is straight-line code; accumulators are only read there.
//
// PW > 0 (producer waves): waves NW .. NW + PW - 1 of the workgroup issue every copy and wait for them, and the NW
// compute waves never wait on memory counters for the ring; the stage barriers hand the buffers between the two.
template <int WBITS, int P, int RM, int RN, int WM, int WN, bool SLICED, bool KTAIL, int GQ = 0, int PW = 0>
__global__ void __launch_bounds__((WM * WN + PW) * 64) gemm_kernel(Params p) {
    static_assert(GQ == 0 || GQ == 1 || GQ == 2 || GQ == 4, "groups of 64, 128 or 256 k");
    static_assert(GQ == 0 || !SLICED, "per-group scales run unsplit");
    static_assert(PW == 0 || GQ == 0, "producer waves: no per-group scales");
    constexpr StageShape SHAPE = stage_shape(WBITS, P, RM, RN, WM, WN, PW);
    constexpr int SW = SHAPE.sw, NS = SHAPE.ns;
    constexpr int NW = WM * WN;                 // compute wavefronts
    constexpr int NI = PW > 0 ? PW : NW;        // wavefronts issuing the copies
    constexpr int BM = WM * RM * 16, BN = WN * RN * 16;
    constexpr int KW = WBITS == 1 ? 128 : 64;   // k per native word
    constexpr int KS = KW / 64;                 // MFMA k-steps per word
    constexpr int CHS = SW * KW / 16;           // 16-byte activation units per row per stage
    constexpr int SWZ_DIV = CHS >= 16 ? 1 : 16 / CHS;
    constexpr int SWZ_MASK = (CHS >= 16 ? 16 : CHS) - 1;
    constexpr int A_UNITS = P * BM * CHS;
    constexpr int A_BYTES = A_UNITS * 16;
    constexpr int B_WORDS = (BN / 16) * SW;     // (tile, word) pairs per stage, 64 lanes each
    constexpr int STAGE_BYTES = A_BYTES + B_WORDS * 256;
    constexpr int LA = A_UNITS / 64 / NI;       // activation copies per issuing wavefront per stage
    constexpr int LB = B_WORDS / NI;            // weight copies per issuing wavefront per stage
    constexpr int L = LA + LB;
    static_assert(A_UNITS % (64 * NI) == 0, "activation stage must split evenly over the issuing wavefronts");
    static_assert(B_WORDS % NI == 0, "weight stage must split evenly over the issuing wavefronts");
    static_assert(L * (NS - 1) < 64, "in-flight copies exceed the vmcnt range");
    static_assert(L == SHAPE.copies && STAGE_BYTES == SHAPE.stage_bytes, "host and device stage geometry differ");
    static_assert(NS >= 2, "at least double buffering");
    static_assert(NS * STAGE_BYTES <= kLdsBudget, "the ring exceeds the LDS a workgroup may allocate");
    extern __shared__ __attribute__((aligned(16))) int8_t lds[];  // NS * STAGE_BYTES

    // the wavefront index is uniform; readfirstlane tells the compiler so (wave-derived math then runs on SALU)
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool producer = PW > 0 && wave >= NW;  // wave-uniform
    const int iw = PW > 0 ? (producer ? wave - NW : 0) : wave;  // index among the issuing waves
    const int wm = wave / WN, wn = wave % WN;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int nquads = (p.J + 3) >> 2;
    const int qa = SLICED ? (int)blockIdx.z * p.quads_per_slice : 0;
    const int qb = SLICED ? min(nquads, qa + p.quads_per_slice) : nquads;
    const int ja = 4 * qa, jb = min(4 * qb, p.J);
    const int nst = (jb - ja + SW - 1) / SW;    // stages

    auto swz = [](int r) { return (r / SWZ_DIV) & SWZ_MASK; };

    // Per-lane copy sources, fixed for the whole K loop: q plus a 32-bit per-lane byte offset (the host guarantees
    // that q spans < 2 GiB), so every copy is one global_load_lds with a uniform base. Activation rows past M are
    // clamped to row M-1 (their outputs are never stored). Units at k >= kend (K, or the end of this split-K slice)
    // only occur in a workgroup's last stage; they copy the start of their row (in bounds) and the last stage's
    // compute zeroes the weights of those k.
    const int kend = min(p.K, jb * KW);
    uint32_t a_off[LA];
    int a_koff[LA];
#pragma unroll
    for (int i = 0; i < LA; ++i) {
        const int u = (i * NI + iw) * 64 + lane;
        const int row = u / CHS, chp = u - row * CHS;
        const int c = row / BM, r = row - c * BM;
        a_koff[i] = (chp ^ swz(r)) * 16;
        const int m = min(m0 + r, p.M - 1);
        a_off[i] = (uint32_t)(c * p.part_stride + (long long)m * p.ldq + a_koff[i]);
    }
    const int tile0 = n0 >> 4;
    const int jtail = (p.J - 1) & ~3, wq_tail = p.J - jtail;       // the last (possibly short) quad
    const uint32_t b_lane = (uint32_t)lane * 16u, b_lane_tail = (uint32_t)(lane * wq_tail) * 4u;

    // Issue the copies of stage s into ring buffer s % NS.
    auto issue = [&](int s) {
        int8_t *buf = lds + (s % NS) * STAGE_BYTES;
        const int jstage = ja + s * SW;
        const int k0 = jstage * KW;
        if (k0 + SW * KW <= kend) {  // uniform: every unit of the stage is inside [0, kend)
            const int8_t *abase = p.q + k0;
#pragma unroll
            for (int i = 0; i < LA; ++i) dma16(abase + a_off[i], buf + (i * NI + iw) * 64 * 16);
        } else {
#pragma unroll
            for (int i = 0; i < LA; ++i) {
                const uint32_t off = k0 + a_koff[i] < kend ? a_off[i] + (uint32_t)k0 : a_off[i] - (uint32_t)a_koff[i];
                dma16(p.q + off, buf + (i * NI + iw) * 64 * 16);
            }
        }
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            const int b = i * NI + iw;               // wave-uniform
            const int tt = b / SW, w = b - tt * SW;
            const int t = tile0 + tt, j = jstage + w;
            // words past the slice or past N are never used (their k are masked, their columns never stored)
            const int jj = j < jb ? j : ja, tc = t < p.NT ? t : p.NT - 1;
            const int jq = jj & ~3;
            const char *wbase = (const char *)(p.w + ((long long)tc * p.J + jq) * 64 + (jj & 3));
            dma4(wbase + (jq == jtail ? b_lane_tail : b_lane), buf + A_BYTES + b * 256);
        }
    };

    v4i acc[P][RM][RN];
#pragma unroll
    for (int c = 0; c < P; ++c)
#pragma unroll
        for (int i = 0; i < RM; ++i)
#pragma unroll
            for (int jn = 0; jn < RN; ++jn) acc[c][i][jn] = (v4i){0, 0, 0, 0};

    // Epilogue operands (per-token scales also feed the per-group folding inside the K loop).
    EpiOperands rows[RM], cols[RN];

    // Per-group scales: FP32 running values, the accumulators at the previous group end, and the alpha block in LDS
    // (f32 [group][column], row stride ALD floats: 16-byte rows whose starts spread over the banks), placed after the
    // ring buffers this workgroup uses.
    constexpr int ALD = BN + 4;
    float racc[RM][RN][4];
    int prev[GQ > 0 ? P : 1][RM][RN][4];
    float *alds = (float *)(lds + min(NS, nst) * STAGE_BYTES);
    if constexpr (GQ > 0) {
#pragma unroll
        for (int i = 0; i < RM; ++i)
#pragma unroll
            for (int jn = 0; jn < RN; ++jn)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    racc[i][jn][r] = 0.f;
#pragma unroll
                    for (int c = 0; c < P; ++c) prev[c][i][jn][r] = 0;
                }
    }

    // Folds the group that ends with the k-step starting at kstep into racc (per-group scales only).
    auto fold = [&](int kstep) {
        if constexpr (GQ > 0) {
        const int g = kstep / (64 * GQ);
#pragma unroll
        for (int jn = 0; jn < RN; ++jn) {
            const float4 al = *(const float4 *)(alds + g * ALD + (wn * RN + jn) * 16 + (lane >> 4) * 4);
            const float alv[4] = {al.x, al.y, al.z, al.w};
#pragma unroll
            for (int i = 0; i < RM; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int d[3] = {0, 0, 0};
#pragma unroll
                    for (int c = 0; c < P; ++c) {
                        d[c] = acc[c][i][jn][r] - prev[c][i][jn][r];
                        prev[c][i][jn][r] = acc[c][i][jn][r];
                    }
                    racc[i][jn][r] = __builtin_fmaf(combine<P>(d, rows[i].s, p.flags), alv[r], racc[i][jn][r]);
                }
        }
        }
    };

    // One stage of MFMAs: straight-line code. No accumulator may pass a control-flow merge (an `if` around MFMAs, a
    // loop whose trip count is not a compile-time constant): at such merges the compiler emitted AGPR copy chains, and
    // those builds returned wrong values in accumulator component 0. The masked last stage is therefore a separate
    // instantiation rather than a branch inside the loop; after any change here, run the every-tile and every-split
    // GPU tests, which compare every tile and split with the oracle. Operand reads from LDS run ahead of the MFMAs:
    // narrow tiles (P * RM <= 2, few MFMAs per k-step) issue every read of the stage before the first MFMA, so a stage
    // pays one LDS latency instead of one per k-step; wider tiles read k-step t + 1 while the MFMAs of step t run.
    // MASKED (the last stage) zeroes the weights at k >= kend: per 16-byte group of a lane's operand, or per byte for
    // KTAIL.
    auto compute = [&](int s, auto masked_tag) {
        constexpr bool MASKED = decltype(masked_tag)::value;
        const int8_t *buf = lds + (s % NS) * STAGE_BYTES;
        constexpr int STEPS = SW * KS;  // MFMA k-steps per stage
        constexpr bool FULL = P * RM <= KEA_FULL_PRM;
        constexpr int ASLOTS = FULL ? STEPS : 2, WSLOTS = FULL ? SW : 2;
        v4i af[ASLOTS][P][RM];
        uint32_t wv[WSLOTS][RN];
        auto fetch = [&](int t, int slot) {
            const int w = t / KS, h = t % KS;
            if (h == 0) {
#pragma unroll
                for (int jn = 0; jn < RN; ++jn)
                    wv[w % WSLOTS][jn] =
                        *(const uint32_t *)(buf + A_BYTES + ((wn * RN + jn) * SW + w) * 256 + lane * 4);
            }
#pragma unroll
            for (int c = 0; c < P; ++c)
#pragma unroll
                for (int i = 0; i < RM; ++i) {
                    const int r = (wm * RM + i) * 16 + (lane & 15);
                    const int ch = w * (KW / 16) + h * 4 + (lane >> 4);
                    af[slot][c][i] = *(const v4i *)(buf + ((c * BM + r) * CHS + (ch ^ swz(r))) * 16);
                }
        };
        if constexpr (FULL) {
#pragma unroll
            for (int t = 0; t < STEPS; ++t) fetch(t, t);
        } else {
            fetch(0, 0);
        }
#pragma unroll
        for (int t = 0; t < STEPS; ++t) {
            const int w = t / KS, h = t % KS;
            if (!FULL && t + 1 < STEPS) fetch(t + 1, (t + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);  // keep the next k-step's LDS reads ahead of this one's MFMAs
            const int slot = FULL ? t : t & 1;
            const int kstep = (ja + s * SW + w) * KW + h * 64;
#pragma unroll
            for (int jn = 0; jn < RN; ++jn) {
                const uint32_t w32 = wv[w % WSLOTS][jn];
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
                if constexpr (MASKED && KTAIL) {
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const int valid = kend - (kstep + (lane >> 4) * 16 + 4 * d);
                        const uint32_t keep = valid >= 4 ? 0xFFFFFFFFu : (valid <= 0 ? 0u : (1u << (8 * valid)) - 1u);
                        bf[d] = (int)((uint32_t)bf[d] & keep);
                    }
                } else if constexpr (MASKED) {  // kend is a multiple of 16 here
                    const bool keep = kstep + (lane >> 4) * 16 < kend;
#pragma unroll
                    for (int d = 0; d < 4; ++d) bf[d] = keep ? bf[d] : 0;
                }
#pragma unroll
                for (int c = 0; c < P; ++c)
#pragma unroll
                    for (int i = 0; i < RM; ++i)
                        acc[c][i][jn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf, af[slot][c][i], acc[c][i][jn], 0, 0, 0);
            }
            // t is a fully unrolled step index, so group ends are compile-time positions (no branch)
            if constexpr (GQ > 0) {
                if ((t + 1) % GQ == 0) fold(kstep);
            }
        }
    };

    // Waits for stage s given that `later` stages were issued after it.
    auto wait_stage = [&](int later) {
        switch (later) {
            case 0: wait_vmcnt<0>(); break;
            case 1: wait_vmcnt<(NS > 1 ? L * 1 : 0)>(); break;
            case 2: wait_vmcnt<(NS > 2 ? L * 2 : 0)>(); break;
            case 3: wait_vmcnt<(NS > 3 ? L * 3 : 0)>(); break;
            case 4: wait_vmcnt<(NS > 4 ? L * 4 : 0)>(); break;
            case 5: wait_vmcnt<(NS > 5 ? L * 5 : 0)>(); break;
            case 6: wait_vmcnt<(NS > 6 ? L * 6 : 0)>(); break;
            default: wait_vmcnt<(NS > 7 ? L * 7 : 0)>(); break;
        }
    };
    static_assert(NS <= 8, "wait_stage covers up to 7 later stages");

    // Producer waves: every copy of the ring, each stage waited for and handed over at the stage barrier; they take
    // part in exactly the compute waves' barriers (nst of them) and leave before the epilogue.
    if constexpr (PW > 0) {
        if (producer) {
#pragma unroll
            for (int s = 0; s < NS - 1; ++s)
                if (s < nst) issue(s);
            for (int s = 0; s < nst - 1; ++s) {
                wait_stage(min(NS - 2, nst - 1 - s));
                stage_barrier();  // stage s is in LDS; the compute waves are done with stage s-1's buffer
                if (s + NS - 1 < nst) issue(s + NS - 1);
            }
            wait_vmcnt<0>();
            stage_barrier();
            return;
        }
    }

    // Epilogue operands are fetched before the ring so their latency overlaps the main loads (the copies below are
    // issued after these loads, so the stage waits never depend on them).
    if constexpr (!SLICED) {
#pragma unroll
        for (int i = 0; i < RM; ++i) load_row_scales<P>(p, m0 + (wm * RM + i) * 16 + (lane & 15), rows[i]);
#pragma unroll
        for (int jn = 0; jn < RN; ++jn)
            load_col_scales(p, n0 + (wn * RN + jn) * 16 + (lane >> 4) * 4, cols[jn], GQ == 0);
    }
    // Residual values: prefetched with the other epilogue operands on small tiles, loaded in the epilogue otherwise
    // (keeps the register budget of the wide tiles).
    constexpr bool RES_PREFETCH = !SLICED && RM * RN <= 2;
    float resv[RES_PREFETCH ? RM : 1][RES_PREFETCH ? RN : 1][4];
    if constexpr (RES_PREFETCH) {
        if (p.res) {
#pragma unroll
            for (int i = 0; i < RM; ++i)
#pragma unroll
                for (int jn = 0; jn < RN; ++jn)
                    load_residual(p, m0 + (wm * RM + i) * 16 + (lane & 15), n0 + (wn * RN + jn) * 16 + (lane >> 4) * 4,
                                  resv[i][jn]);
        }
    }

    // Per-group scales: the tile's alpha rows [n0, n0 + BN) x groups [0, 2^gp_shift) go to LDS as f32 in chunks of
    // ACH values per lane (zero past the last group; rows past N clamped, never stored). The first chunk's loads are
    // issued before the ring's and stored after, so their latency overlaps the first stage's.
    constexpr int ACH = 8;
    float av[ACH];
    const int atotal = BN << p.gp_shift, gmask = (1 << p.gp_shift) - 1;
    auto alpha_load = [&](int base) {
#pragma unroll
        for (int u = 0; u < ACH; ++u) {
            const int idx = base + (u * NW + wave) * 64 + lane;
            const int g = idx & gmask, c = idx >> p.gp_shift;
            av[u] = 0.f;
            if (c < BN && g < p.groups)
                av[u] = load_scalar(p.ws, p.ws_dtype, (long long)min(n0 + c, p.N - 1) * p.groups + g);
        }
    };
    auto alpha_store = [&](int base) {
#pragma unroll
        for (int u = 0; u < ACH; ++u) {
            const int idx = base + (u * NW + wave) * 64 + lane;
            const int g = idx & gmask, c = idx >> p.gp_shift;
            if (c < BN) alds[g * ALD + c] = av[u];
        }
    };
    if constexpr (GQ > 0) alpha_load(0);

    if constexpr (PW == 0) {
#pragma unroll
        for (int s = 0; s < NS - 1; ++s)
            if (s < nst) issue(s);
    }

    if constexpr (GQ > 0) {
        alpha_store(0);
        for (int base = ACH * 64 * NW; base < atotal; base += ACH * 64 * NW) {
            alpha_load(base);
            alpha_store(base);
        }
        // LDS writes complete before the first stage barrier publishes them (lgkmcnt(0); vmcnt, expcnt untouched)
        __builtin_amdgcn_s_waitcnt(0xF | (3 << 14) | (7 << 4));
    }
    using plain_t = std::integral_constant<bool, false>;
    using masked_t = std::integral_constant<bool, true>;
    for (int s = 0; s < nst - 1; ++s) {
        if constexpr (PW == 0) {
            const int issued_after = min(NS - 2, nst - 1 - s);  // stages issued after s so far
            wait_stage(issued_after);
        }
        stage_barrier();  // stage s is in LDS for every wavefront; stage s-1's buffer is free
        if constexpr (PW == 0) {
            if (s + NS - 1 < nst) issue(s + NS - 1);
        }
        compute(s, plain_t{});
    }
    // the last stage (the host never launches an empty K range, so nst >= 1)
    if constexpr (PW == 0) wait_vmcnt<0>();
    stage_barrier();
    compute(nst - 1, masked_t{});

    // ---- epilogue: the MFMA result row is the weight row n, the column the activation row m ----
    // DT >= 0: the output dtype as a compile-time constant; then 16x16 tiles wholly inside [M, N) take a path without
    // per-lane bounds or dtype selection (the tile test is wave-uniform). DT < 0: the general epilogue.
    constexpr bool SMALL = RM * RN <= 2;
    auto epilogue = [&](auto dt_tag, auto res_tag, auto silu_tag, auto glu_tag) {
        constexpr int DT = decltype(dt_tag)::value;
        constexpr bool RES = decltype(res_tag)::value;
        constexpr int SILU = decltype(silu_tag)::value;
        constexpr bool GLU = decltype(glu_tag)::value;
#pragma unroll
        for (int i = 0; i < RM; ++i) {
            const int mt = m0 + (wm * RM + i) * 16, m = mt + (lane & 15);
            if (m >= p.M) continue;
            void *yrow = (int8_t *)p.y + (long long)m * p.ldy * (DT == KEA_F32 ? 4 : 2);  // unused when DT < 0
#pragma unroll
            for (int jn = 0; jn < RN; ++jn) {
                const int nt = n0 + (wn * RN + jn) * 16, nb = nt + (lane >> 4) * 4;
                if (nb >= p.N) continue;
                int a[P][4];
#pragma unroll
                for (int c = 0; c < P; ++c)
#pragma unroll
                    for (int r = 0; r < 4; ++r) a[c][r] = acc[c][i][jn][r];
                if constexpr (SLICED) {
#pragma unroll
                    for (int c = 0; c < P; ++c)
                        store_int4(p.slices + (((long long)blockIdx.z * P + c) * p.M + m) * p.N + nb, p.slice_vec,
                                   nb, p.N, a[c]);
                } else {
                    EpiOperands e = cols[jn];
#pragma unroll
                    for (int c = 0; c < 3; ++c) e.s[c] = rows[i].s[c];
                    if constexpr (RES_PREFETCH) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) e.res[r] = resv[i][jn][r];
                    } else {
                        load_residual(p, m, nb, e.res);
                    }
                    if constexpr (GQ > 0) {
                        epilogue4_groups<P>(p, m, nb, a, racc[i][jn], e);
                    } else if constexpr (DT >= 0) {
                        if (mt + 16 <= p.M && nt + 16 <= p.N) {
                            epilogue4_full<P, DT, RES, SMALL, SILU, GLU>(p, yrow, nb, a, e);
                            continue;
                        }
                        epilogue4<P>(p, m, nb, a, e);
                    } else {
                        epilogue4<P>(p, m, nb, a, e);
                    }
                }
            }
        }
    };
    // Outputs without raw accumulators and with a vector-aligned y branch once on the dtype (and GLU outputs, which
    // take neither residual nor SiLU, on the GLU); the rest take the general epilogue.
    const bool glu = (p.flags & KEA_FLAG_GLU) != 0;
    const bool plain = !SLICED && GQ == 0 && p.y && !p.acc && p.y_vec && !glu;
    const bool plain_glu = !SLICED && GQ == 0 && p.y && !p.acc && p.y_vec && glu && !p.res;
    using kRes = std::true_type;
    using kNoRes = std::false_type;
    using kGlu = std::true_type;
    using kNoGlu = std::false_type;
    using kSiluAtRunTime = std::integral_constant<int, -1>;
    using kNoSilu = std::integral_constant<int, 0>;
    using kGeneral = std::integral_constant<int, -1>;
    if (plain_glu) {
        if (p.y_dtype == KEA_F32) epilogue(std::integral_constant<int, KEA_F32>{}, kNoRes{}, kNoSilu{}, kGlu{});
        else if (p.y_dtype == KEA_F16) epilogue(std::integral_constant<int, KEA_F16>{}, kNoRes{}, kNoSilu{}, kGlu{});
        else epilogue(std::integral_constant<int, KEA_BF16>{}, kNoRes{}, kNoSilu{}, kGlu{});
        return;
    }
    // Tiles of one or two 16x16 blocks per wave (the small-M shapes) keep one epilogue copy per dtype with the
    // residual, bias and SiLU tested at run time: separate copies measured slower there (config 1: 4.13 vs 4.27 us).
    if constexpr (SMALL) {
        if (plain && p.y_dtype == KEA_F16) epilogue(std::integral_constant<int, KEA_F16>{}, kNoRes{}, kSiluAtRunTime{}, kNoGlu{});
        else if (plain && p.y_dtype == KEA_BF16) epilogue(std::integral_constant<int, KEA_BF16>{}, kNoRes{}, kSiluAtRunTime{}, kNoGlu{});
        else if (plain && p.y_dtype == KEA_F32) epilogue(std::integral_constant<int, KEA_F32>{}, kNoRes{}, kSiluAtRunTime{}, kNoGlu{});
        else epilogue(kGeneral{}, kNoRes{}, kSiluAtRunTime{}, kNoGlu{});
        return;
    }
    // Wider tiles: one copy per dtype, residual and SiLU, so the full-block path carries neither test nor a SiLU
    // evaluated only to be discarded.
    auto by_flags = [&](auto dt_tag) {
        const bool silu = (p.flags & KEA_FLAG_SILU) != 0;
        if (p.res) {
            if (silu) epilogue(dt_tag, kRes{}, std::integral_constant<int, 1>{}, kNoGlu{});
            else epilogue(dt_tag, kRes{}, kNoSilu{}, kNoGlu{});
        } else {
            if (silu) epilogue(dt_tag, kNoRes{}, std::integral_constant<int, 1>{}, kNoGlu{});
            else epilogue(dt_tag, kNoRes{}, kNoSilu{}, kNoGlu{});
        }
    };
    if (plain && p.y_dtype == KEA_F16) {
        by_flags(std::integral_constant<int, KEA_F16>{});
    } else if (plain && p.y_dtype == KEA_BF16) {
        by_flags(std::integral_constant<int, KEA_BF16>{});
    } else if (plain && p.y_dtype == KEA_F32) {
        by_flags(std::integral_constant<int, KEA_F32>{});
    } else {
        epilogue(kGeneral{}, kNoRes{}, kSiluAtRunTime{}, kNoGlu{});
    }
}

template <int WBITS, int P, int RM, int RN, int WM, int WN, int PW>
KernelFn pick_sliced(bool sliced) {
    return sliced ? gemm_kernel<WBITS, P, RM, RN, WM, WN, true, false, 0, PW>
                  : gemm_kernel<WBITS, P, RM, RN, WM, WN, false, false, 0, PW>;
}

template <int WBITS, int P, int RM, int RN, int WM, int WN, int PW>
KernelFn pick_fit(bool sliced) {
    if constexpr (tile_fits(WBITS, P, RM, RN, WM, WN, PW)) return pick_sliced<WBITS, P, RM, RN, WM, WN, PW>(sliced);
    else return nullptr;
}

// The instance of kTiles[I] (its geometry read from the table itself, so ids and shapes cannot drift apart).
template <int WBITS, int P, int I>
KernelFn pick_index(bool sliced) {
    constexpr Tile t = kTiles[I];
    return pick_fit<WBITS, P, t.rm, t.rn, t.wm, t.wn, t.pw>(sliced);
}

template <int WBITS, int P>
KernelFn pick_tile(int id, bool sliced) {
    static_assert(kNumTiles == 12, "one case per tile id");
    switch (id) {
        case 1: return pick_index<WBITS, P, 0>(sliced);
        case 2: return pick_index<WBITS, P, 1>(sliced);
        case 3: return pick_index<WBITS, P, 2>(sliced);
        case 4: return pick_index<WBITS, P, 3>(sliced);
        case 5: return pick_index<WBITS, P, 4>(sliced);
        case 6: return pick_index<WBITS, P, 5>(sliced);
        case 7: return pick_index<WBITS, P, 6>(sliced);
        case 8: return pick_index<WBITS, P, 7>(sliced);
        case 9: return pick_index<WBITS, P, 8>(sliced);
        case 10: return pick_index<WBITS, P, 9>(sliced);
        case 11: return pick_index<WBITS, P, 10>(sliced);
        case 12: return pick_index<WBITS, P, 11>(sliced);
        default: return nullptr;
    }
}

template <int WBITS, int P>
KernelFn pick_ktail() { return gemm_kernel<WBITS, P, 1, 1, 2, 2, false, true>; }

// Per-group scales: tile 1 (16x64, P >= 2) or tile 4 (32x32, P = 1, and the byte-precise K tail), unsplit.
template <int WBITS, int P, int GQ>
KernelFn pick_group_gq(int id, bool ktail) {
    if (ktail) return gemm_kernel<WBITS, P, 1, 1, 2, 2, false, true, GQ>;
    return id == 1 ? gemm_kernel<WBITS, P, 1, 1, 1, 4, false, false, GQ> : gemm_kernel<WBITS, P, 1, 1, 2, 2, false, false, GQ>;
}
template <int WBITS, int P>
KernelFn pick_group_p(int gq, int id, bool ktail) {
    if (gq == 1) return pick_group_gq<WBITS, P, 1>(id, ktail);
    if (gq == 2) return pick_group_gq<WBITS, P, 2>(id, ktail);
    return pick_group_gq<WBITS, P, 4>(id, ktail);
}

template <int P>
KernelFn pick_parts(int id, bool sliced, bool ktail, int gq) {
    if (gq) return pick_group_p<KEA_RING_WBITS, P>(gq, id, ktail);
    if (ktail) return pick_ktail<KEA_RING_WBITS, P>();
    return pick_tile<KEA_RING_WBITS, P>(id, sliced);
}

}  // namespace

namespace kea {

#if KEA_RING_WBITS == 1
KernelFn ring_pick_w1(int parts, int id, bool sliced, bool ktail, int gq) {
#else
KernelFn ring_pick_w2(int parts, int id, bool sliced, bool ktail, int gq) {
#endif
    return parts == 1 ? pick_parts<1>(id, sliced, ktail, gq)
         : parts == 2 ? pick_parts<2>(id, sliced, ktail, gq) : pick_parts<3>(id, sliced, ktail, gq);
}

}  // namespace kea
