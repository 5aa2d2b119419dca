// The wave-split low-bit GEMM (kea_gemm_wsplit.hip): tile table and launcher shared with the host code of
// kea_gemm.hip, which owns argument validation and the choice between this kernel and the LDS-ring kernel.
#pragma once

#include <hip/hip_runtime.h>

#include "kea_gemm_common.h"

namespace kea {

// A wave-split tile: BM = 16 * rm activation rows x BN = 16 * nt output columns per workgroup of nw wave64s. The
// workgroup's K range is cut into nw consecutive ranges of `s` k-steps of 64, one per wave; each wave loads its
// operands straight into registers and runs its MFMAs, and the nw partial int32 tiles are summed through LDS in
// wave order (exact) before the epilogue.
struct WsplitTile {
    int rm, nt, nw;
    const char *name;
};

constexpr WsplitTile kWsplitTiles[] = {
    {1, 8, 4, "16x128 k/4"},    // first wave-split id
    {2, 4, 4, "32x64 k/4"},
    {1, 4, 4, "16x64 k/4"},
    {1, 8, 8, "16x128 k/8"},
    {2, 4, 8, "32x64 k/8"},
    {1, 2, 4, "16x32 k/4"},
    {2, 8, 4, "32x128 k/4"},
    {1, 4, 8, "16x64 k/8"},
    {1, 2, 8, "16x32 k/8"},
    {1, 1, 8, "16x16 k/8"},
    {1, 1, 4, "16x16 k/4"},
};
constexpr int kNumWsplitTiles = sizeof(kWsplitTiles) / sizeof(kWsplitTiles[0]);

// k-steps per wave that have kernel instances (the largest covers 16 x 64 = 1024 k per wave)
constexpr int kWsplitSteps[] = {2, 4, 8, 16};

// Steps per wave for `steps` k-steps of 64 over `nw` waves: the smallest instantiated count that covers them (even
// for 1-bit weights, whose words hold two k-steps), or 0 when none does.
inline int wsplit_steps(int wbits, long long steps, int nw) {
    long long need = (steps + nw - 1) / nw;
    if (wbits == 1) need = (need + 1) & ~1LL;
    for (int s : kWsplitSteps)
        if (s >= need) return s;
    return 0;
}

// Registers a wave of the tile needs for `s` steps (operands + accumulators, 32-bit), and whether that fits the
// register file share of one wave (nw = 4: one wave per SIMD; nw = 8: two), with room left for addresses and
// temporaries.
constexpr int wsplit_reg_budget(int nw) { return nw == 4 ? 320 : 160; }

// LDS bytes of the partial-sum exchange: nw waves x parts x rm x nt blocks of 64 lanes x 4 int32.
inline int wsplit_lds_bytes(int parts, const WsplitTile &t) { return t.nw * parts * t.rm * t.nt * 1024; }

inline bool wsplit_fits(int wbits, int parts, const WsplitTile &t, int s) {
    const int words = wbits == 1 ? s / 2 : s;
    const int regs = parts * t.rm * s * 4 + t.nt * words + parts * t.rm * t.nt * 4;
    return regs <= wsplit_reg_budget(t.nw) && wsplit_lds_bytes(parts, t) <= 160 * 1024;
}

using WsplitFn = void (*)(const int8_t *, const uint32_t *, const void *, const void *, int, int, int, int, int,
                         int, Params);

// The kernel instance for a wave-split tile index, s k-steps per wave, SLICED and RAGGED flags (nullptr when that
// register budget does not fit). Defined per activation part count.
WsplitFn wsplit_pick_p1(int wbits, int tile, int s, bool sliced, bool ragged);
WsplitFn wsplit_pick_p2(int wbits, int tile, int s, bool sliced, bool ragged);
WsplitFn wsplit_pick_p3(int wbits, int tile, int s, bool sliced, bool ragged);

// A resolved wave-split launch: kernel instance, grid, workgroup size, dynamic LDS and the dtype bits of its scales.
struct WsplitLaunch {
    WsplitFn fn;
    dim3 grid, block;
    int lds;
    int meta;
};

// Resolves the launch of the wave-split kernel over grid (ceil(N / BN), ceil(M / BM), splits) with `s` k-steps per
// wave (p.steps_per_slice is the K range of one workgroup in k-steps) and raises the kernel's LDS limit where it needs
// more than 64 KiB. SLICED: the kernel writes int32 slices. Returns a hipError_t.
hipError_t wsplit_prepare(const Params &p, int wbits, int parts, int tile, int s, int splits, bool sliced,
                          WsplitLaunch *out);

// Enqueues a resolved wave-split launch on `stream`; returns the launch's hipError_t.
inline hipError_t wsplit_enqueue(const WsplitLaunch &l, const Params &p, hipStream_t stream) {
    hipLaunchKernelGGL(l.fn, l.grid, l.block, l.lds, stream, p.q, p.w, p.qs, p.ws, p.M, p.N, p.K, (int)p.ldq, l.meta,
                       (int)p.part_stride, p);
    return hipGetLastError();
}

}  // namespace kea
