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

// Whether an instance reads 1-bit weights from the bit-plane part of the native layout (one v_and_b32 per 4 weights,
// plus one MFMA per k-step for the activation row sums) rather than from the word part (a mask and a byte permute per 4
// weights). Measured over the tile sweep's shapes on MI355X: bit-planes are 4-17% faster with one activation part on
// tiles of 4 or 8 n-tiles and 7-10% faster with two parts on 16 x 128 tiles; on narrower tiles and at three parts the
// extra row-sum MFMA costs more than the cheaper expansion saves (up to 10% slower on 16 x 16 tiles).
constexpr bool wsplit_planes(int wbits, int parts, int rm, int nt) {
    return wbits == 1 && (parts == 1 ? nt >= 4 : parts == 2 && rm == 1 && nt == 8);
}

// 16x16 blocks a wave accumulates per part and row block: the tile's nt, plus (bit-plane weights) the block of
// activation row sums that recovers the signed products from the masked ones.
constexpr int wsplit_blocks(bool planes, int nt) { return planes ? nt + 1 : nt; }

// Registers of one wave (operands + accumulators, 32-bit): activation fragments, weights (bit-planes: one 16-byte unit
// per k-step; words: one per n-tile and native word, which holds two k-steps at 1 bit and one at 2 bits) and the
// accumulator blocks.
constexpr int wsplit_regs_of(bool planes, int wbits, int parts, int rm, int nt, int s) {
    return parts * rm * s * 4 + (planes ? 4 * s : nt * (wbits == 1 ? s / 2 : s)) +
           parts * rm * wsplit_blocks(planes, nt) * 4;
}
constexpr int wsplit_regs(int wbits, int parts, int rm, int nt, int s) {
    return wsplit_regs_of(wsplit_planes(wbits, parts, rm, nt), wbits, parts, rm, nt, s);
}

// int32 of one wave's slice of the partial-sum exchange: parts x rm x nt blocks of 64 lanes x 4, plus (bit-planes) the
// row sums, one int32 per lane for each part and row block.
constexpr int wsplit_part(bool planes, int parts, int rm, int nt) { return parts * rm * (nt * 256 + (planes ? 64 : 0)); }

// LDS bytes of the partial-sum exchange: nw wave slices.
constexpr int wsplit_lds(int wbits, int parts, int rm, int nt, int nw) {
    return nw * wsplit_part(wsplit_planes(wbits, parts, rm, nt), parts, rm, nt) * 4;
}
inline int wsplit_lds_bytes(int wbits, int parts, const WsplitTile &t) {
    return wsplit_lds(wbits, parts, t.rm, t.nt, t.nw);
}

inline bool wsplit_fits(int wbits, int parts, const WsplitTile &t, int s) {
    return wsplit_regs(wbits, parts, t.rm, t.nt, s) <= wsplit_reg_budget(t.nw) &&
           wsplit_lds_bytes(wbits, parts, t) <= 160 * 1024;
}

// The per-group kernel reads the word part of the 1-bit layout and keeps one accumulator block per n-tile.
inline bool wsplit_group_regs_fit(int wbits, int parts, const WsplitTile &t, int s) {
    return wsplit_regs_of(false, wbits, parts, t.rm, t.nt, s) <= wsplit_reg_budget(t.nw);
}

using WsplitFn = void (*)(const int8_t *, const uint32_t *, const void *, const void *, int, int, int, int, int,
                         int, Params);

// The kernel instance for a wave-split tile index, s k-steps per wave, SLICED and RAGGED flags (nullptr when that
// register budget does not fit). Defined per activation part count.
WsplitFn wsplit_pick_p1(int wbits, int tile, int s, bool sliced, bool ragged);
WsplitFn wsplit_pick_p2(int wbits, int tile, int s, bool sliced, bool ragged);
WsplitFn wsplit_pick_p3(int wbits, int tile, int s, bool sliced, bool ragged);

// Per-group weight scales on a wave-split tile (kea_gemm_wsplit_group_inst.h): instances for 16-row tiles of at most
// four n-tiles whose workgroup covers K exactly, gq k-steps of 64 per group. Defined per activation part count.
WsplitFn wsplit_group_pick_p1(int wbits, int tile, int gq, int s);
WsplitFn wsplit_group_pick_p2(int wbits, int tile, int gq, int s);
WsplitFn wsplit_group_pick_p3(int wbits, int tile, int gq, int s);

// Outputs each thread of a per-group launch folds (1, 2 or 4 consecutive columns of one row of the 16 x 16nt tile).
constexpr int wsplit_group_opt(int nt, int nw) {
    return 256 * nt >= nw * 64 * 4 ? 4 : 256 * nt >= nw * 64 * 2 ? 2 : 1;
}

// Whether a per-group launch holds each thread's alpha values in registers (threads folding one output, with room in
// the wave's register budget for the tile's operands and accumulators, the G alpha words and a 64-register chunk of
// group sums); otherwise the tile's alpha block is staged in LDS as f32 and read per group. (Register-held alpha for two
// outputs a thread measured slower than LDS staging: 9.6 against 6.3 us at config 2 on the 16x32 k/4 tile.)
constexpr bool wsplit_group_alpha_regs(int parts, int nt, int nw, int s, int gq) {
    const int groups = nw * (s / gq);
    return wsplit_group_opt(nt, nw) == 1 && groups <= 64 &&
           parts * s * 4 + nt * s + parts * nt * 4 + groups + 64 <= wsplit_reg_budget(nw);
}

// LDS bytes of a per-group launch: each of the tile's nw * s / gq groups has its int32 sums (parts x nt blocks of 64
// lanes x 4) and its staged alpha: with alpha held in registers the tile's raw [16 * nt][G] block (f32 at most),
// otherwise one f32 row of 16 * nt + 4 floats per group.
constexpr int wsplit_group_lds(int parts, int nt, int nw, int s, int gq) {
    return nw * (s / gq) * (parts * nt * 1024 + (wsplit_group_alpha_regs(parts, nt, nw, s, gq) ? nt * 16 * 4
                                                                                                   : (nt * 16 + 4) * 4));
}
inline int wsplit_group_lds_bytes(int parts, const WsplitTile &t, int s, int gq) {
    return wsplit_group_lds(parts, t.nt, t.nw, s, gq);
}

// k-steps per wave of a per-group launch of tile t at this K (one workgroup covering K exactly with whole groups per
// wave and whole weight quads per wave), or 0 when the tile cannot take per-group scales at this K.
inline int wsplit_group_steps(int wbits, int parts, long long k, const WsplitTile &t, int gq) {
    if (t.rm != 1 || t.nt > 4 || k % 64 != 0) return 0;
    const long long ksteps = k / 64;
    if (ksteps % t.nw != 0) return 0;
    const long long s = ksteps / t.nw;
    if (s != 2 && s != 4 && s != 8 && s != 16) return 0;
    if (s % gq != 0 || (wbits == 1 && s % 2 != 0)) return 0;
    const long long words = wbits == 1 ? s / 2 : s, J = wbits == 1 ? (k + 127) / 128 : ksteps;
    if (words > 1 && J % 4 != 0) return 0;
    if (!wsplit_group_regs_fit(wbits, parts, t, (int)s) || wsplit_group_lds_bytes(parts, t, (int)s, gq) > 160 * 1024)
        return 0;
    return (int)s;
}

// A resolved wave-split launch: kernel instance, grid, workgroup size, dynamic LDS, the dtype bits of its scales and
// the word offset of the weight layout part it reads (the bit-plane part where wsplit_planes says so).
struct WsplitLaunch {
    WsplitFn fn;
    dim3 grid, block;
    int lds;
    int meta;
    long long w_off;
};

// Resolves the launch of the wave-split kernel over grid (ceil(N / BN), ceil(M / BM), splits) with `s` k-steps per
// wave (p.steps_per_slice is the K range of one workgroup in k-steps) and raises the kernel's LDS limit where it needs
// more than 64 KiB. SLICED: the kernel writes int32 slices. Returns a hipError_t.
hipError_t wsplit_prepare(const Params &p, int wbits, int parts, int tile, int s, int splits, bool sliced,
                          WsplitLaunch *out);

// Resolves a per-group launch of tile `tile` (s = wsplit_group_steps(...) != 0, p.groups set): grid
// (ceil(N / BN), ceil(M / 16)), the instance and its LDS. Returns a hipError_t.
hipError_t wsplit_group_prepare(const Params &p, int wbits, int parts, int tile, int gq, int s, WsplitLaunch *out);

// Enqueues a resolved wave-split launch on `stream`; returns the launch's hipError_t.
inline hipError_t wsplit_enqueue(const WsplitLaunch &l, const Params &p, hipStream_t stream) {
    hipLaunchKernelGGL(l.fn, l.grid, l.block, l.lds, stream, p.q, p.w + l.w_off, p.qs, p.ws, p.M, p.N, p.K,
                       (int)p.ldq, l.meta, (int)p.part_stride, p);
    return hipGetLastError();
}

}  // namespace kea
