// The LDS-ring low-bit GEMM kernel (gemm_kernel) and its tile table, shared by the translation units that instantiate
// it (kea_gemm_ring_w1.hip, kea_gemm_ring_w2.hip: one per weight width, compiled in parallel) and by the host code of
// kea_gemm.hip (validation, tile choice, launch).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "kea_gemm_common.h"

namespace kea {

// Stage geometry shared by the kernels and the host launcher. A stage is 256 k (2 native words at 1 bit, 4 at 2
// bits), i.e. 16 activation units of 16 bytes per row. The ring depth NS is kMaxStages unless the LDS budget
// (kLdsBudget, the 160 KB a gfx950 workgroup may allocate) or the 6-bit vmcnt counter allow fewer (at least 2).
struct StageShape {
    int sw;           // native words per stage
    int stage_bytes;  // LDS bytes per ring buffer
    int copies;       // global->LDS copies per wavefront per stage
    int ns;           // ring buffers
};
constexpr int kLdsBudget = 160 * 1024;
// Ring depth cap. Sweeps on MI355X over the BASELINE shapes: two buffers per workgroup beat deeper rings nearly
// everywhere (up to 1.7x at P = 3), because the LDS a deeper ring takes costs more in co-resident workgroups (the
// latency hiding that matters) than the extra stages in flight give back. Grids of at most one workgroup per CU
// (small M, K = 4096) measured slower with eight buffers too: there a stage's time is set by the copies' throughput,
// not by their latency.
#ifndef KEA_MAX_STAGES
#define KEA_MAX_STAGES 2
#endif
constexpr int kMaxStages = KEA_MAX_STAGES;

#ifndef KEA_STAGE_K
#define KEA_STAGE_K 256
#endif
// Tiles with P * RM at most this read a whole stage's LDS operands before its first MFMA (see compute below).
#ifndef KEA_FULL_PRM
#define KEA_FULL_PRM 2
#endif
__host__ __device__ constexpr StageShape stage_shape(int wbits, int parts, int rm, int rn, int wm, int wn, int pw = 0) {
    const int nw = pw > 0 ? pw : wm * wn, bm = wm * rm * 16, bn = wn * rn * 16;  // nw: the waves issuing copies
    const int sw = KEA_STAGE_K / (wbits == 1 ? 128 : 64);
    const int a_units = parts * bm * (KEA_STAGE_K / 16);
    const int b_words = (bn / 16) * sw;
    const int stage = a_units * 16 + b_words * 256;
    const int copies = a_units / 64 / nw + b_words / nw;
    int ns = kLdsBudget / stage;
    if (ns > 63 / copies + 1) ns = 63 / copies + 1;
    if (ns > kMaxStages) ns = kMaxStages;
    if (ns < 2) ns = 2;
    return StageShape{sw, stage, copies, ns};
}

// pw > 0: the workgroup has pw more waves that only issue the global->LDS copies of the ring (producer waves),
// while the wm x wn compute waves only read LDS and run the MFMAs and the epilogue.
struct Tile {
    int rm, rn, wm, wn;
    const char *name;
    int pw = 0;
};

// Tile configurations (ids are 1-based in the ABI). Results are identical for every tile.
constexpr Tile kTiles[] = {
    {1, 1, 1, 4, "16x64 w1x4 r1x1"},   // 1
    {2, 1, 1, 4, "32x64 w1x4 r2x1"},   // 2
    {1, 2, 2, 2, "32x64 w2x2 r1x2"},   // 3
    {1, 1, 2, 2, "32x32 w2x2 r1x1"},   // 4
    {4, 1, 1, 4, "64x64 w1x4 r4x1"},   // 5
    {4, 2, 2, 4, "128x128 w2x4 r4x2 p8", 8},  // 6: tile 11's compute waves and 8 producer waves
    {4, 2, 1, 4, "64x128 w1x4 r4x2 p4", 4},   // 7: tile 8's compute waves and 4 producer waves
    {4, 2, 1, 4, "64x128 w1x4 r4x2"},  // 8
    {2, 2, 1, 4, "32x128 w1x4 r2x2"},  // 9
    {2, 4, 2, 4, "64x256 w2x4 r2x4"},  // 10
    {4, 2, 2, 4, "128x128 w2x4 r4x2"}, // 11
    {1, 2, 2, 4, "32x128 w2x4 r1x2"},  // 12
};
constexpr int kNumTiles = sizeof(kTiles) / sizeof(kTiles[0]);

// Register budget of a tile: accumulators plus double-buffered activation fragments (in 32-bit registers). Up to 8
// waves per workgroup (two per SIMD) they may take 256 of a wave's 256; with more waves a SIMD holds three or four of
// them in its 512 registers per lane, and the arrays must leave 64 of a wave's share to the rest of the kernel. Two
// ring buffers of the tile's stage must fit the LDS a workgroup may allocate.
constexpr bool tile_fits(int wbits, int parts, int rm, int rn, int wm, int wn, int pw = 0) {
    const int waves = wm * wn + pw, per_simd = (waves + 3) / 4;
    return parts * rm * rn * 4 + 2 * parts * rm * 4 <= (waves <= 8 ? 256 : 512 / per_simd - 64) &&
           2 * stage_shape(wbits, parts, rm, rn, wm, wn, pw).stage_bytes <= kLdsBudget;
}

using KernelFn = void (*)(Params);

// The ring kernel instance for a tile id of kTiles (sliced: split-K partials; ktail: byte-precise K masking; gq > 0:
// per-group weight scales of 64 * gq k), or nullptr when the tile does not fit. Defined per weight width.
KernelFn ring_pick_w1(int parts, int id, bool sliced, bool ktail, int gq);
KernelFn ring_pick_w2(int parts, int id, bool sliced, bool ktail, int gq);

// K % 16 != 0 runs the byte-precise variant of tile kTailTile, unsplit.
constexpr int kTailTile = 4;

}  // namespace kea
