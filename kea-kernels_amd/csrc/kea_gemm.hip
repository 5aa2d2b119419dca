// Low-bit GEMM for MI355X (gfx950): 1-bit sign / 2-bit ternary weights x int8 activations on int8 MFMA.
//
// What it computes is the reference's b1_dot / _int8_dot contract (kk/binary/kernels.py:7-16, :134-565;
// kk/binary/kernels_parts.py:28-55; kk/ternary/fused_kernels.py:53-120): P residual int8 activation parts, exact
// int32 accumulators acc_c = sum_k q_c[m, k] * w[n, k], then the FP32 epilogue
//     r = comb_P(acc, s) ; r = bias ? fma(r, alpha, bias) : r * alpha ; optional SiLU ; RN to the output type.
// How it computes it is gfx950-native:
//   * weights stay 1 or 2 bits per value in HBM in a wavefront-native word layout (kea_layout.cpp): a lane's four
//     consecutive words arrive with one 128-bit global load, and one word yields the int8 MFMA operand of its lane
//     for 2 (1-bit) or 1 (2-bit) k-steps of 64;
//   * expansion to int8 is a mask (v_and_b32) plus a byte permute (v_perm_b32) per 4 weights, with the permute's
//     constant table mapping the masked selector bytes to 0x01 / 0xFF (1-bit) or 0x00 / 0x01 / 0xFF (2-bit);
//   * activations and weight words both stream global -> LDS by direct copies (global_load_lds) into a ring of stage
//     buffers (256 k each; two by default), tracked with vmcnt; activation rows are XOR-swizzled 16-byte units;
//   * v_mfma_i32_16x16x64_i8 with the weight fragment as the A operand, so each lane ends up owning 4 consecutive
//     output columns of one row: the epilogue stores 8-byte (fp16/bf16) or 16-byte (fp32) vectors;
//   * split-K writes exact int32 slices [S][P][M][N] and a second kernel sums them in slice order (integer
//     addition is exact, so every split gives the unsplit result bit for bit).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <new>
#include <string>
#include <type_traits>

#include "kea_epilogue.h"
#include "kea_gemm_common.h"
#include "kea_gemm_ring.h"
#include "kea_gemm_table.h"
#include "kea_gemm_wsplit.h"
#include "kea_internal.h"

namespace kea {

thread_local std::string g_last_error;

int fail(int code, const std::string &message) {
    g_last_error = message;
    return code;
}

}  // namespace kea

namespace {

using namespace kea;

// Split-K finish: slices [S][P][M][N] summed in slice order (exact int32), then the epilogue of 4 columns.
template <int P>
__global__ void __launch_bounds__(256) finish_kernel(Params p, int S) {
    const int groups = (p.N + 3) >> 2;
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long long)p.M * groups) return;
    const int m = (int)(idx / groups), nb = (int)(idx % groups) * 4;
    int a[P][4];
#pragma unroll
    for (int c = 0; c < P; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) a[c][r] = 0;
    // Slices are read in batches of up to 8 whose loads are all issued before any is summed (one memory latency per
    // batch instead of one per slice); the sum itself runs in slice order.
    const long long plane = (long long)p.M * p.N;
    const int32_t *base = p.slices + (long long)m * p.N + nb;
    const bool vec = p.slice_vec && nb + 3 < p.N;
    for (int z0 = 0; z0 < S; z0 += 8) {
        int4 v[8][P];
#pragma unroll
        for (int z = 0; z < 8; ++z)
#pragma unroll
            for (int c = 0; c < P; ++c) {
                v[z][c] = make_int4(0, 0, 0, 0);
                if (z0 + z < S) {
                    const int32_t *src = base + ((long long)(z0 + z) * P + c) * plane;
                    if (vec) {
                        v[z][c] = *(const int4 *)src;
                    } else {
                        v[z][c].x = src[0];
                        if (nb + 1 < p.N) v[z][c].y = src[1];
                        if (nb + 2 < p.N) v[z][c].z = src[2];
                        if (nb + 3 < p.N) v[z][c].w = src[3];
                    }
                }
            }
#pragma unroll
        for (int z = 0; z < 8; ++z)
#pragma unroll
            for (int c = 0; c < P; ++c) {
                a[c][0] += v[z][c].x; a[c][1] += v[z][c].y; a[c][2] += v[z][c].z; a[c][3] += v[z][c].w;
            }
    }
    EpiOperands e;
    load_row_scales<P>(p, m, e);
    load_col_scales(p, nb, e);
    load_residual(p, m, nb, e.res);
    epilogue4<P>(p, m, nb, a, e);
}

// ---------------------------------------------------------------------------------------------------------------
// Host side: tile table, validation, launch.

inline long long cdivl(long long a, long long b) { return (a + b - 1) / b; }

KernelFn pick_group(int wbits, int parts, int gq, int id, bool ktail) {
    return wbits == 1 ? ring_pick_w1(parts, id, false, ktail, gq) : ring_pick_w2(parts, id, false, ktail, gq);
}

KernelFn pick_kernel(int wbits, int parts, int id, bool sliced, bool ktail) {
    return wbits == 1 ? ring_pick_w1(parts, id, sliced, ktail, 0) : ring_pick_w2(parts, id, sliced, ktail, 0);
}

using FinishFn = void (*)(Params, int);
FinishFn pick_finish(int parts) {
    if (parts == 1) return finish_kernel<1>;
    if (parts == 2) return finish_kernel<2>;
    return finish_kernel<3>;
}

// The LDS-ring tile for shapes the measured table cannot serve (see choose_tile): small M wants many workgroups (the
// 16x64 tile at P >= 2, 32x32 at P = 1); as M grows the activation tile, re-read once per column tile, bounds a CU,
// so the winners widen in N.
int ring_tile(int parts, long long m, long long n) {
    if (parts >= 3) {
        if (m >= 850) return n >= 4096 ? 10 : 12;
        if (n <= 1024) return 1;
        if (m < 320) return (n >= 4096 && m >= 192) ? 12 : 1;
        if (m < 450) return n >= 3072 ? 3 : 1;
        if (n >= 4096) return 12;
        return (n >= 3072 || m >= 600) ? 3 : 12;
    }
    if (parts == 2) {
        if (m >= 850 && n >= 4096) return 10;
        if (m >= 192 && m < 320 && n >= 4096) return 12;
        return (m >= 512 && n >= 2048) ? 9 : (m >= 320 && n >= 3072) ? 3 : 1;
    }
    if (m <= 64) return 4;
    if (m < 512) return ((n >= 4096 && m >= 192) || (n >= 3072 && m >= 320)) ? 2 : 4;
    if (m < 850) return n <= 1024 ? 4 : n >= 4096 ? 5 : m < 600 ? 2 : 5;
    return n <= 1024 ? 2 : n >= 4096 ? 11 : 5;
}

// Tile choice: a pure function of (wbits, parts, m, n, k) read from the table measured on MI355X (kea_gemm_table.h:
// the fastest tile of every swept shape). Rows of the same weight width, part count, N and K give the tile of the
// nearest swept M in log scale; other shapes take the nearest entry of the same width and part count in
// (log M, log N, log K), K and N weighted above M.
int choose_tile(int wbits, int parts, long long m, long long n, long long k) {
    struct Logs {
        float m[kTileTableSize], n[kTileTableSize], k[kTileTableSize];
        Logs() {
            for (int i = 0; i < kTileTableSize; ++i) {
                m[i] = std::log2((float)kTileTable[i].m);
                n[i] = std::log2((float)kTileTable[i].n);
                k[i] = std::log2((float)kTileTable[i].k);
            }
        }
    };
    static const Logs logs;  // built once (thread-safe static initialisation)
    const float lm = std::log2((float)std::max(1LL, m)), ln = std::log2((float)n), lk = std::log2((float)k);
    int best = 0;
    float best_d = 1e30f;
    for (int i = 0; i < kTileTableSize; ++i) {
        const TileChoice &e = kTileTable[i];
        if (e.wbits != wbits || e.parts != parts) continue;
        const float dm = lm - logs.m[i], dn = ln - logs.n[i], dk = lk - logs.k[i];
        const float d = (e.n == n && e.k == k) ? std::fabs(dm) : 1e6f + dm * dm + 4.f * dn * dn + 4.f * dk * dk;
        if (d < best_d) {
            best_d = d;
            best = e.tile;
        }
    }
    return best ? best : ring_tile(parts, m, n);
}

// The tile for per-group weight scales where the per-channel choice is a wave-split tile (small M; at M = 1000 the
// ring's group tile wins: 20.3 against 24.9 us at N = 1024, K = 4096): the first wave-split tile of a measured
// preference order that takes groups at this K (kea::wsplit_group_steps), else the LDS-ring group tile. The order puts
// first the tiles whose every thread folds one output of the tile (the group fold is one FP32 chain per output):
// config 2 with group-128 scales took 5.2-5.5 us on 16x32 k/8, 6.5-7.0 on 16x16 k/4 and k/8, 6.3 on 16x32 k/4 and
// 7.2-8.9 on the 64-column tiles, against 11.1 us on the ring's best group tile.
int group_tile(int wbits, int parts, long long k, int gq) {
    static const char *const order[] = {"16x32 k/8", "16x16 k/4", "16x16 k/8", "16x32 k/4", "16x64 k/8", "16x64 k/4"};
    for (const char *name : order)
        for (int i = 0; i < kNumWsplitTiles; ++i)
            if (std::string(kWsplitTiles[i].name) == name && kea::wsplit_group_steps(wbits, parts, k, kWsplitTiles[i], gq))
                return kNumTiles + 1 + i;
    return parts >= 2 ? 1 : 4;
}

// Split factor for split_k == 0: split K only for long K ranges (>= 2048) whose tiling leaves at most 64 workgroups,
// by powers of two up to 8 slices and 256 workgroups (ternary, one part, K >= 4096: up to 128 workgroups, 512 after
// the split); the split's second launch costs more than it saves otherwise.
int choose_split(int wbits, int parts, long long m, long long n, long long k, int id) {
    if (id > kNumTiles) return 1;  // wave-split tiles split K inside the workgroup; more only when K needs it
    const Tile &t = kTiles[id - 1];
    const long long bm = t.wm * t.rm * 16, bn = t.wn * t.rn * 16;
    const long long wgs = cdivl(m, bm) * cdivl(n, bn);
    const long long J = wbits == 1 ? cdivl(k, 128) : cdivl(k, 64);
    const long long quads = cdivl(J, 4);
    // Ternary weights at one part and K >= 4096 carry twice the weight bytes per k: there four slices of a
    // 128-workgroup tiling still pay (config 2: 8.1 -> 7.7 us); elsewhere a tiling above 64 workgroups runs unsplit.
    const bool wide = wbits == 2 && parts == 1 && k >= 4096 && wgs <= 128;
    if (k < 2048 || (wgs > 64 && !wide)) return 1;
    const long long cap = wide ? 512 : 256;
    long long s = 1;
    while (s * 2 <= std::min<long long>(8, quads) && wgs * s * 2 <= cap) s *= 2;
    return (int)s;
}

}  // namespace

extern "C" {

const char *kea_last_error(void) { return kea::g_last_error.c_str(); }

int kea_version(void) { return 100; }

int kea_config_count(void) { return kNumTiles + kNumWsplitTiles; }

const char *kea_config_name(int config) {
    if (config < 1 || config > kNumTiles + kNumWsplitTiles) return "";
    return config <= kNumTiles ? kTiles[config - 1].name : kWsplitTiles[config - kNumTiles - 1].name;
}

static int resolve(int wbits, int parts, int64_t m, int64_t n, int64_t k, int split_k, int config, int *tile,
                   int *split, int *qps) {
    if (wbits != 1 && wbits != 2) return kea::fail(KEA_EINVAL, "wbits must be 1 or 2");
    if (parts < 1 || parts > 3) return kea::fail(KEA_EINVAL, "parts must be 1, 2 or 3");
    if (m < 0 || n < 1 || k < 1 || m > INT32_MAX || n > INT32_MAX || k > INT32_MAX)
        return kea::fail(KEA_EINVAL, "bad sizes");
    if (config < 0 || config > kNumTiles + kNumWsplitTiles) return kea::fail(KEA_EINVAL, "unknown config id");
    if (split_k < 0) return kea::fail(KEA_EINVAL, "split_k must be >= 0");
    int id = config ? config : choose_tile(wbits, parts, m, n, k);
    if (!config && id > kNumTiles) {
        // an automatic wave-split pick must fit its registers and LDS, run unsplit when K % 16 != 0, and honour a
        // requested split exactly (the K range of one of its workgroups is at least nw * 2 k-steps)
        const WsplitTile &wt = kWsplitTiles[id - kNumTiles - 1];
        const long long ksteps = cdivl(k, 64), want = split_k > 1 ? split_k : 1;
        const int s = kea::wsplit_steps(wbits, cdivl(ksteps, want), wt.nw);
        const bool ok = s && kea::wsplit_fits(wbits, parts, wt, s) && (!(k & 15) || s * wt.nw * 64 >= k) &&
                        (split_k <= 1 || cdivl(ksteps, (long long)wt.nw * s) == split_k);
        if (!ok) id = ring_tile(parts, m, n);
    }
    if (id > kNumTiles) {
        // wave-split tile: a workgroup covers nw waves x s k-steps; the split is raised to what the K range needs
        const WsplitTile &wt = kWsplitTiles[id - kNumTiles - 1];
        const long long ksteps = cdivl(k, 64);
        long long want = split_k ? split_k : choose_split(wbits, parts, m, n, k, id);
        if (k & 15) want = 1;  // byte-precise K masking runs unsplit
        want = std::max(1LL, std::min(want, ksteps));
        int s = kea::wsplit_steps(wbits, cdivl(ksteps, want), wt.nw);
        while (!s) s = kea::wsplit_steps(wbits, cdivl(ksteps, ++want), wt.nw);
        if (!kea::wsplit_fits(wbits, parts, wt, s))
            return kea::fail(KEA_EINVAL, std::string("wave-split tile ") + wt.name + " does not fit " +
                                             std::to_string(parts) + " activation parts at this K");
        const long long per = (long long)wt.nw * s;  // k-steps per workgroup
        int splits = (int)cdivl(ksteps, per);
        if ((k & 15) && splits > 1)
            return kea::fail(KEA_EINVAL, "K % 16 != 0 needs an unsplit K range: use a larger wave-split tile");
        *tile = id;
        *split = splits;
        *qps = (int)per;
        return KEA_OK;
    }
    const Tile &tl = kTiles[id - 1];
    if (!tile_fits(wbits, parts, tl.rm, tl.rn, tl.wm, tl.wn, tl.pw))
        return kea::fail(KEA_EINVAL, std::string("tile ") + kTiles[id - 1].name + " does not fit " +
                                         std::to_string(parts) + " activation parts");
    const long long J = wbits == 1 ? cdivl(k, 128) : cdivl(k, 64);
    const long long quads = cdivl(J, 4);
    int s = split_k ? split_k : choose_split(wbits, parts, m, n, k, id);
    if (k & 15) {  // byte-precise K masking exists for one unsplit tile only
        id = kTailTile;
        s = 1;
    }
    if (s > quads) s = (int)quads;
    if (s < 1) s = 1;
    const int per = (int)cdivl(quads, s);
    s = (int)cdivl(quads, per);  // no empty slices
    *tile = id;
    *split = s;
    *qps = per;
    return KEA_OK;
}

int64_t kea_lowbit_gemm_workspace(int wbits, int parts, int64_t m, int64_t n, int64_t k, int64_t ws_group,
                                  int split_k, int config) {
    int tile, s, qps;
    if (ws_group) split_k = 1;
    if (resolve(wbits, parts, m, n, k, split_k, config, &tile, &s, &qps) != KEA_OK) return -1;
    return s > 1 ? (int64_t)s * parts * m * n * 4 : 0;
}

int kea_lowbit_gemm_tile(int wbits, int parts, int64_t m, int64_t n, int64_t k) {
    int tile, s, qps;
    if (resolve(wbits, parts, m, n, k, 1, 0, &tile, &s, &qps) != KEA_OK) return -1;
    return tile;
}

int kea_lowbit_gemm_split(int wbits, int parts, int64_t m, int64_t n, int64_t k, int64_t ws_group, int config) {
    int tile, s, qps;
    if (ws_group) return 1;
    if (resolve(wbits, parts, m, n, k, 0, config, &tile, &s, &qps) != KEA_OK) return -1;
    return s;
}

}  // extern "C"

namespace {

// A validated GEMM launch, resolved once (tile, split, kernel instance, grid, LDS) and enqueued any number of times.
struct LaunchSpec {
    Params p;
    bool empty;          // m == 0: nothing to launch
    bool wsplit;         // the wave-split kernel (else the LDS-ring kernel)
    WsplitLaunch wl;
    KernelFn ring_fn;
    dim3 grid, block;
    int lds_bytes;
    int splits, parts;   // splits > 1: a finish launch follows
    dim3 finish_grid;
};

int gemm_prepare(int wbits, const int8_t *q, int64_t part_stride, int64_t ldq, int parts, const void *qs, int qs_dtype,
                 int64_t qs_stride, const uint32_t *w, int64_t n, int64_t k, const void *wscale, int ws_dtype,
                 int64_t ws_group, const void *bias, int bias_dtype, void *y, int y_dtype, int64_t ldy,
                 int32_t *acc_out, int64_t acc_ld, int64_t m, int flags, int split_k, int config, void *workspace,
                 int64_t workspace_bytes, const float *residual, int64_t ldr, float factor, LaunchSpec *ls) {
    int tile, s, qps, gq = 0;
    *ls = LaunchSpec{};
    if (ws_group != 0) {
        if (ws_group != 64 && ws_group != 128 && ws_group != 256)
            return kea::fail(KEA_EINVAL, "ws_group must be 0 (per-channel scales), 64, 128 or 256");
        if (config != 0 && config != 1 && config != 4 && config <= kNumTiles)
            return kea::fail(KEA_EINVAL, "per-group weight scales run tile configs 1 and 4 or a wave-split tile");
        if (split_k > 1) return kea::fail(KEA_EINVAL, "per-group weight scales run unsplit (split_k 0 or 1)");
        gq = (int)(ws_group / 64);
        if (config > kNumTiles && config <= kNumTiles + kNumWsplitTiles &&
            !kea::wsplit_group_steps(wbits, parts, k, kWsplitTiles[config - kNumTiles - 1], gq))
            return kea::fail(KEA_EINVAL, std::string("per-group weight scales on wave-split tile ") +
                                             kWsplitTiles[config - kNumTiles - 1].name +
                                             " need 16-row blocks, at most 64 columns and one workgroup covering K "
                                             "exactly (K = waves x 64 x 2..16, whole groups per wave)");
        if (!config) config = choose_tile(wbits, parts, m, n, k) > kNumTiles ? group_tile(wbits, parts, k, gq)
                                                                             : parts >= 2 ? 1 : 4;
        split_k = 1;
    }
    int rc = resolve(wbits, parts, m, n, k, split_k, config, &tile, &s, &qps);
    if (rc != KEA_OK) return rc;
    if (flags & ~(KEA_FLAG_SILU | KEA_FLAG_ORDER | KEA_FLAG_GLU)) return kea::fail(KEA_EINVAL, "unknown flags");
    const bool glu = (flags & KEA_FLAG_GLU) != 0;
    if (glu && ((flags & KEA_FLAG_SILU) || ws_group || residual || (n & 1)))
        return kea::fail(KEA_EINVAL, "GLU pairs need an even n, per-channel scales, no SiLU and no residual");
    if (m > 0 && (!w || !qs || !wscale)) return kea::fail(KEA_EINVAL, "q, qs, w and wscale are required");
    if (m > 0 && !y && !acc_out) return kea::fail(KEA_EINVAL, "nothing to write: y and acc_out are both NULL");
    if (qs_dtype != KEA_F32 && qs_dtype != KEA_F16) return kea::fail(KEA_EINVAL, "qs dtype must be f32 or f16");
    if (ws_dtype != KEA_F32 && ws_dtype != KEA_F16) return kea::fail(KEA_EINVAL, "wscale dtype must be f32 or f16");
    if (bias && bias_dtype != KEA_F32 && bias_dtype != KEA_F16) return kea::fail(KEA_EINVAL, "bias dtype must be f32 or f16");
    if (y && y_dtype != KEA_F32 && y_dtype != KEA_F16 && y_dtype != KEA_BF16)
        return kea::fail(KEA_EINVAL, "y dtype must be f32, f16 or bf16");
    if (y && ldy < (glu ? n / 2 : n)) return kea::fail(KEA_EINVAL, glu ? "ldy < n / 2" : "ldy < n");
    if (acc_out && acc_ld < n) return kea::fail(KEA_EINVAL, "acc_ld < n");
    if (residual && !y) return kea::fail(KEA_EINVAL, "a residual needs y");
    if (residual && ldr < n) return kea::fail(KEA_EINVAL, "ldr < n");
    if (m == 0) {
        ls->empty = true;
        return KEA_OK;
    }
    if (!q) return kea::fail(KEA_EINVAL, "q is required");
    if (ldq < k) return kea::fail(KEA_EINVAL, "ldq < k");
    if (parts > 1 && part_stride < m * ldq) return kea::fail(KEA_EINVAL, "part_stride < m * ldq (parts overlap)");
    if (((uintptr_t)q & 15) || (ldq & 15) || (parts > 1 && (part_stride & 15)))
        return kea::fail(KEA_EALIGN, "q needs 16-byte aligned rows: q % 16 == 0, ldq % 16 == 0, part_stride % 16 == 0");
    if ((uintptr_t)w & 15) return kea::fail(KEA_EALIGN, "weight words must be 16-byte aligned");
    const auto misaligned = [](const void *v, int dtype) { return ((uintptr_t)v & (dtype == KEA_F32 ? 3 : 1)) != 0; };
    if (misaligned(qs, qs_dtype) || misaligned(wscale, ws_dtype) || (bias && misaligned(bias, bias_dtype)))
        return kea::fail(KEA_EALIGN, "qs, wscale and bias must be aligned to their element size");
    if ((int64_t)(parts - 1) * part_stride + m * ldq > (int64_t)INT32_MAX)
        return kea::fail(KEA_EINVAL, "q spans more than 2 GiB: split the call along M");
    // the epilogues address the per-column vectors (scales, bias) with 32-bit byte offsets
    if (n >= (int64_t(1) << 30)) return kea::fail(KEA_EINVAL, "too large for one launch: split the call along N");

    Params &p = ls->p;
    p.q = q; p.part_stride = part_stride; p.ldq = ldq;
    p.qs = qs; p.qs_stride = qs_stride; p.qs_dtype = qs_dtype;
    p.w = w; p.ws = wscale; p.ws_dtype = ws_dtype;
    p.bias = bias; p.bias_dtype = bias_dtype;
    p.y = y; p.ldy = ldy; p.y_dtype = y_dtype;
    p.acc = acc_out; p.acc_ld = acc_ld;
    p.res = residual; p.ldr = ldr; p.res_factor = factor;
    p.M = (int)m; p.N = (int)n; p.K = (int)k;
    p.J = (int)(wbits == 1 ? cdivl(k, 128) : cdivl(k, 64));
    p.NT = (int)cdivl(n, 16);
    p.quads_per_slice = qps;
    p.flags = flags;
    const int esz = (y_dtype == KEA_F32) ? 4 : 2;
    const int yv = glu ? 2 : 4;  // elements per vector store
    p.y_vec = y && (ldy % yv == 0) && ((uintptr_t)y % (yv * esz) == 0);
    p.acc_vec = acc_out && (acc_ld % 4 == 0) && ((uintptr_t)acc_out % 16 == 0);
    ls->splits = s;
    ls->parts = parts;
    if (s > 1) {
        const int64_t need = (int64_t)s * parts * m * n * 4;
        if (!workspace || workspace_bytes < need)
            return kea::fail(KEA_ESPACE, "split-K workspace too small: need " + std::to_string(need) + " bytes");
        if ((uintptr_t)workspace & 15) return kea::fail(KEA_EALIGN, "workspace must be 16-byte aligned");
        if (!kea::fits_dispatch(cdivl(m * cdivl(n, 4), 256), 256))
            return kea::fail(KEA_EINVAL, "too large for one launch: split the call along N or M");
        p.slices = (int32_t *)workspace;
        p.slice_vec = (n % 4 == 0);
        ls->finish_grid = dim3((unsigned)cdivl(m * cdivl(n, 4), 256));
    }

    if (tile > kNumTiles) {
        const WsplitTile &wt = kWsplitTiles[tile - kNumTiles - 1];
        if (!kea::fits_dispatch(cdivl(n, wt.nt * 16), wt.nw * 64))
            return kea::fail(KEA_EINVAL, "too large for one launch: split the call along N or M");
        if (gq) {
            const int gs = kea::wsplit_group_steps(wbits, parts, k, wt, gq);
            p.groups = (int)cdivl(k, ws_group);
            p.steps_per_slice = wt.nw * gs;
            const hipError_t e = gs ? kea::wsplit_group_prepare(p, wbits, parts, tile - kNumTiles - 1, gq, gs, &ls->wl)
                                    : hipErrorInvalidDeviceFunction;
            if (e != hipSuccess)
                return kea::fail((int)e, std::string("no per-group wave-split kernel: ") + hipGetErrorString(e));
            ls->wsplit = true;
            ls->splits = 1;
            return KEA_OK;
        }
        p.steps_per_slice = qps;
        const hipError_t e = kea::wsplit_prepare(p, wbits, parts, tile - kNumTiles - 1, qps / wt.nw, s, s > 1, &ls->wl);
        if (e != hipSuccess) return kea::fail((int)e, std::string("no wave-split kernel: ") + hipGetErrorString(e));
        ls->wsplit = true;
        return KEA_OK;
    }
    const Tile &t = kTiles[tile - 1];
    const int bm = t.wm * t.rm * 16, bn = t.wn * t.rn * 16;
    // Ring buffers actually used: a workgroup touches buffer s % NS for its stages s < nst, so with nst < NS only
    // the first nst buffers need LDS.
    const long long words_per_wg = std::min<long long>(4LL * qps, (long long)p.J);
    const StageShape shape = stage_shape(wbits, parts, t.rm, t.rn, t.wm, t.wn, t.pw);
    const int nst = (int)cdivl(words_per_wg, shape.sw);
    int lds_bytes = std::min(shape.ns, nst) * shape.stage_bytes;
    if (gq) {
        // alpha block: the groups the stages span (KEA_STAGE_K / 64 k-steps per stage), padded to a power of two
        const int spanned = nst * (KEA_STAGE_K / 64) / gq;
        int shift = 0;
        while ((1 << shift) < spanned) ++shift;
        p.groups = (int)cdivl(k, ws_group);
        p.gp_shift = shift;
        lds_bytes += (1 << shift) * (bn + 4) * 4;
        if (lds_bytes > kLdsBudget)
            return kea::fail(KEA_EINVAL, "too many weight-scale groups for one workgroup's LDS: use a larger ws_group");
    }
    if (!kea::fits_dispatch(cdivl(n, bn), (t.wm * t.wn + t.pw) * 64))
        return kea::fail(KEA_EINVAL, "too large for one launch: split the call along N or M");
    ls->grid = dim3((unsigned)cdivl(n, bn), (unsigned)cdivl(m, bm), (unsigned)s);
    ls->block = dim3((t.wm * t.wn + t.pw) * 64);
    ls->ring_fn = gq ? pick_group(wbits, parts, gq, tile, (k & 15) != 0)
                     : pick_kernel(wbits, parts, tile, s > 1, (k & 15) != 0);
    if (!ls->ring_fn) return kea::fail(KEA_EINVAL, "no kernel instance for this tile");
    if (lds_bytes > 65536) {
        hipError_t e = hipFuncSetAttribute((const void *)ls->ring_fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           lds_bytes);
        if (e != hipSuccess) return kea::fail((int)e, std::string("LDS attribute refused: ") + hipGetErrorString(e));
    }
    ls->lds_bytes = lds_bytes;
    return KEA_OK;
}

int gemm_launch(const LaunchSpec &ls, hipStream_t st) {
    if (ls.empty) return KEA_OK;
    hipError_t e;
    if (ls.wsplit) {
        e = kea::wsplit_enqueue(ls.wl, ls.p, st);
    } else {
        hipLaunchKernelGGL(ls.ring_fn, ls.grid, ls.block, ls.lds_bytes, st, ls.p);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return kea::fail((int)e, std::string("gemm launch failed: ") + hipGetErrorString(e));
    if (ls.splits > 1) {
        hipLaunchKernelGGL(pick_finish(ls.parts), ls.finish_grid, dim3(256), 0, st, ls.p, ls.splits);
        e = hipGetLastError();
        if (e != hipSuccess) return kea::fail((int)e, std::string("finish launch failed: ") + hipGetErrorString(e));
    }
    return KEA_OK;
}

int gemm_impl(int wbits, const int8_t *q, int64_t part_stride, int64_t ldq, int parts, const void *qs, int qs_dtype,
              int64_t qs_stride, const uint32_t *w, int64_t n, int64_t k, const void *wscale, int ws_dtype,
              int64_t ws_group, const void *bias, int bias_dtype, void *y, int y_dtype, int64_t ldy, int32_t *acc_out,
              int64_t acc_ld, int64_t m, int flags, int split_k, int config, void *workspace, int64_t workspace_bytes,
              const float *residual, int64_t ldr, float factor, void *stream) {
    LaunchSpec ls;
    const int rc = gemm_prepare(wbits, q, part_stride, ldq, parts, qs, qs_dtype, qs_stride, w, n, k, wscale, ws_dtype,
                                ws_group, bias, bias_dtype, y, y_dtype, ldy, acc_out, acc_ld, m, flags, split_k,
                                config, workspace, workspace_bytes, residual, ldr, factor, &ls);
    if (rc != KEA_OK) return rc;
    return gemm_launch(ls, (hipStream_t)stream);
}

}  // namespace

struct kea_gemm_plan {
    LaunchSpec spec;
};

// A quantizer launch followed by a plan's GEMM on the parts it wrote: the quantizer's arguments and the byte offsets
// of the scales and the split-K slices in the caller's workspace (the int8 parts start at its first byte).
struct kea_project_plan {
    LaunchSpec spec;
    int x_dtype, silu;
    int64_t xb, xt, xk, t;
    const float *norm_w, *norm_b;
    float eps;
    int64_t qs_off, slices_off, need;
};

namespace {

// Points a plan's copy at new outputs; the vector-store flags follow their alignment (the row strides are the plan's).
void bind_outputs(Params &p, void *y, int32_t *acc_out) {
    p.y = y;
    p.acc = acc_out;
    const int esz = p.y_dtype == KEA_F32 ? 4 : 2, yv = (p.flags & KEA_FLAG_GLU) ? 2 : 4;
    p.y_vec = y && (p.ldy % yv == 0) && ((uintptr_t)y % (yv * esz) == 0);
    p.acc_vec = acc_out && (p.acc_ld % 4 == 0) && ((uintptr_t)acc_out % 16 == 0);
}

int64_t round16(int64_t v) { return (v + 15) & ~(int64_t)15; }

}  // namespace

extern "C" {

kea_gemm_plan *kea_lowbit_gemm_plan(int wbits, const int8_t *q, int64_t part_stride, int64_t ldq, int parts,
                                    const void *qs, int qs_dtype, int64_t qs_stride, const uint32_t *w, int64_t n,
                                    int64_t k, const void *wscale, int ws_dtype, int64_t ws_group, const void *bias,
                                    int bias_dtype, void *y, int y_dtype, int64_t ldy, int32_t *acc_out,
                                    int64_t acc_ld, int64_t m, int flags, int split_k, int config, void *workspace,
                                    int64_t workspace_bytes, const float *residual, int64_t ldr, float factor) {
    kea_gemm_plan *plan = new (std::nothrow) kea_gemm_plan;
    if (!plan) {
        kea::fail(KEA_EINVAL, "out of host memory for a plan");
        return nullptr;
    }
    const int rc = gemm_prepare(wbits, q, part_stride, ldq, parts, qs, qs_dtype, qs_stride, w, n, k, wscale, ws_dtype,
                                ws_group, bias, bias_dtype, y, y_dtype, ldy, acc_out, acc_ld, m, flags, split_k,
                                config, workspace, workspace_bytes, residual, ldr, factor, &plan->spec);
    if (rc != KEA_OK) {
        delete plan;
        return nullptr;
    }
    return plan;
}

int kea_lowbit_gemm_plan_launch(const kea_gemm_plan *plan, void *stream) {
    if (!plan) return kea::fail(KEA_EINVAL, "plan is NULL");
    return gemm_launch(plan->spec, (hipStream_t)stream);
}

int kea_lowbit_gemm_plan_launch_with(const kea_gemm_plan *plan, const int8_t *q, const void *qs, void *y,
                                     int32_t *acc_out, const float *residual, void *workspace,
                                     int64_t workspace_bytes, void *stream) {
    if (!plan) return kea::fail(KEA_EINVAL, "plan is NULL");
    if (plan->spec.empty) return KEA_OK;
    LaunchSpec ls = plan->spec;  // a copy: the plan stays read-only, so concurrent launches of it are safe
    Params &p = ls.p;
    if (!q || ((uintptr_t)q & 15)) return kea::fail(KEA_EALIGN, "q must be a 16-byte aligned device pointer");
    if (!qs) return kea::fail(KEA_EINVAL, "qs is required");
    if ((uintptr_t)qs & (p.qs_dtype == KEA_F32 ? 3 : 1))
        return kea::fail(KEA_EALIGN, "qs must be aligned to its element size");
    if ((y != nullptr) != (p.y != nullptr) || (acc_out != nullptr) != (p.acc != nullptr) ||
        (residual != nullptr) != (p.res != nullptr))
        return kea::fail(KEA_EINVAL, "y, acc_out and residual must be given exactly where the plan has them");
    p.q = q;
    p.qs = qs;
    p.res = residual;
    bind_outputs(p, y, acc_out);
    if (ls.splits > 1) {
        const int64_t need = (int64_t)ls.splits * ls.parts * p.M * p.N * 4;
        if (!workspace || workspace_bytes < need)
            return kea::fail(KEA_ESPACE, "split-K workspace too small: need " + std::to_string(need) + " bytes");
        if ((uintptr_t)workspace & 15) return kea::fail(KEA_EALIGN, "workspace must be 16-byte aligned");
        p.slices = (int32_t *)workspace;
    }
    return gemm_launch(ls, (hipStream_t)stream);
}

int64_t kea_lowbit_gemm_plan_workspace(const kea_gemm_plan *plan) {
    if (!plan || plan->spec.empty || plan->spec.splits <= 1) return 0;
    return (int64_t)plan->spec.splits * plan->spec.parts * plan->spec.p.M * plan->spec.p.N * 4;
}

void kea_lowbit_gemm_plan_free(kea_gemm_plan *plan) { delete plan; }

kea_project_plan *kea_lowbit_project_plan(const kea_gemm_plan *plan, int x_dtype, int64_t xb, int64_t xt, int64_t xk,
                                          int64_t t, const float *norm_w, const float *norm_b, float eps,
                                          int input_silu) {
    if (!plan) {
        kea::fail(KEA_EINVAL, "plan is NULL");
        return nullptr;
    }
    const LaunchSpec &ls = plan->spec;
    const Params &p = ls.p;
    if (ls.empty) {
        kea::fail(KEA_EINVAL, "a projection plan needs at least one row");
        return nullptr;
    }
    if (!p.y || p.acc || p.res) {
        kea::fail(KEA_EINVAL, "a projection plan's GEMM writes y only (no acc_out, no residual)");
        return nullptr;
    }
    if (p.part_stride != (long long)p.M * p.ldq || p.qs_stride != p.M) {
        kea::fail(KEA_EINVAL, "a projection plan's GEMM reads the quantizer's layout: part_stride = m * ldq and "
                              "qs_stride = m");
        return nullptr;
    }
    if (kea::quantize_check(x_dtype, t, p.M, p.K, ls.parts, p.ldq, p.qs_dtype, norm_w, norm_b) != KEA_OK)
        return nullptr;
    kea_project_plan *pp = new (std::nothrow) kea_project_plan;
    if (!pp) {
        kea::fail(KEA_EINVAL, "out of host memory for a plan");
        return nullptr;
    }
    pp->spec = ls;
    pp->x_dtype = x_dtype;
    pp->silu = input_silu;
    pp->xb = xb;
    pp->xt = xt;
    pp->xk = xk;
    pp->t = t;
    pp->norm_w = norm_w;
    pp->norm_b = norm_b;
    pp->eps = eps;
    const int64_t qbytes = (int64_t)ls.parts * p.M * p.ldq;
    const int qs_esz = p.qs_dtype == KEA_F32 ? 4 : 2;
    pp->qs_off = round16(qbytes);
    pp->slices_off = round16(pp->qs_off + (int64_t)ls.parts * p.M * qs_esz);
    pp->need = ls.splits > 1 ? pp->slices_off + (int64_t)ls.splits * ls.parts * p.M * p.N * 4 : pp->slices_off;
    return pp;
}

int64_t kea_lowbit_project_workspace(const kea_project_plan *pp) { return pp ? pp->need : 0; }

int kea_lowbit_project_launch(const kea_project_plan *pp, const void *x, void *y, void *workspace,
                              int64_t workspace_bytes, void *stream) {
    if (!pp) return kea::fail(KEA_EINVAL, "plan is NULL");
    if (!x || !y) return kea::fail(KEA_EINVAL, "x and y are required");
    if (!workspace || workspace_bytes < pp->need)
        return kea::fail(KEA_ESPACE, "projection workspace too small: need " + std::to_string(pp->need) + " bytes");
    if ((uintptr_t)workspace & 15) return kea::fail(KEA_EALIGN, "workspace must be 16-byte aligned");
    LaunchSpec ls = pp->spec;  // a copy: the plan stays read-only, so concurrent launches of it are safe
    Params &p = ls.p;
    uint8_t *ws = (uint8_t *)workspace;
    int rc = kea::quantize_enqueue(x, pp->x_dtype, pp->xb, pp->xt, pp->xk, pp->t, p.M, p.K, ls.parts, pp->norm_w,
                                   pp->norm_b, pp->eps, pp->silu, (int8_t *)ws, p.ldq, ws + pp->qs_off, p.qs_dtype,
                                   stream);
    if (rc != KEA_OK) return rc;
    p.q = (const int8_t *)ws;
    p.qs = ws + pp->qs_off;
    bind_outputs(p, y, nullptr);
    if (ls.splits > 1) p.slices = (int32_t *)(ws + pp->slices_off);
    return gemm_launch(ls, (hipStream_t)stream);
}

void kea_lowbit_project_plan_free(kea_project_plan *pp) { delete pp; }

int kea_lowbit_gemm(int wbits, const int8_t *q, int64_t part_stride, int64_t ldq, int parts, const void *qs,
                    int qs_dtype, int64_t qs_stride, const uint32_t *w, int64_t n, int64_t k, const void *wscale,
                    int ws_dtype, int64_t ws_group, const void *bias, int bias_dtype, void *y, int y_dtype,
                    int64_t ldy, int32_t *acc_out, int64_t acc_ld, int64_t m, int flags, int split_k, int config,
                    void *workspace, int64_t workspace_bytes, void *stream) {
    return gemm_impl(wbits, q, part_stride, ldq, parts, qs, qs_dtype, qs_stride, w, n, k, wscale, ws_dtype, ws_group,
                     bias, bias_dtype, y, y_dtype, ldy, acc_out, acc_ld, m, flags, split_k, config, workspace,
                     workspace_bytes, nullptr, 0, 0.f, stream);
}

// ---- kea_lowbit_gemm_noalloc: split-K slices in a library-owned device array ----

}  // extern "C"

namespace {

constexpr int64_t kScratchInts = KEA_NOALLOC_SCRATCH_BYTES / 4;
// The split-K slices of kea_lowbit_gemm_noalloc: one copy per GPU, held until the process ends. Host code never uses
// this name as an address (it is a host-side stand-in): the device address comes from hipGetSymbolAddress.
static __device__ __align__(256) int32_t scratch[kScratchInts];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void *g_scratch_ptr[kMaxDevices] = {};

// The calling thread's current device's copy of `scratch`, resolved once per device with that device current.
int scratch_for_current_device(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return kea::fail((int)e, std::string("hipGetDevice failed: ") + hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return kea::fail(KEA_ENODEV, "device index out of range for the scratch table");
    std::lock_guard<std::mutex> lock(g_scratch_lock);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return kea::fail(e != hipSuccess ? (int)e : KEA_ENODEV,
                             std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return KEA_OK;
}

}  // namespace

extern "C" {

int kea_lowbit_gemm_noalloc(int wbits, const int8_t *q, int64_t part_stride, int64_t ldq, int parts, const void *qs,
                            int qs_dtype, int64_t qs_stride, const uint32_t *w, int64_t n, int64_t k,
                            const void *wscale, int ws_dtype, int64_t ws_group, const void *bias, int bias_dtype,
                            void *y, int y_dtype, int64_t ldy, int32_t *acc_out, int64_t acc_ld, int64_t m,
                            int flags, int split_k, int config, void *stream) {
    const int64_t need = kea_lowbit_gemm_workspace(wbits, parts, std::max<int64_t>(m, 1), n, k, ws_group, split_k,
                                                   config);
    if (need < 0) return KEA_EINVAL;  // the reason is already in kea_last_error()
    if (need > KEA_NOALLOC_SCRATCH_BYTES)
        return kea::fail(KEA_ESPACE, "kea_lowbit_gemm_noalloc: the split-K slices need " + std::to_string(need) +
                                         " bytes, more than the " + std::to_string(KEA_NOALLOC_SCRATCH_BYTES) +
                                         "-byte scratch array: use kea_lowbit_gemm with a workspace, or a smaller "
                                         "split_k / m");
    void *ws = nullptr;
    if (need > 0) {
        const int rc = scratch_for_current_device(&ws);
        if (rc != KEA_OK) return rc;
    }
    return gemm_impl(wbits, q, part_stride, ldq, parts, qs, qs_dtype, qs_stride, w, n, k, wscale, ws_dtype, ws_group,
                     bias, bias_dtype, y, y_dtype, ldy, acc_out, acc_ld, m, flags, split_k, config, ws,
                     need > 0 ? KEA_NOALLOC_SCRATCH_BYTES : 0, nullptr, 0, 0.f, stream);
}

int kea_lowbit_gemm_residual(int wbits, const int8_t *q, int64_t part_stride, int64_t ldq, int parts, const void *qs,
                             int qs_dtype, int64_t qs_stride, const uint32_t *w, int64_t n, int64_t k,
                             const void *wscale, int ws_dtype, int64_t ws_group, const void *bias, int bias_dtype,
                             void *y, int y_dtype, int64_t ldy, int32_t *acc_out, int64_t acc_ld, int64_t m, int flags,
                             int split_k, int config, void *workspace, int64_t workspace_bytes, const float *residual,
                             int64_t ldr, float factor, void *stream) {
    if (!residual) return kea::fail(KEA_EINVAL, "residual is required");
    return gemm_impl(wbits, q, part_stride, ldq, parts, qs, qs_dtype, qs_stride, w, n, k, wscale, ws_dtype, ws_group,
                     bias, bias_dtype, y, y_dtype, ldy, acc_out, acc_ld, m, flags, split_k, config, workspace,
                     workspace_bytes, residual, ldr, factor, stream);
}

}  // extern "C"

extern "C" {

int kea_lowbit_gemm_slices(int wbits, const int8_t *q, int64_t part_stride, int64_t ldq, int parts,
                           const uint32_t *w, int64_t n, int64_t k, int64_t m, int split, int config,
                           int32_t *slices, void *stream) {
    if (split < 1) return kea::fail(KEA_EINVAL, "split must be >= 1");
    int tile, s, qps;
    int rc = resolve(wbits, parts, m, n, k, split, config, &tile, &s, &qps);
    if (rc != KEA_OK) return rc;
    if (k & 15) return kea::fail(KEA_EINVAL, "deferred slices need k % 16 == 0");
    if (s != split)
        return kea::fail(KEA_EINVAL, "split does not cut the K range into that many non-empty slices (at most " +
                                         std::to_string(s) + ")");
    if (m == 0) return KEA_OK;
    if (!q || !w || !slices) return kea::fail(KEA_EINVAL, "q, w and slices are required");
    if (ldq < k) return kea::fail(KEA_EINVAL, "ldq < k");
    if (parts > 1 && part_stride < m * ldq) return kea::fail(KEA_EINVAL, "part_stride < m * ldq (parts overlap)");
    if (((uintptr_t)q & 15) || (ldq & 15) || (parts > 1 && (part_stride & 15)))
        return kea::fail(KEA_EALIGN, "q needs 16-byte aligned rows");
    if (((uintptr_t)w & 15) || ((uintptr_t)slices & 15)) return kea::fail(KEA_EALIGN, "w and slices must be 16-byte aligned");
    if ((int64_t)(parts - 1) * part_stride + m * ldq > (int64_t)INT32_MAX)
        return kea::fail(KEA_EINVAL, "q spans more than 2 GiB: split the call along M");
    // the epilogues address the per-column vectors (scales, bias) with 32-bit byte offsets
    if (n >= (int64_t(1) << 30)) return kea::fail(KEA_EINVAL, "too large for one launch: split the call along N");
    Params p = {};
    p.q = q; p.part_stride = part_stride; p.ldq = ldq;
    p.w = w;
    p.M = (int)m; p.N = (int)n; p.K = (int)k;
    p.J = (int)(wbits == 1 ? cdivl(k, 128) : cdivl(k, 64));
    p.NT = (int)cdivl(n, 16);
    p.quads_per_slice = qps;
    p.slices = slices;
    p.slice_vec = (n % 4 == 0);
    if (tile > kNumTiles) {
        const WsplitTile &wt = kWsplitTiles[tile - kNumTiles - 1];
        if (!kea::fits_dispatch(cdivl(n, wt.nt * 16), wt.nw * 64))
            return kea::fail(KEA_EINVAL, "too large for one launch: split the call along N");
        p.steps_per_slice = qps;
        WsplitLaunch wl;
        hipError_t e = kea::wsplit_prepare(p, wbits, parts, tile - kNumTiles - 1, qps / wt.nw, s, true, &wl);
        if (e == hipSuccess) e = kea::wsplit_enqueue(wl, p, (hipStream_t)stream);
        if (e != hipSuccess) return kea::fail((int)e, std::string("slice launch failed: ") + hipGetErrorString(e));
        return KEA_OK;
    }
    const Tile &t = kTiles[tile - 1];
    const int bm = t.wm * t.rm * 16, bn = t.wn * t.rn * 16;
    const long long words_per_wg = std::min<long long>(4LL * qps, (long long)p.J);
    const StageShape shape = stage_shape(wbits, parts, t.rm, t.rn, t.wm, t.wn, t.pw);
    const int nst = (int)cdivl(words_per_wg, shape.sw);
    const int lds_bytes = std::min(shape.ns, nst) * shape.stage_bytes;
    if (!kea::fits_dispatch(cdivl(n, bn), (t.wm * t.wn + t.pw) * 64))
        return kea::fail(KEA_EINVAL, "too large for one launch: split the call along N");
    KernelFn fn = pick_kernel(wbits, parts, tile, true, false);
    if (lds_bytes > 65536) {
        hipError_t e = hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
        if (e != hipSuccess) return kea::fail((int)e, std::string("LDS attribute refused: ") + hipGetErrorString(e));
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)cdivl(n, bn), (unsigned)cdivl(m, bm), (unsigned)s),
                       dim3((t.wm * t.wn + t.pw) * 64), lds_bytes, (hipStream_t)stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("slice launch failed: ") + hipGetErrorString(e));
    return KEA_OK;
}

int kea_lowbit_slices_finish(const int32_t *slices, int split, int parts, int64_t m, int64_t n, const void *qs,
                             int qs_dtype, int64_t qs_stride, const void *wscale, int ws_dtype, const void *bias,
                             int bias_dtype, void *y, int y_dtype, int64_t ldy, int32_t *acc_out, int64_t acc_ld,
                             int flags, void *stream) {
    if (split < 1 || parts < 1 || parts > 3 || m < 0 || n < 1 || m > INT32_MAX || n > INT32_MAX)
        return kea::fail(KEA_EINVAL, "bad sizes");
    if (flags & ~(KEA_FLAG_SILU | KEA_FLAG_ORDER)) return kea::fail(KEA_EINVAL, "unknown flags");
    if (qs_dtype != KEA_F32 && qs_dtype != KEA_F16) return kea::fail(KEA_EINVAL, "qs dtype must be f32 or f16");
    if (ws_dtype != KEA_F32 && ws_dtype != KEA_F16) return kea::fail(KEA_EINVAL, "wscale dtype must be f32 or f16");
    if (bias && bias_dtype != KEA_F32 && bias_dtype != KEA_F16) return kea::fail(KEA_EINVAL, "bias dtype must be f32 or f16");
    if (y && y_dtype != KEA_F32 && y_dtype != KEA_F16 && y_dtype != KEA_BF16)
        return kea::fail(KEA_EINVAL, "y dtype must be f32, f16 or bf16");
    if (y && ldy < n) return kea::fail(KEA_EINVAL, "ldy < n");
    if (acc_out && acc_ld < n) return kea::fail(KEA_EINVAL, "acc_ld < n");
    if (m == 0) return KEA_OK;
    if (!slices || !qs || !wscale) return kea::fail(KEA_EINVAL, "slices, qs and wscale are required");
    if (!y && !acc_out) return kea::fail(KEA_EINVAL, "nothing to write: y and acc_out are both NULL");
    if ((uintptr_t)slices & 15) return kea::fail(KEA_EALIGN, "slices must be 16-byte aligned");
    const auto misaligned = [](const void *v, int dtype) { return ((uintptr_t)v & (dtype == KEA_F32 ? 3 : 1)) != 0; };
    if (misaligned(qs, qs_dtype) || misaligned(wscale, ws_dtype) || (bias && misaligned(bias, bias_dtype)))
        return kea::fail(KEA_EALIGN, "qs, wscale and bias must be aligned to their element size");
    // the epilogue addresses the per-column vectors with 32-bit byte offsets
    if (n >= (int64_t(1) << 30)) return kea::fail(KEA_EINVAL, "too large for one launch: split the call along N");
    Params p = {};
    p.qs = qs; p.qs_stride = qs_stride; p.qs_dtype = qs_dtype;
    p.ws = wscale; p.ws_dtype = ws_dtype;
    p.bias = bias; p.bias_dtype = bias_dtype;
    p.y = y; p.ldy = ldy; p.y_dtype = y_dtype;
    p.acc = acc_out; p.acc_ld = acc_ld;
    p.M = (int)m; p.N = (int)n;
    p.flags = flags;
    p.slices = const_cast<int32_t *>(slices);
    p.slice_vec = (n % 4 == 0);
    const int esz = (y_dtype == KEA_F32) ? 4 : 2;
    p.y_vec = y && (ldy % 4 == 0) && ((uintptr_t)y % (4 * esz) == 0);
    p.acc_vec = acc_out && (acc_ld % 4 == 0) && ((uintptr_t)acc_out % 16 == 0);
    const long long work = m * cdivl(n, 4);
    if (!kea::fits_dispatch(cdivl(work, 256), 256))
        return kea::fail(KEA_EINVAL, "too large for one launch: split the call along M");
    hipLaunchKernelGGL(pick_finish(parts), dim3((unsigned)cdivl(work, 256)), dim3(256), 0, (hipStream_t)stream, p, split);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("finish launch failed: ") + hipGetErrorString(e));
    return KEA_OK;
}

}  // extern "C"
