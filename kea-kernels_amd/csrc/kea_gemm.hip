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
#include <cstdint>
#include <cstdio>
#include <string>
#include <type_traits>

#include "kea_epilogue.h"
#include "kea_internal.h"

namespace kea {

thread_local std::string g_last_error;

int fail(int code, const std::string &message) {
    g_last_error = message;
    return code;
}

}  // namespace kea

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

struct Params {
    const int8_t *q;
    long long part_stride, ldq;
    const void *qs;
    long long qs_stride;
    const uint32_t *w;
    const void *ws;
    const void *bias;
    void *y;
    long long ldy;
    int32_t *acc;
    long long acc_ld;
    int32_t *slices;  // split-K partials [S][P][M][N]
    int M, N, K, J;   // J = native words per lane per n-tile
    int NT;           // n-tiles present in the weight buffer
    int quads_per_slice;
    int flags;
    int qs_dtype, ws_dtype, bias_dtype, y_dtype;
    int y_vec;      // 1: y rows allow aligned 4-element vector stores
    int acc_vec;    // 1: acc_out rows allow aligned int4 stores
    int slice_vec;  // 1: the dense [S][P][M][N] slices allow aligned int4 access (N % 4 == 0)
    const float *res;   // optional residual: y = res[m * ldr + n] + value * res_factor (two roundings)
    long long ldr;
    float res_factor;
    int groups;     // per-group scales: G = ceil(K / ws_group) groups, alpha [N][G]
    int gp_shift;   // log2 of the padded group count held in LDS (a power of two >= the groups the stages span)
    int ws_vec, bias_vec;  // 1: per-channel scales / bias allow aligned 4-element vector loads
};

using kea::combine;
using kea::finish;
using kea::kNoBias;
using kea::load_scalar;

// 1-bit: plane (4h + d) of a native word -> four int8 weights. Stored bits are inverted signs, so after the mask
// each selector byte is 0 (weight +1) or 2^(4h+d) (weight -1). The permute table {S0:S1} = {0x000000FF:0x00FFFF01}
// maps selector 0 -> byte 0 = 0x01, 1 -> 0xFF, 2 -> 0xFF, 4 -> byte 4 = 0xFF, 8 -> sign of byte 1 = 0xFF and
// every selector >= 13 -> 0xFF.
template <int PLANE>
__device__ __forceinline__ int b1_expand(uint32_t w) {
    return (int)__builtin_amdgcn_perm(0x000000FFu, 0x00FFFF01u, w & (0x01010101u << PLANE));
}
// 2-bit: codes 00 / 01 / 10 (0, +1, -1) at bits 2d of each byte. Low pair: selectors {0, 1, 2} pick bytes
// {0x00, 0x01, 0xFF} of 0x00FF0100. High pair (mask 0x0C): selectors {0, 4, 8} pick byte 0 = 0x00, byte 4 = 0x01
// and the sign of byte 1 (0x80) = 0xFF.
__device__ __forceinline__ int t2_lo(uint32_t w) {
    return (int)__builtin_amdgcn_perm(0x00000000u, 0x00FF0100u, w & 0x03030303u);
}
__device__ __forceinline__ int t2_hi(uint32_t w) {
    return (int)__builtin_amdgcn_perm(0x00000001u, 0x00008000u, w & 0x0C0C0C0Cu);
}

__device__ __forceinline__ uint16_t to_f16_bits(float v) {
    _Float16 h = (_Float16)v;  // IEEE round to nearest even
    return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ uint16_t to_bf16_bits(float v) {
    __bf16 h = (__bf16)v;  // IEEE round to nearest even
    return __builtin_bit_cast(uint16_t, h);
}

// Stores 4 consecutive outputs y[row][nb .. nb+3] (nb + r < N checked per element unless the vector path applies).
__device__ __forceinline__ void store4(const Params &p, long long off, int nb, const float *v) {
    const bool full = p.y_vec && nb + 3 < p.N;
    if (p.y_dtype == KEA_F32) {
        float *y = (float *)p.y + off;
        if (full) {
            *(float4 *)y = make_float4(v[0], v[1], v[2], v[3]);
        } else {
            for (int r = 0; r < 4; ++r)
                if (nb + r < p.N) y[r] = v[r];
        }
    } else {
        uint16_t h[4];
        for (int r = 0; r < 4; ++r) h[r] = p.y_dtype == KEA_F16 ? to_f16_bits(v[r]) : to_bf16_bits(v[r]);
        uint16_t *y = (uint16_t *)p.y + off;
        if (full) {
            uint2 packed;
            packed.x = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
            packed.y = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
            *(uint2 *)y = packed;
        } else {
            for (int r = 0; r < 4; ++r)
                if (nb + r < p.N) y[r] = h[r];
        }
    }
}

// GLU pairs: u[0..1] = y[row][cb], y[row][cb + 1] (cb = nb / 2; the second only when nb + 3 < N).
__device__ __forceinline__ void store2(const Params &p, long long off, int nb, const float *u) {
    const bool full = p.y_vec && nb + 3 < p.N;
    if (p.y_dtype == KEA_F32) {
        float *y = (float *)p.y + off;
        if (full) {
            *(float2 *)y = make_float2(u[0], u[1]);
        } else {
            y[0] = u[0];
            if (nb + 3 < p.N) y[1] = u[1];
        }
    } else {
        uint16_t h[2];
        for (int r = 0; r < 2; ++r) h[r] = p.y_dtype == KEA_F16 ? to_f16_bits(u[r]) : to_bf16_bits(u[r]);
        uint16_t *y = (uint16_t *)p.y + off;
        if (full) {
            *(uint32_t *)y = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
        } else {
            y[0] = h[0];
            if (nb + 3 < p.N) y[1] = h[1];
        }
    }
}

__device__ __forceinline__ void store_int4(int32_t *dst, bool vec, int nb, int N, const int *v) {
    if (vec && nb + 3 < N) {
        *(int4 *)dst = make_int4(v[0], v[1], v[2], v[3]);
    } else {
        for (int r = 0; r < 4; ++r)
            if (nb + r < N) dst[r] = v[r];
    }
}

// Epilogue operands of one row m and 4 consecutive columns nb..nb+3 (indices clamped into range; the clamped
// values are never stored).
struct EpiOperands {
    float s[3];      // per-token scales of the P parts
    float alpha[4];  // per-channel scales
    float bias[4];
    float res[4];    // residual values (when Params::res is set)
};

// Residual values of row m, columns nb..nb+3 (clamped indices; the clamped values are never stored).
__device__ __forceinline__ void load_residual(const Params &p, int m, int nb, float *r) {
    if (!p.res) return;
    const int mm = m < p.M ? m : p.M - 1;
    const float *src = p.res + (long long)mm * p.ldr;
    if ((p.ldr & 3) == 0 && ((uintptr_t)p.res & 15) == 0 && nb + 3 < p.N) {
        const float4 v = *(const float4 *)(src + nb);
        r[0] = v.x; r[1] = v.y; r[2] = v.z; r[3] = v.w;
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = src[nb + i < p.N ? nb + i : p.N - 1];
    }
}

template <int P>
__device__ __forceinline__ void load_row_scales(const Params &p, int m, EpiOperands &e) {
    const int mm = m < p.M ? m : p.M - 1;
#pragma unroll
    for (int c = 0; c < 3; ++c) e.s[c] = c < P ? load_scalar(p.qs, p.qs_dtype, c * p.qs_stride + mm) : 0.f;
}

// Four consecutive values of a per-column vector (f32 or f16) at nb..nb+3: one vector load when they are all in range
// and the vector is aligned, else clamped scalar loads (the clamped values are never stored).
__device__ __forceinline__ void load_col4(const void *v, int dtype, bool vec, int nb, int N, float *out) {
    if (vec && nb + 3 < N) {
        if (dtype == KEA_F16) {
            const uint2 h = *(const uint2 *)((const _Float16 *)v + nb);
            const _Float16 *hv = (const _Float16 *)&h;
            out[0] = (float)hv[0]; out[1] = (float)hv[1]; out[2] = (float)hv[2]; out[3] = (float)hv[3];
        } else {
            const float4 f = *(const float4 *)((const float *)v + nb);
            out[0] = f.x; out[1] = f.y; out[2] = f.z; out[3] = f.w;
        }
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) out[r] = load_scalar(v, dtype, nb + r < N ? nb + r : N - 1);
    }
}

__device__ __forceinline__ void load_col_scales(const Params &p, int nb, EpiOperands &e, bool with_alpha = true) {
    if (with_alpha) {
        load_col4(p.ws, p.ws_dtype, p.ws_vec, nb, p.N, e.alpha);
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) e.alpha[r] = 0.f;
    }
    if (p.bias) {
        load_col4(p.bias, p.bias_dtype, p.bias_vec, nb, p.N, e.bias);
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) e.bias[r] = kNoBias;
    }
}

// The epilogue of 4 consecutive columns nb..nb+3 of row m from exact accumulators a[c][r].
template <int P>
__device__ __forceinline__ void epilogue4(const Params &p, int m, int nb, const int (*a)[4], const EpiOperands &e) {
    if (p.y) {
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            int ar[3] = {a[0][r], P > 1 ? a[1][r] : 0, P > 2 ? a[2][r] : 0};
            v[r] = finish(combine<P>(ar, e.s, p.flags), e.alpha[r], p.bias != nullptr, e.bias[r], p.flags);
            if (p.res) v[r] = e.res[r] + v[r] * p.res_factor;
        }
        if (p.flags & KEA_FLAG_GLU) {  // column pairs (value, gate): value * sigmoid(gate)
            const float u[2] = {v[0] * (1.0f / (1.0f + expf(-v[1]))), v[2] * (1.0f / (1.0f + expf(-v[3])))};
            store2(p, (long long)m * p.ldy + nb / 2, nb, u);
        } else {
            store4(p, (long long)m * p.ldy + nb, nb, v);
        }
    }
    if (p.acc) {
#pragma unroll
        for (int c = 0; c < P; ++c)
            store_int4(p.acc + ((long long)c * p.M + m) * p.acc_ld + nb, p.acc_vec, nb, p.N, a[c]);
    }
}

// epilogue4 for a plain output (no GLU pairs, no raw accumulators) of compile-time dtype DT whose 4 columns are all
// inside N with a vector-aligned y: the same values, one vector store at yrow + nb (yrow: the row's first element),
// no per-lane selection. RES: the residual is applied (Params::res is set).
template <int P, int DT, bool RES, bool SMALL>
__device__ __forceinline__ void epilogue4_full(const Params &p, void *yrow, int nb, const int (*a)[4],
                                               const EpiOperands &e) {
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        int ar[3] = {a[0][r], P > 1 ? a[1][r] : 0, P > 2 ? a[2][r] : 0};
        if constexpr (SMALL) {
            v[r] = finish(combine<P>(ar, e.s, p.flags), e.alpha[r], p.bias != nullptr, e.bias[r], p.flags);
            if (p.res) v[r] = e.res[r] + v[r] * p.res_factor;
        } else {
            v[r] = finish(combine<P>(ar, e.s, p.flags), e.alpha[r], e.bias[r], p.flags);
            if constexpr (RES) v[r] = e.res[r] + v[r] * p.res_factor;
        }
    }
    if constexpr (DT == KEA_F32) {
        *(float4 *)((float *)yrow + nb) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
        uint16_t h[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) h[r] = DT == KEA_F16 ? to_f16_bits(v[r]) : to_bf16_bits(v[r]);
        uint2 packed;
        packed.x = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
        packed.y = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
        *(uint2 *)((uint16_t *)yrow + nb) = packed;
    }
}

// The per-group epilogue of 4 consecutive columns: r holds sum_g fma(comb_P(acc_g), alpha[n][g], .) from the main
// loop; then r = bias ? r + bias : r, optional SiLU, store. a[c][r] are the full-K accumulators (for acc_out).
template <int P>
__device__ __forceinline__ void epilogue4_groups(const Params &p, int m, int nb, const int (*a)[4], const float *racc,
                                                 const EpiOperands &e) {
    if (p.y) {
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float x = racc[r];
            if (p.bias) x = x + e.bias[r];
            if (p.flags & KEA_FLAG_SILU) x = kea::silu_epilogue(x);
            if (p.res) x = e.res[r] + x * p.res_factor;
            v[r] = x;
        }
        store4(p, (long long)m * p.ldy + nb, nb, v);
    }
    if (p.acc) {
#pragma unroll
        for (int c = 0; c < P; ++c)
            store_int4(p.acc + ((long long)c * p.M + m) * p.acc_ld + nb, p.acc_vec, nb, p.N, a[c]);
    }
}

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
__host__ __device__ constexpr StageShape stage_shape(int wbits, int parts, int rm, int rn, int wm, int wn) {
    const int nw = wm * wn, bm = wm * rm * 16, bn = wn * rn * 16;
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
template <int WBITS, int P, int RM, int RN, int WM, int WN, bool SLICED, bool KTAIL, int GQ = 0>
__global__ void __launch_bounds__(WM *WN * 64) gemm_kernel(Params p) {
    static_assert(GQ == 0 || GQ == 1 || GQ == 2 || GQ == 4, "groups of 64, 128 or 256 k");
    static_assert(GQ == 0 || !SLICED, "per-group scales run unsplit");
    constexpr StageShape SHAPE = stage_shape(WBITS, P, RM, RN, WM, WN);
    constexpr int SW = SHAPE.sw, NS = SHAPE.ns;
    constexpr int NW = WM * WN;                 // wavefronts
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
    constexpr int LA = A_UNITS / 64 / NW;       // activation copies per wavefront per stage
    constexpr int LB = B_WORDS / NW;            // weight copies per wavefront per stage
    constexpr int L = LA + LB;
    static_assert(A_UNITS % (64 * NW) == 0, "activation stage must split evenly over the wavefronts");
    static_assert(B_WORDS % NW == 0, "weight stage must split evenly over the wavefronts");
    static_assert(L * (NS - 1) < 64, "in-flight copies exceed the vmcnt range");
    static_assert(L == SHAPE.copies && STAGE_BYTES == SHAPE.stage_bytes, "host and device stage geometry differ");
    static_assert(NS >= 2, "at least double buffering");
    static_assert(NS * STAGE_BYTES <= kLdsBudget, "the ring exceeds the LDS a workgroup may allocate");
    extern __shared__ __attribute__((aligned(16))) int8_t lds[];  // NS * STAGE_BYTES

    // the wavefront index is uniform; readfirstlane tells the compiler so (wave-derived math then runs on SALU)
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
        const int u = (i * NW + wave) * 64 + lane;
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
            for (int i = 0; i < LA; ++i) dma16(abase + a_off[i], buf + (i * NW + wave) * 64 * 16);
        } else {
#pragma unroll
            for (int i = 0; i < LA; ++i) {
                const uint32_t off = k0 + a_koff[i] < kend ? a_off[i] + (uint32_t)k0 : a_off[i] - (uint32_t)a_koff[i];
                dma16(p.q + off, buf + (i * NW + wave) * 64 * 16);
            }
        }
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            const int b = i * NW + wave;             // wave-uniform
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

    // One stage of MFMAs: straight-line code (no accumulator ever passes a control-flow merge; merges made the
    // compiler emit AGPR copy chains). Operand reads from LDS run ahead of the MFMAs: narrow tiles (P * RM <= 2, few
    // MFMAs per k-step) issue every read of the stage before the first MFMA, so a stage pays one LDS latency instead
    // of one per k-step; wider tiles read k-step t + 1 while the MFMAs of step t run. MASKED (the last stage) zeroes
    // the weights at k >= kend: per 16-byte group of a lane's operand, or per byte for KTAIL.
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

#pragma unroll
    for (int s = 0; s < NS - 1; ++s)
        if (s < nst) issue(s);

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
        const int issued_after = min(NS - 2, nst - 1 - s);  // stages issued after s so far
        wait_stage(issued_after);
        stage_barrier();  // stage s is in LDS for every wavefront; stage s-1's buffer is free
        if (s + NS - 1 < nst) issue(s + NS - 1);
        compute(s, plain_t{});
    }
    // the last stage (the host never launches an empty K range, so nst >= 1)
    wait_vmcnt<0>();
    stage_barrier();
    compute(nst - 1, masked_t{});

    // ---- epilogue: the MFMA result row is the weight row n, the column the activation row m ----
    // DT >= 0: the output dtype as a compile-time constant; then 16x16 tiles wholly inside [M, N) take a path without
    // per-lane bounds or dtype selection (the tile test is wave-uniform). DT < 0: the general epilogue.
    constexpr bool SMALL = RM * RN <= 2;
    auto epilogue = [&](auto dt_tag, auto res_tag) {
        constexpr int DT = decltype(dt_tag)::value;
        constexpr bool RES = decltype(res_tag)::value;
#pragma unroll
        for (int i = 0; i < RM; ++i) {
            const int mt = m0 + (wm * RM + i) * 16, m = mt + (lane & 15);
            if (m >= p.M) continue;
            void *yrow = (int8_t *)p.y + (long long)m * p.ldy * (DT == KEA_F32 ? 4 : 2);
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
                            epilogue4_full<P, DT, RES, SMALL>(p, yrow, nb, a, e);
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
    // plain outputs (no GLU pairs, no raw accumulators, vector-aligned y) branch once on the dtype
    const bool plain = !SLICED && GQ == 0 && p.y && !p.acc && !(p.flags & KEA_FLAG_GLU) && p.y_vec;
    using kRes = std::true_type;
    using kNoRes = std::false_type;
    // Tiles of one or two 16x16 blocks per wave (the small-M shapes) keep one epilogue copy per dtype with the
    // residual and bias tested at run time: separate copies measured slower there (config 1: 4.13 vs 4.27 us).
    if constexpr (SMALL) {
        if (plain && p.y_dtype == KEA_F16) epilogue(std::integral_constant<int, KEA_F16>{}, kNoRes{});
        else if (plain && p.y_dtype == KEA_BF16) epilogue(std::integral_constant<int, KEA_BF16>{}, kNoRes{});
        else if (plain && p.y_dtype == KEA_F32) epilogue(std::integral_constant<int, KEA_F32>{}, kNoRes{});
        else epilogue(std::integral_constant<int, -1>{}, kNoRes{});
        return;
    }
    if (plain && p.y_dtype == KEA_F16) {
        if (p.res) epilogue(std::integral_constant<int, KEA_F16>{}, kRes{});
        else epilogue(std::integral_constant<int, KEA_F16>{}, kNoRes{});
    } else if (plain && p.y_dtype == KEA_BF16) {
        if (p.res) epilogue(std::integral_constant<int, KEA_BF16>{}, kRes{});
        else epilogue(std::integral_constant<int, KEA_BF16>{}, kNoRes{});
    } else if (plain && p.y_dtype == KEA_F32) {
        if (p.res) epilogue(std::integral_constant<int, KEA_F32>{}, kRes{});
        else epilogue(std::integral_constant<int, KEA_F32>{}, kNoRes{});
    } else {
        epilogue(std::integral_constant<int, -1>{}, kNoRes{});
    }
}

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

struct Tile {
    int rm, rn, wm, wn;
    const char *name;
};

// Tile configurations (ids are 1-based in the ABI). Results are identical for every tile.
constexpr Tile kTiles[] = {
    {1, 1, 1, 4, "16x64 w1x4 r1x1"},   // 1
    {2, 1, 1, 4, "32x64 w1x4 r2x1"},   // 2
    {1, 2, 2, 2, "32x64 w2x2 r1x2"},   // 3
    {1, 1, 2, 2, "32x32 w2x2 r1x1"},   // 4
    {4, 1, 1, 4, "64x64 w1x4 r4x1"},   // 5
    {8, 1, 1, 4, "128x64 w1x4 r8x1"},  // 6
    {2, 4, 2, 2, "64x128 w2x2 r2x4"},  // 7
    {4, 2, 1, 4, "64x128 w1x4 r4x2"},  // 8
    {2, 2, 1, 4, "32x128 w1x4 r2x2"},  // 9
    {2, 4, 2, 4, "64x256 w2x4 r2x4"},  // 10
    {4, 2, 2, 4, "128x128 w2x4 r4x2"}, // 11
    {1, 2, 2, 4, "32x128 w2x4 r1x2"},  // 12
};
constexpr int kNumTiles = sizeof(kTiles) / sizeof(kTiles[0]);

// Register budget of a tile: accumulators plus double-buffered activation fragments (in 32-bit registers); and two
// ring buffers of the tile's stage within the LDS a workgroup may allocate.
constexpr bool tile_fits(int wbits, int parts, int rm, int rn, int wm, int wn) {
    return parts * rm * rn * 4 + 2 * parts * rm * 4 <= 256 &&
           2 * stage_shape(wbits, parts, rm, rn, wm, wn).stage_bytes <= kLdsBudget;
}

inline long long cdivl(long long a, long long b) { return (a + b - 1) / b; }

using KernelFn = void (*)(Params);

template <int WBITS, int P, int RM, int RN, int WM, int WN>
KernelFn pick_sliced(bool sliced) {
    return sliced ? gemm_kernel<WBITS, P, RM, RN, WM, WN, true, false>
                  : gemm_kernel<WBITS, P, RM, RN, WM, WN, false, false>;
}

template <int WBITS, int P, int RM, int RN, int WM, int WN>
KernelFn pick_fit(bool sliced) {
    if constexpr (tile_fits(WBITS, P, RM, RN, WM, WN)) return pick_sliced<WBITS, P, RM, RN, WM, WN>(sliced);
    else return nullptr;
}

template <int WBITS, int P>
KernelFn pick_tile(int id, bool sliced) {
    switch (id) {
        case 1: return pick_fit<WBITS, P, 1, 1, 1, 4>(sliced);
        case 2: return pick_fit<WBITS, P, 2, 1, 1, 4>(sliced);
        case 3: return pick_fit<WBITS, P, 1, 2, 2, 2>(sliced);
        case 4: return pick_fit<WBITS, P, 1, 1, 2, 2>(sliced);
        case 5: return pick_fit<WBITS, P, 4, 1, 1, 4>(sliced);
        case 6: return pick_fit<WBITS, P, 8, 1, 1, 4>(sliced);
        case 7: return pick_fit<WBITS, P, 2, 4, 2, 2>(sliced);
        case 8: return pick_fit<WBITS, P, 4, 2, 1, 4>(sliced);
        case 9: return pick_fit<WBITS, P, 2, 2, 1, 4>(sliced);
        case 10: return pick_fit<WBITS, P, 2, 4, 2, 4>(sliced);
        case 11: return pick_fit<WBITS, P, 4, 2, 2, 4>(sliced);
        case 12: return pick_fit<WBITS, P, 1, 2, 2, 4>(sliced);
        default: return nullptr;
    }
}

// K % 16 != 0 runs the byte-precise variant of tile kTailTile, unsplit.
constexpr int kTailTile = 4;
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
KernelFn pick_group(int wbits, int parts, int gq, int id, bool ktail) {
    if (wbits == 1)
        return parts == 1 ? pick_group_p<1, 1>(gq, id, ktail)
             : parts == 2 ? pick_group_p<1, 2>(gq, id, ktail) : pick_group_p<1, 3>(gq, id, ktail);
    return parts == 1 ? pick_group_p<2, 1>(gq, id, ktail)
         : parts == 2 ? pick_group_p<2, 2>(gq, id, ktail) : pick_group_p<2, 3>(gq, id, ktail);
}

KernelFn pick_kernel(int wbits, int parts, int id, bool sliced, bool ktail) {
    if (ktail) {
        if (wbits == 1) return parts == 1 ? pick_ktail<1, 1>() : parts == 2 ? pick_ktail<1, 2>() : pick_ktail<1, 3>();
        return parts == 1 ? pick_ktail<2, 1>() : parts == 2 ? pick_ktail<2, 2>() : pick_ktail<2, 3>();
    }
    if (wbits == 1) {
        if (parts == 1) return pick_tile<1, 1>(id, sliced);
        if (parts == 2) return pick_tile<1, 2>(id, sliced);
        return pick_tile<1, 3>(id, sliced);
    }
    if (parts == 1) return pick_tile<2, 1>(id, sliced);
    if (parts == 2) return pick_tile<2, 2>(id, sliced);
    return pick_tile<2, 3>(id, sliced);
}

using FinishFn = void (*)(Params, int);
FinishFn pick_finish(int parts) {
    if (parts == 1) return finish_kernel<1>;
    if (parts == 2) return finish_kernel<2>;
    return finish_kernel<3>;
}

// Tile and split choice: a pure function of (wbits, parts, m, n, k), fitted to MI355X sweeps of every tile x split
// over BASELINE.json's shapes, the reference's tuned (N, K, M) points and the encoder's shapes at P = 1, 2 and 3 (HIP
// graph replay, M from 1 to 1000). Small M wants many workgroups: the 16x64 (P >= 2) and 32x32 (P = 1) tiles, whose
// register budgets leave room for co-resident workgroups. As M grows the activation tile, re-read once per column
// tile, becomes the traffic that bounds a CU, so the winners widen in N: 32x64 / 64x64 at P = 1, and at P >= 2 (where
// the activations are P times larger) the eight-wavefront 32x128 and 64x256 tiles, 10-17% faster than the
// four-wavefront ones at M = 1000.
int choose_tile(int wbits, int parts, long long m, long long n, long long k) {
    (void)wbits; (void)k;
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

// Split factor for split_k == 0: split K only for long K ranges (>= 2048) whose tiling leaves at most 64 workgroups,
// by powers of two up to 8 slices and 256 workgroups (ternary, one part, K >= 4096: up to 128 workgroups, 512 after
// the split); the split's second launch costs more than it saves otherwise.
int choose_split(int wbits, int parts, long long m, long long n, long long k, int id) {
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

int kea_config_count(void) { return kNumTiles; }

const char *kea_config_name(int config) {
    if (config < 1 || config > kNumTiles) return "";
    return kTiles[config - 1].name;
}

static int resolve(int wbits, int parts, int64_t m, int64_t n, int64_t k, int split_k, int config, int *tile,
                   int *split, int *qps) {
    if (wbits != 1 && wbits != 2) return kea::fail(KEA_EINVAL, "wbits must be 1 or 2");
    if (parts < 1 || parts > 3) return kea::fail(KEA_EINVAL, "parts must be 1, 2 or 3");
    if (m < 0 || n < 1 || k < 1 || m > INT32_MAX || n > INT32_MAX || k > INT32_MAX)
        return kea::fail(KEA_EINVAL, "bad sizes");
    if (config < 0 || config > kNumTiles) return kea::fail(KEA_EINVAL, "unknown config id");
    if (split_k < 0) return kea::fail(KEA_EINVAL, "split_k must be >= 0");
    int id = config ? config : choose_tile(wbits, parts, m, n, k);
    const Tile &tl = kTiles[id - 1];
    if (!tile_fits(wbits, parts, tl.rm, tl.rn, tl.wm, tl.wn))
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

static int gemm_impl(int wbits, const int8_t *q, int64_t part_stride, int64_t ldq, int parts, const void *qs,
                     int qs_dtype, int64_t qs_stride, const uint32_t *w, int64_t n, int64_t k, const void *wscale,
                     int ws_dtype, int64_t ws_group, const void *bias, int bias_dtype, void *y, int y_dtype,
                     int64_t ldy, int32_t *acc_out, int64_t acc_ld, int64_t m, int flags, int split_k, int config,
                     void *workspace, int64_t workspace_bytes, const float *residual, int64_t ldr, float factor,
                     void *stream) {
    int tile, s, qps, gq = 0;
    if (ws_group != 0) {
        if (ws_group != 64 && ws_group != 128 && ws_group != 256)
            return kea::fail(KEA_EINVAL, "ws_group must be 0 (per-channel scales), 64, 128 or 256");
        if (config != 0 && config != 1 && config != 4)
            return kea::fail(KEA_EINVAL, "per-group weight scales run tile configs 1 and 4 only");
        if (split_k > 1) return kea::fail(KEA_EINVAL, "per-group weight scales run unsplit (split_k 0 or 1)");
        gq = (int)(ws_group / 64);
        if (!config) config = parts >= 2 ? 1 : 4;
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
    if (m == 0) return KEA_OK;
    if (!q) return kea::fail(KEA_EINVAL, "q is required");
    if (ldq < k) return kea::fail(KEA_EINVAL, "ldq < k");
    if (parts > 1 && part_stride < m * ldq) return kea::fail(KEA_EINVAL, "part_stride < m * ldq (parts overlap)");
    if (((uintptr_t)q & 15) || (ldq & 15) || (parts > 1 && (part_stride & 15)))
        return kea::fail(KEA_EALIGN, "q needs 16-byte aligned rows: q % 16 == 0, ldq % 16 == 0, part_stride % 16 == 0");
    if ((uintptr_t)w & 15) return kea::fail(KEA_EALIGN, "weight words must be 16-byte aligned");
    if ((int64_t)(parts - 1) * part_stride + m * ldq > (int64_t)INT32_MAX)
        return kea::fail(KEA_EINVAL, "q spans more than 2 GiB: split the call along M");

    Params p = {};
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
    p.ws_vec = ((uintptr_t)wscale % (ws_dtype == KEA_F16 ? 8 : 16)) == 0;
    p.bias_vec = bias && ((uintptr_t)bias % (bias_dtype == KEA_F16 ? 8 : 16)) == 0;

    const Tile &t = kTiles[tile - 1];
    const int bm = t.wm * t.rm * 16, bn = t.wn * t.rn * 16;
    // Ring buffers actually used: a workgroup touches buffer s % NS for its stages s < nst, so with nst < NS only
    // the first nst buffers need LDS.
    const long long words_per_wg = std::min<long long>(4LL * qps, (long long)p.J);
    const StageShape shape = stage_shape(wbits, parts, t.rm, t.rn, t.wm, t.wn);
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
    if (!kea::fits_dispatch(cdivl(n, bn), t.wm * t.wn * 64) ||
        (s > 1 && !kea::fits_dispatch(cdivl(m * cdivl(n, 4), 256), 256)))
        return kea::fail(KEA_EINVAL, "too large for one launch: split the call along N or M");
    dim3 grid((unsigned)cdivl(n, bn), (unsigned)cdivl(m, bm), (unsigned)s);
    dim3 block(t.wm * t.wn * 64);
    hipStream_t st = (hipStream_t)stream;
    if (s > 1) {
        const int64_t need = (int64_t)s * parts * m * n * 4;
        if (!workspace || workspace_bytes < need)
            return kea::fail(KEA_ESPACE, "split-K workspace too small: need " + std::to_string(need) + " bytes");
        if ((uintptr_t)workspace & 15) return kea::fail(KEA_EALIGN, "workspace must be 16-byte aligned");
        p.slices = (int32_t *)workspace;
        p.slice_vec = (n % 4 == 0);
    }
    KernelFn fn = gq ? pick_group(wbits, parts, gq, tile, (k & 15) != 0)
                     : pick_kernel(wbits, parts, tile, s > 1, (k & 15) != 0);
    if (lds_bytes > 65536) {
        hipError_t e = hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
        if (e != hipSuccess) return kea::fail((int)e, std::string("LDS attribute refused: ") + hipGetErrorString(e));
    }
    hipLaunchKernelGGL(fn, grid, block, lds_bytes, st, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("gemm launch failed: ") + hipGetErrorString(e));
    if (s > 1) {
        const long long work = m * cdivl(n, 4);
        hipLaunchKernelGGL(pick_finish(parts), dim3((unsigned)cdivl(work, 256)), dim3(256), 0, st, p, s);
        e = hipGetLastError();
        if (e != hipSuccess) return kea::fail((int)e, std::string("finish launch failed: ") + hipGetErrorString(e));
    }
    return KEA_OK;
}

int kea_lowbit_gemm(int wbits, const int8_t *q, int64_t part_stride, int64_t ldq, int parts, const void *qs,
                    int qs_dtype, int64_t qs_stride, const uint32_t *w, int64_t n, int64_t k, const void *wscale,
                    int ws_dtype, int64_t ws_group, const void *bias, int bias_dtype, void *y, int y_dtype,
                    int64_t ldy, int32_t *acc_out, int64_t acc_ld, int64_t m, int flags, int split_k, int config,
                    void *workspace, int64_t workspace_bytes, void *stream) {
    return gemm_impl(wbits, q, part_stride, ldq, parts, qs, qs_dtype, qs_stride, w, n, k, wscale, ws_dtype, ws_group,
                     bias, bias_dtype, y, y_dtype, ldy, acc_out, acc_ld, m, flags, split_k, config, workspace,
                     workspace_bytes, nullptr, 0, 0.f, stream);
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
    Params p = {};
    p.q = q; p.part_stride = part_stride; p.ldq = ldq;
    p.w = w;
    p.M = (int)m; p.N = (int)n; p.K = (int)k;
    p.J = (int)(wbits == 1 ? cdivl(k, 128) : cdivl(k, 64));
    p.NT = (int)cdivl(n, 16);
    p.quads_per_slice = qps;
    p.slices = slices;
    p.slice_vec = (n % 4 == 0);
    const Tile &t = kTiles[tile - 1];
    const int bm = t.wm * t.rm * 16, bn = t.wn * t.rn * 16;
    const long long words_per_wg = std::min<long long>(4LL * qps, (long long)p.J);
    const StageShape shape = stage_shape(wbits, parts, t.rm, t.rn, t.wm, t.wn);
    const int nst = (int)cdivl(words_per_wg, shape.sw);
    const int lds_bytes = std::min(shape.ns, nst) * shape.stage_bytes;
    if (!kea::fits_dispatch(cdivl(n, bn), t.wm * t.wn * 64))
        return kea::fail(KEA_EINVAL, "too large for one launch: split the call along N");
    KernelFn fn = pick_kernel(wbits, parts, tile, true, false);
    if (lds_bytes > 65536) {
        hipError_t e = hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
        if (e != hipSuccess) return kea::fail((int)e, std::string("LDS attribute refused: ") + hipGetErrorString(e));
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)cdivl(n, bn), (unsigned)cdivl(m, bm), (unsigned)s), dim3(t.wm * t.wn * 64),
                       lds_bytes, (hipStream_t)stream, p);
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
    p.ws_vec = ((uintptr_t)wscale % (ws_dtype == KEA_F16 ? 8 : 16)) == 0;
    p.bias_vec = bias && ((uintptr_t)bias % (bias_dtype == KEA_F16 ? 8 : 16)) == 0;
    const long long work = m * cdivl(n, 4);
    if (!kea::fits_dispatch(cdivl(work, 256), 256))
        return kea::fail(KEA_EINVAL, "too large for one launch: split the call along M");
    hipLaunchKernelGGL(pick_finish(parts), dim3((unsigned)cdivl(work, 256)), dim3(256), 0, (hipStream_t)stream, p, split);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("finish launch failed: ") + hipGetErrorString(e));
    return KEA_OK;
}

}  // extern "C"
