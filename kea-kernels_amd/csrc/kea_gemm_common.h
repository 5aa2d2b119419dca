// Pieces shared by the low-bit GEMM kernels (kea_gemm.hip: the LDS-ring kernel, the split-K finish;
// kea_gemm_wsplit.hip: the wave-split kernel): the launch parameter block, the 1-/2-bit expansion to int8 MFMA
// operands and the fused epilogue of four consecutive output columns.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kea_epilogue.h"
#include "kea_internal.h"

namespace kea {

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
    int steps_per_slice;   // wave-split kernel: k-steps of 64 per workgroup (one K slice)
};

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
    // The FP32 value is rounded to FP32 first and then to FP16 (the contract's two roundings). Without the empty asm
    // the instruction selector may fuse an fma that produced v into a mixed-precision fma with one FP16 rounding
    // (v_fma_mixlo_f16), which differs in the last FP16 bit for some inputs.
    asm("" : "+v"(v));
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

// A per-column vector of f32 or f16 values (per-channel scales, bias) read through a range-checked buffer
// descriptor: its base is the vector's start aligned down to 4 bytes (`delta` bytes before it) and its extent ends at
// the 4-byte word holding the last element, so a load past the vector's end returns zeros instead of touching memory
// (those values belong to columns past N, which are never stored) and no per-element clamp is needed.
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
struct ColVec {
    __amdgpu_buffer_rsrc_t rsrc;
    int delta;
};
__device__ __forceinline__ ColVec col_vec(const void *v, bool f16, int n) {
    const uintptr_t a = (uintptr_t)v & ~(uintptr_t)3;
    const int d = (int)((uintptr_t)v & 3);
    // data format 32 in the descriptor's last word: the raw (untyped) buffer form of gfx9
    // 32-bit byte extent and offsets: the host launches the GEMM kernels with n < 2^30
    const uint32_t extent = ((uint32_t)d + (uint32_t)n * (f16 ? 2u : 4u) + 3u) & ~3u;
    return ColVec{__builtin_amdgcn_make_buffer_rsrc((void *)a, (short)0, (int)extent, 0x00020000), d};
}
// The 16 bytes from the 4-byte word holding element nb (nb % 4 == 0): f32 elements nb .. nb+3 are its words 0..3; f16
// elements nb .. nb+3 start at bit 8 * delta of word 0 (delta 0 or 2: f16 vectors are 2-byte aligned).
__device__ __forceinline__ v4u col_load4(const ColVec &c, bool f16, int nb) {
    return __builtin_amdgcn_raw_buffer_load_b128(c.rsrc, (int)(((uint32_t)c.delta + (uint32_t)nb * (f16 ? 2u : 4u)) & ~3u),
                                                 0, 0);
}
__device__ __forceinline__ void col_to_f32(v4u w, bool f16, int delta, float (&out)[4]) {
    if (f16) {  // wave-uniform
        const uint32_t sh = (uint32_t)delta * 8u;
        const uint32_t h01 = __builtin_amdgcn_alignbit(w.y, w.x, sh), h23 = __builtin_amdgcn_alignbit(w.z, w.y, sh);
        out[0] = (float)__builtin_bit_cast(_Float16, (uint16_t)h01);
        out[1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(h01 >> 16));
        out[2] = (float)__builtin_bit_cast(_Float16, (uint16_t)h23);
        out[3] = (float)__builtin_bit_cast(_Float16, (uint16_t)(h23 >> 16));
    } else {
        // the whole vector is cast: hipcc's __builtin_bit_cast of one component access (w.y, ...) reads component 0
        const v4f f = __builtin_bit_cast(v4f, w);
        out[0] = f.x;
        out[1] = f.y;
        out[2] = f.z;
        out[3] = f.w;
    }
}

// Four consecutive values nb..nb+3 (nb % 4 == 0) of a per-column vector of N values (f32 or f16): one range-checked
// 16-byte load (values past N read 0; their columns are never stored).
__device__ __forceinline__ void load_col4(const void *v, int dtype, int nb, int N, float *out) {
    const bool f16 = dtype == KEA_F16;
    const ColVec c = col_vec(v, f16, N);
    float f[4];
    col_to_f32(col_load4(c, f16, nb), f16, c.delta, f);
#pragma unroll
    for (int r = 0; r < 4; ++r) out[r] = f[r];
}

__device__ __forceinline__ void load_col_scales(const Params &p, int nb, EpiOperands &e, bool with_alpha = true) {
    if (with_alpha) {
        load_col4(p.ws, p.ws_dtype, nb, p.N, e.alpha);
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) e.alpha[r] = 0.f;
    }
    if (p.bias) {
        load_col4(p.bias, p.bias_dtype, nb, p.N, e.bias);
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) e.bias[r] = kNoBias;
    }
}

// The GLU of a column pair (value, gate): value * sigmoid(gate), the one expression every epilogue uses.
__device__ __forceinline__ float glu_pair(float value, float gate) { return value * (1.0f / (1.0f + expf(-gate))); }

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
            const float u[2] = {glu_pair(v[0], v[1]), glu_pair(v[2], v[3])};
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

// epilogue4 for an output without raw accumulators, of compile-time dtype DT, whose 4 columns are all inside N with a
// vector-aligned y: the same values, one vector store at yrow + nb (yrow: the row's first element), no per-lane
// selection. RES: the residual is applied (Params::res is set). SILU: 1 / 0 the SiLU is / is not applied (known at
// compile time: a run-time flag makes the compiler evaluate the SiLU for every output and select), -1: as
// Params::flags says. GLU: the two column pairs become two outputs at yrow + nb / 2 (no residual, no SiLU).
template <int P, int DT, bool RES, bool SMALL, int SILU = -1, bool GLU = false>
__device__ __forceinline__ void epilogue4_full(const Params &p, void *yrow, int nb, const int (*a)[4],
                                               const EpiOperands &e) {
    static_assert(!GLU || (!RES && SILU == 0), "the GLU output takes neither a residual nor the SiLU");
    const int flags = SILU < 0 ? p.flags : SILU ? (p.flags | KEA_FLAG_SILU) : (p.flags & ~KEA_FLAG_SILU);
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        int ar[3] = {a[0][r], P > 1 ? a[1][r] : 0, P > 2 ? a[2][r] : 0};
        if constexpr (SMALL) {
            v[r] = finish(combine<P>(ar, e.s, flags), e.alpha[r], p.bias != nullptr, e.bias[r], flags);
            if (p.res) v[r] = e.res[r] + v[r] * p.res_factor;
        } else {
            v[r] = finish(combine<P>(ar, e.s, flags), e.alpha[r], e.bias[r], flags);
            if constexpr (RES) v[r] = e.res[r] + v[r] * p.res_factor;
        }
    }
    if constexpr (GLU) {
        const float u0 = glu_pair(v[0], v[1]), u1 = glu_pair(v[2], v[3]);
        if constexpr (DT == KEA_F32) {
            *(float2 *)((float *)yrow + nb / 2) = make_float2(u0, u1);
        } else {
            const uint32_t h0 = DT == KEA_F16 ? to_f16_bits(u0) : to_bf16_bits(u0);
            const uint32_t h1 = DT == KEA_F16 ? to_f16_bits(u1) : to_bf16_bits(u1);
            *(uint32_t *)((uint16_t *)yrow + nb / 2) = h0 | (h1 << 16);
        }
    } else if constexpr (DT == KEA_F32) {
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

}  // namespace kea
