// Residual int8 activation quantizer with optional fused LayerNorm and input SiLU.
//
// Semantics follow the reference's quantizers (kk/binary/kernels.py:567-616 and the Triton `_quantize`,
// kk/ternary/fused_kernels.py:31-50):
//     z = x ; z = LayerNorm(z) * w + b (optional) ; z = z * sigmoid(z) (optional)
//     for c < P:  s_c = max(max|z| / 127, 1e-30) ; q_c = rint(z / s_c) ; z = z - q_c * s_c
// with IEEE division and round-half-even (the reference's `div.full` / `ex2.approx` NVIDIA approximations are not
// reproduced). With fp16 scales the scale is rounded to fp16 (kept >= the smallest fp16 subnormal, <= the largest
// finite fp16) before use and q is clamped to [-127, 127].
//
// Layout: a row is handled by WPR wave64s (1 for K <= 256, 4 above), thread th of the row holding the 4-element
// chunks k = 4 * (th + 64 * WPR * i) + j: consecutive threads read consecutive 16-byte chunks (one float4 load each
// when the row is contiguous and aligned) and store the 4 quantized bytes as one dword. The LayerNorm sums, the only
// reductions that are not exact, use one fixed order that the CPU oracle restates: each thread sums its elements in
// increasing k, a xor butterfly over the 64 lanes of each wave (offsets 1, 2, 4, ..., 32; kea_wave.h), then the wave
// totals in wave order. The max reductions are exact in any order.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "kea_epilogue.h"
#include "kea_internal.h"
#include "kea_merge.h"
#include "kea_rowq.h"
#include "kea_wave.h"
#include "../../include/kea_encoder.h"

namespace {

using kea::quantize_code;
using kea::wave_max;
using kea::wave_sum;

__device__ __forceinline__ float load_x(const void *x, int dtype, long long i) {
    if (dtype == KEA_F16) return (float)(((const _Float16 *)x)[i]);
    return ((const float *)x)[i];
}

// Row-wide reduction over the WPR waves of a row: wave butterfly, then the wave totals in wave order through LDS.
// slot: a distinct LDS slot per reduction of the kernel (no barrier is needed before a slot's reuse).
template <int WPR, bool MAX>
__device__ __forceinline__ float row_reduce(float v, float (*red)[WPR], int slot, int wave) {
    v = MAX ? wave_max(v) : wave_sum(v);
    if constexpr (WPR == 1) {
        return v;
    } else {
        if ((threadIdx.x & 63) == 0) red[slot][wave] = v;
        __syncthreads();
        float r = red[slot][0];
#pragma unroll
        for (int w = 1; w < WPR; ++w) r = MAX ? fmaxf(r, red[slot][w]) : r + red[slot][w];
        return r;
    }
}

// VPT: 4-element chunks per thread (K <= 256 * WPR * VPT). VEC: contiguous, 16-byte aligned rows and LayerNorm weights
// (float4 loads), K % 4 == 0 and ldq % 4 == 0 (dword stores); otherwise element-wise access with any strides.
template <int VPT, int WPR, bool VEC>
__global__ void __launch_bounds__(256)
quantize_kernel(const void *x, int x_dtype, long long xb, long long xt, long long xk, long long t, int M, int K,
                int parts, const float *nw, const float *nb, float eps, int input_silu, int8_t *q, long long ldq,
                void *qs, int qs_dtype) {
    constexpr int RPB = 4 / WPR;     // rows per block
    constexpr int TPR = 64 * WPR;    // threads per row
    __shared__ float red[RPB][5][WPR];
    const int th = threadIdx.x % TPR, rl = threadIdx.x / TPR, wave = th >> 6;
    const int m = blockIdx.x * RPB + rl;
    if (m >= M) return;  // whole rows leave together: the row's barriers stay matched
    const long long base = (long long)(m / t) * xb + (long long)(m % t) * xt;
    // LayerNorm weights are loaded with the row (their latency overlaps the row's and the reductions')
    float lw[VPT][4], lb[VPT][4];
    if (nw) {
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int k0 = 4 * (th + TPR * i);
            if constexpr (VEC) {  // K % 4 == 0: a chunk is inside the row or past it; one 16-byte load each
                float4 w4 = make_float4(0.f, 0.f, 0.f, 0.f), b4 = w4;
                if (k0 < K) {
                    w4 = *(const float4 *)(nw + k0);
                    b4 = *(const float4 *)(nb + k0);
                }
                lw[i][0] = w4.x; lw[i][1] = w4.y; lw[i][2] = w4.z; lw[i][3] = w4.w;
                lb[i][0] = b4.x; lb[i][1] = b4.y; lb[i][2] = b4.z; lb[i][3] = b4.w;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    lw[i][j] = k0 + j < K ? nw[k0 + j] : 0.f;
                    lb[i][j] = k0 + j < K ? nb[k0 + j] : 0.f;
                }
            }
        }
    }
    float z[VPT][4];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int k0 = 4 * (th + TPR * i);
        if constexpr (VEC) {
            if (k0 < K) {
                if (x_dtype == KEA_F16) {
                    const uint2 h = *(const uint2 *)((const _Float16 *)x + base + k0);
                    const _Float16 *hv = (const _Float16 *)&h;
                    z[i][0] = (float)hv[0]; z[i][1] = (float)hv[1]; z[i][2] = (float)hv[2]; z[i][3] = (float)hv[3];
                } else {
                    const float4 v = *(const float4 *)((const float *)x + base + k0);
                    z[i][0] = v.x; z[i][1] = v.y; z[i][2] = v.z; z[i][3] = v.w;
                }
            } else {
                z[i][0] = z[i][1] = z[i][2] = z[i][3] = 0.f;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) z[i][j] = k0 + j < K ? load_x(x, x_dtype, base + (long long)(k0 + j) * xk) : 0.f;
        }
    }
    if (nw) {
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < VPT; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) sum = sum + z[i][j];
        const float mean = row_reduce<WPR, false>(sum, red[rl], 0, wave) / (float)K;
        float sq = 0.f;
#pragma unroll
        for (int i = 0; i < VPT; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int k = 4 * (th + TPR * i) + j;
                z[i][j] = k < K ? z[i][j] - mean : 0.f;
                sq = sq + z[i][j] * z[i][j];
            }
        const float var = row_reduce<WPR, false>(sq, red[rl], 1, wave) / (float)K;
        const float inv = 1.0f / sqrtf(var + eps);
#pragma unroll
        for (int i = 0; i < VPT; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int k = 4 * (th + TPR * i) + j;
                if (k < K) z[i][j] = z[i][j] * inv * lw[i][j] + lb[i][j];
            }
    }
    if (input_silu) {
#pragma unroll
        for (int i = 0; i < VPT; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) z[i][j] = z[i][j] * (1.0f / (1.0f + expf(-z[i][j])));
    }
    for (int c = 0; c < parts; ++c) {
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < VPT; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) amax = fmaxf(amax, fabsf(z[i][j]));
        amax = row_reduce<WPR, true>(amax, red[rl], 2 + c, wave);
        float s = fmaxf(amax / 127.0f, 1.0e-30f);
        if (qs_dtype == KEA_F16) {
            _Float16 h = (_Float16)s;
            float hs = (float)h;
            hs = fmaxf(hs, 5.9604644775390625e-08f);  // 2^-24, the smallest fp16 subnormal
            hs = fminf(hs, 65504.0f);
            s = hs;
            if (th == 0) ((_Float16 *)qs)[(long long)c * M + m] = (_Float16)s;
        } else if (th == 0) {
            ((float *)qs)[(long long)c * M + m] = s;
        }
        const float inv = 1.0f / s;
        int8_t *row = q + ((long long)c * M + m) * ldq;
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int k0 = 4 * (th + TPR * i);
            uint32_t packed = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) packed |= quantize_code(z[i][j], s, inv) << (8 * j);
            if constexpr (VEC) {
                if (k0 < K) *(uint32_t *)(row + k0) = packed;  // k0 + 3 < ldq: ldq >= K and ldq % 4 == 0
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (k0 + j < K) row[k0 + j] = (int8_t)(packed >> (8 * j));
            }
        }
        const long long kpad = VEC ? (long long)((K + 3) & ~3) : (long long)K;
        for (long long k = kpad + th; k < ldq; k += TPR) row[k] = 0;
    }
}

// Quantizes the row a thread group holds in registers (thread th of TPR = 64 * WPR holds the 4-element chunks
// k = 4 * (th + TPR * i) + j; zero past K) into P residual parts, exactly as quantize_kernel (f32 scales, ldq % 4 == 0).
template <int VPT, int WPR>
__device__ __forceinline__ void quantize_parts(float (*z)[4], int K, int parts, int8_t *q, long long ldq, float *qs,
                                               int M, int m, int th, float (*red)[WPR], int wave) {
    constexpr int TPR = 64 * WPR;
    for (int c = 0; c < parts; ++c) {
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < VPT; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) amax = fmaxf(amax, fabsf(z[i][j]));
        amax = row_reduce<WPR, true>(amax, red, 2 + c, wave);
        const float s = fmaxf(amax / 127.0f, 1.0e-30f);
        if (th == 0) qs[(long long)c * M + m] = s;
        const float inv = 1.0f / s;
        int8_t *row = q + ((long long)c * M + m) * ldq;
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int k0 = 4 * (th + TPR * i);
            uint32_t packed = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) packed |= quantize_code(z[i][j], s, inv) << (8 * j);
            if (k0 < K) *(uint32_t *)(row + k0) = packed;
        }
        for (long long k = ((K + 3) & ~3) + th; k < ldq; k += TPR) row[k] = 0;
    }
}

// LayerNorm of the row in registers with the library's fixed summation order (see the file comment).
template <int VPT, int WPR>
__device__ __forceinline__ void layer_norm_row(float (*z)[4], int K, const float *w, const float *b, float eps,
                                               int th, float (*red)[WPR], int wave, int slot) {
    constexpr int TPR = 64 * WPR;
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) sum = sum + z[i][j];
    const float mean = row_reduce<WPR, false>(sum, red, slot, wave) / (float)K;
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = 4 * (th + TPR * i) + j;
            z[i][j] = k < K ? z[i][j] - mean : 0.f;
            sq = sq + z[i][j] * z[i][j];
        }
    const float var = row_reduce<WPR, false>(sq, red, slot + 1, wave) / (float)K;
    const float inv = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int k0 = 4 * (th + TPR * i);
        if (k0 < K) {
            const float4 lw = *(const float4 *)(w + k0), lb = *(const float4 *)(b + k0);
            z[i][0] = z[i][0] * inv * lw.x + lb.x; z[i][1] = z[i][1] * inv * lw.y + lb.y;
            z[i][2] = z[i][2] * inv * lw.z + lb.z; z[i][3] = z[i][3] * inv * lw.w + lb.w;
        }
    }
}

// x_out = LayerNorm0(x) (stored), then the P-part quantization of LayerNorm1(x_out): the output LayerNorm of one
// encoder layer fused with the normalised quantization that feeds the next layer's first projection (the reference's
// row epilogue, kk/ternary/row_fusion.py:28-53). WPR waves per row with the quantizer's rule and summation order,
// rows contiguous, K % 4 == 0.
template <int VPT, int WPR>
__global__ void __launch_bounds__(256)
norm_quantize_kernel(const float *x, long long ldx, int M, int K, const float *w0, const float *b0, float eps0,
                     float *x_out, long long ldo, const float *w1, const float *b1, float eps1, int parts, int8_t *q,
                     long long ldq, float *qs) {
    constexpr int RPB = 4 / WPR, TPR = 64 * WPR;
    __shared__ float red[RPB][7][WPR];
    const int th = threadIdx.x % TPR, rl = threadIdx.x / TPR, wave = th >> 6, m = blockIdx.x * RPB + rl;
    if (m >= M) return;  // whole rows leave together: the row's barriers stay matched
    float z[VPT][4];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int k0 = 4 * (th + TPR * i);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (k0 < K) v = *(const float4 *)(x + (long long)m * ldx + k0);
        z[i][0] = v.x; z[i][1] = v.y; z[i][2] = v.z; z[i][3] = v.w;
    }
    layer_norm_row<VPT, WPR>(z, K, w0, b0, eps0, th, red[rl], wave, 5);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int k0 = 4 * (th + TPR * i);
        if (k0 < K) *(float4 *)(x_out + (long long)m * ldo + k0) = make_float4(z[i][0], z[i][1], z[i][2], z[i][3]);
    }
    layer_norm_row<VPT, WPR>(z, K, w1, b1, eps1, th, red[rl], wave, 0);
    quantize_parts<VPT, WPR>(z, K, parts, q, ldq, qs, M, m, th, red[rl], wave);
}

// The P-part quantization of the attention output rows that the key-split attention left as two halves: the merge
// of kea_merge.h (the same bits the split attention's merge kernel writes), then quantize_parts. WPR waves per row
// with the quantizer's rule (K = heads * 128).
template <int VPT, int WPR>
__global__ void __launch_bounds__(256)
attention_merge_quantize_kernel(kea::SplitWs ws, long long rows, int heads, int parts, int8_t *q, long long ldq,
                                float *qs) {
    constexpr int RPB = 4 / WPR, TPR = 64 * WPR;
    __shared__ float red[RPB][5][WPR];
    const int th = threadIdx.x % TPR, rl = threadIdx.x / TPR, wave = th >> 6;
    const long long m = (long long)blockIdx.x * RPB + rl;
    if (m >= rows) return;  // whole rows leave together: the row's barriers stay matched
    const int K = heads * 128;
    float z[VPT][4];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int k0 = 4 * (th + TPR * i);
        if (k0 < K) kea::merged4(ws, rows, heads, m, k0, z[i]);
        else z[i][0] = z[i][1] = z[i][2] = z[i][3] = 0.f;
    }
    quantize_parts<VPT, WPR>(z, K, parts, q, ldq, qs, (int)rows, (int)m, th, red[rl], wave);
}

// GLU + depthwise convolution (as glu_dwconv_kernel, same operation order), SiLU, then the P-part quantization of the
// row: the middle of the convolution module fused with the quantizer of the second pointwise convolution. One
// workgroup (4 waves) per token row; thread th holds the channel chunks 4 * (th + 256 i) .. + 3 (C % 4 == 0).
// KW > 0: compile-time kernel width; every tap's loads are issued before the arithmetic (rows clamped into [0, T) so
// each address is in bounds; taps outside the sequence are then skipped, exactly as in the runtime-width loop).
// GLU = false: x already holds the GLU values (C columns; the GLU ran in the producing GEMM's epilogue with the same
// formula), so the convolution reads them directly.
template <int VPT, int KW, bool GLU>
__global__ void __launch_bounds__(256)
glu_dwconv_quantize_kernel(const float *x, long long ldx, const float *w, const float *bias, int T, int C, int kw_rt,
                           int parts, int8_t *q, long long ldq, float *qs) {
    __shared__ float red[1][7][4];
    const int th = threadIdx.x, wave = th >> 6, t = blockIdx.x, b = blockIdx.y, m = b * T + t;
    const int M = gridDim.y * T;
    const float *xb = x + (long long)b * T * ldx;
    float z[VPT][4];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c0 = 4 * (th + 256 * i);
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        if (c0 < C) {
            if (bias) {
                const float4 bv = *(const float4 *)(bias + c0);
                acc[0] = bv.x; acc[1] = bv.y; acc[2] = bv.z; acc[3] = bv.w;
            }
            if constexpr (KW > 0) {
                constexpr int half = KW / 2;
                float4 a[KW], g[GLU ? KW : 1];
#pragma unroll
                for (int j = 0; j < KW; ++j) {
                    const int tt = min(max(t + j - half, 0), T - 1);
                    a[j] = *(const float4 *)(xb + (long long)tt * ldx + c0);
                    if constexpr (GLU) g[j] = *(const float4 *)(xb + (long long)tt * ldx + C + c0);
                }
                float4 wv[KW];   // w[(c0 + e) * KW + j]: the 4 channels' taps are 4 * KW consecutive floats
                const float *wc = w + (long long)c0 * KW;
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int j = 0; j < KW; ++j) (&wv[j].x)[e] = wc[e * KW + j];
#pragma unroll
                for (int j = 0; j < KW; ++j) {
                    if (t + j - half < 0 || t + j - half >= T) continue;
                    const float av[4] = {a[j].x, a[j].y, a[j].z, a[j].w};
                    const float ww[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
                    if constexpr (GLU) {
                        const float gv[4] = {g[j].x, g[j].y, g[j].z, g[j].w};
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[e] = __builtin_fmaf(ww[e], av[e] * (1.0f / (1.0f + expf(-gv[e]))), acc[e]);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(ww[e], av[e], acc[e]);
                    }
                }
            } else {
                const int half = kw_rt / 2;
                for (int j = 0; j < kw_rt; ++j) {
                    const int tt = t + j - half;
                    if (tt < 0 || tt >= T) continue;
                    const float *row = xb + (long long)tt * ldx;
                    const float4 a = *(const float4 *)(row + c0);
                    const float av[4] = {a.x, a.y, a.z, a.w};
                    if constexpr (GLU) {
                        const float4 g = *(const float4 *)(row + C + c0);
                        const float gv[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[e] = __builtin_fmaf(w[(c0 + e) * kw_rt + j], av[e] * (1.0f / (1.0f + expf(-gv[e]))),
                                                    acc[e]);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(w[(c0 + e) * kw_rt + j], av[e], acc[e]);
                    }
                }
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) z[i][e] = acc[e] * (1.0f / (1.0f + expf(-acc[e])));  // SiLU (0 past C)
    }
    quantize_parts<VPT, 4>(z, C, parts, q, ldq, qs, M, m, th, red[0], wave);
}

// The exact row epilogue: per row m (WPR waves, the quantizer's layout and reduction order), the split-K slices
// summed in slice order (exact int32), the GEMM epilogue (kea::combine / kea::finish: the unsplit kernel's value, bit
// for bit), the residual x = res + value * factor, an optional LayerNorm stored as y, then optionally the P-part
// quantization of LayerNorm(y) for the next projection. The reference's _row_epilogue_exact / _row_epilogue
// (kk/binary/row_exact.py:62-122, kk/ternary/row_fusion.py:27-52).
struct RowParams {
    const int32_t *slices;
    int split, M, N, flags;
    const float *qs;
    long long qs_stride;
    const void *ws, *bias;
    int ws_dtype, bias_dtype;
    const float *res;
    long long ldr;
    float factor;
    const float *ow, *ob;
    float oeps;
    float *y;
    long long ldy;
    const float *nw, *nb;
    float eps;
    int qparts;
    int8_t *q;
    long long ldq;
    float *qsc;
};

template <int P, int VPT, int WPR>
__global__ void __launch_bounds__(256) row_epilogue_kernel(RowParams rp) {
    constexpr int RPB = 4 / WPR, TPR = 64 * WPR;
    constexpr int G = VPT >= 4 ? 1 : (VPT == 2 ? 2 : 4);  // slices whose loads are issued together
    __shared__ float red[RPB][7][WPR];
    const int th = threadIdx.x % TPR, rl = threadIdx.x / TPR, wave = th >> 6, m = blockIdx.x * RPB + rl;
    if (m >= rp.M) return;  // whole rows leave together: the row's barriers stay matched
    const int N = rp.N;
    const long long plane = (long long)rp.M * N;
    int a[VPT][P][4];
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
        for (int c = 0; c < P; ++c) a[i][c][0] = a[i][c][1] = a[i][c][2] = a[i][c][3] = 0;
    for (int z0 = 0; z0 < rp.split; z0 += G) {
        int4 v[G][P][VPT];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int c = 0; c < P; ++c)
#pragma unroll
                for (int i = 0; i < VPT; ++i) {
                    const int n0 = 4 * (th + TPR * i);
                    v[g][c][i] = make_int4(0, 0, 0, 0);
                    if (z0 + g < rp.split && n0 < N)
                        v[g][c][i] = *(const int4 *)(rp.slices + ((long long)(z0 + g) * P + c) * plane +
                                                     (long long)m * N + n0);
                }
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int c = 0; c < P; ++c)
#pragma unroll
                for (int i = 0; i < VPT; ++i) {
                    a[i][c][0] += v[g][c][i].x; a[i][c][1] += v[g][c][i].y;
                    a[i][c][2] += v[g][c][i].z; a[i][c][3] += v[g][c][i].w;
                }
    }
    float s[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) s[c] = c < P ? rp.qs[c * rp.qs_stride + m] : 0.f;
    float z[VPT][4];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int n0 = 4 * (th + TPR * i);
        z[i][0] = z[i][1] = z[i][2] = z[i][3] = 0.f;
        if (n0 < N) {
            float4 r4 = make_float4(0.f, 0.f, 0.f, 0.f);
            if (rp.res) r4 = *(const float4 *)(rp.res + (long long)m * rp.ldr + n0);
            const float res[4] = {r4.x, r4.y, r4.z, r4.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int ar[3] = {a[i][0][e], P > 1 ? a[i][P > 1 ? 1 : 0][e] : 0,
                                   P > 2 ? a[i][P > 2 ? 2 : 0][e] : 0};
                const float alpha = kea::load_scalar(rp.ws, rp.ws_dtype, n0 + e);
                const float b = rp.bias ? kea::load_scalar(rp.bias, rp.bias_dtype, n0 + e) : kea::kNoBias;
                float v = kea::finish(kea::combine<P>(ar, s, rp.flags), alpha, b, rp.flags);
                if (rp.res) v = res[e] + v * rp.factor;
                z[i][e] = v;
            }
        }
    }
    if (rp.ow) layer_norm_row<VPT, WPR>(z, N, rp.ow, rp.ob, rp.oeps, th, red[rl], wave, 5);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int n0 = 4 * (th + TPR * i);
        if (n0 < N) *(float4 *)(rp.y + (long long)m * rp.ldy + n0) = make_float4(z[i][0], z[i][1], z[i][2], z[i][3]);
    }
    if (rp.q) {
        if (rp.nw) layer_norm_row<VPT, WPR>(z, N, rp.nw, rp.nb, rp.eps, th, red[rl], wave, 0);
        quantize_parts<VPT, WPR>(z, N, rp.qparts, rp.q, rp.ldq, rp.qsc, rp.M, m, th, red[rl], wave);
    }
}

}  // namespace

namespace kea {

int quantize_check(int x_dtype, int64_t t, int64_t m, int64_t k, int parts, int64_t ldq, int qs_dtype,
                   const float *norm_w, const float *norm_b) {
    if (parts < 1 || parts > 3) return fail(KEA_EINVAL, "parts must be 1, 2 or 3");
    if (m < 0 || k < 1 || m > INT32_MAX || k > 8192) return fail(KEA_EINVAL, "bad sizes (k must be 1..8192)");
    if (t < 1) return fail(KEA_EINVAL, "t must be >= 1");
    if (ldq < k) return fail(KEA_EINVAL, "ldq < k");
    if (x_dtype != KEA_F32 && x_dtype != KEA_F16) return fail(KEA_EINVAL, "x dtype must be f32 or f16");
    if (qs_dtype != KEA_F32 && qs_dtype != KEA_F16) return fail(KEA_EINVAL, "qs dtype must be f32 or f16");
    if ((norm_w == nullptr) != (norm_b == nullptr)) return fail(KEA_EINVAL, "norm weight and bias go together");
    const int wpr = k > 256 ? 4 : 1;
    if (!fits_dispatch((m + 4 / wpr - 1) / (4 / wpr), 256))
        return fail(KEA_EINVAL, "too large for one launch: split the call along M");
    return KEA_OK;
}

int quantize_enqueue(const void *x, int x_dtype, int64_t xb, int64_t xt, int64_t xk, int64_t t, int64_t m, int64_t k,
                     int parts, const float *norm_w, const float *norm_b, float eps, int input_silu, int8_t *q,
                     int64_t ldq, void *qs, int qs_dtype, void *stream) {
    hipStream_t st = (hipStream_t)stream;
    const int esz = x_dtype == KEA_F16 ? 2 : 4;
    const int wpr = k > 256 ? 4 : 1;               // waves per row (the oracle restates this rule)
    const int vpt = (int)((k + 256 * wpr - 1) / (256 * wpr));
    const bool vec = xk == 1 && k % 4 == 0 && ldq % 4 == 0 && xb % 4 == 0 && xt % 4 == 0 &&
                     ((uintptr_t)x % (4 * esz)) == 0 && ((uintptr_t)q % 4) == 0 &&
                     (((uintptr_t)norm_w | (uintptr_t)norm_b) % 16) == 0;
    const dim3 grid((unsigned)((m + 4 / wpr - 1) / (4 / wpr))), block(256);
#define KEA_Q(V, W)                                                                                                \
    do {                                                                                                           \
        if (vec)                                                                                                   \
            hipLaunchKernelGGL((quantize_kernel<V, W, true>), grid, block, 0, st, x, x_dtype, xb, xt, xk, t,       \
                               (int)m, (int)k, parts, norm_w, norm_b, eps, input_silu, q, ldq, qs, qs_dtype);       \
        else                                                                                                       \
            hipLaunchKernelGGL((quantize_kernel<V, W, false>), grid, block, 0, st, x, x_dtype, xb, xt, xk, t,      \
                               (int)m, (int)k, parts, norm_w, norm_b, eps, input_silu, q, ldq, qs, qs_dtype);       \
    } while (0)
    if (wpr == 1) {
        KEA_Q(1, 1);
    } else {
        if (vpt <= 1) KEA_Q(1, 4);
        else if (vpt <= 2) KEA_Q(2, 4);
        else if (vpt <= 4) KEA_Q(4, 4);
        else KEA_Q(8, 4);
    }
#undef KEA_Q
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail((int)e, std::string("quantize launch failed: ") + hipGetErrorString(e));
    return KEA_OK;
}

}  // namespace kea

extern "C" int kea_quantize(const void *x, int x_dtype, int64_t xb, int64_t xt, int64_t xk, int64_t t, int64_t m,
                            int64_t k, int parts, const float *norm_w, const float *norm_b, float eps,
                            int input_silu, int8_t *q, int64_t ldq, void *qs, int qs_dtype, void *stream) {
    const int rc = kea::quantize_check(x_dtype, t, m, k, parts, ldq, qs_dtype, norm_w, norm_b);
    if (rc != KEA_OK) return rc;
    if (m == 0) return KEA_OK;
    if (!x || !q || !qs) return kea::fail(KEA_EINVAL, "x, q and qs are required");
    return kea::quantize_enqueue(x, x_dtype, xb, xt, xk, t, m, k, parts, norm_w, norm_b, eps, input_silu, q, ldq, qs,
                                 qs_dtype, stream);
}

extern "C" int kea_norm_quantize(const float *x, int64_t ldx, int64_t m, int64_t k, const float *norm0_w,
                                 const float *norm0_b, float eps0, float *x_out, int64_t ldo, const float *norm1_w,
                                 const float *norm1_b, float eps1, int parts, int8_t *q, int64_t ldq, float *qs,
                                 void *stream) {
    if (parts < 1 || parts > 3) return kea::fail(KEA_EINVAL, "parts must be 1, 2 or 3");
    if (m < 0 || k < 4 || k > 4096 || m > INT32_MAX || k % 4) return kea::fail(KEA_EINVAL, "bad sizes (k in 4..4096, k % 4 == 0)");
    if (ldx < k || ldo < k || ldq < k) return kea::fail(KEA_EINVAL, "leading dimension too small");
    if (m == 0) return KEA_OK;
    if (!x || !x_out || !q || !qs || !norm0_w || !norm0_b || !norm1_w || !norm1_b)
        return kea::fail(KEA_EINVAL, "null pointer");
    if (((uintptr_t)x | (uintptr_t)x_out | (uintptr_t)norm0_w | (uintptr_t)norm0_b | (uintptr_t)norm1_w |
         (uintptr_t)norm1_b) & 15 || (ldx | ldo) & 3 || ((uintptr_t)q | (uintptr_t)ldq) & 3)
        return kea::fail(KEA_EALIGN, "rows and norm weights need 16-byte alignment, q rows 4-byte alignment");
    const int wpr = k > 256 ? 4 : 1, vpt = (int)((k + 256 * wpr - 1) / (256 * wpr));
    if (!kea::fits_dispatch((m + 4 / wpr - 1) / (4 / wpr), 256)) return kea::fail(KEA_EINVAL, "too large for one launch: split the call along M");
    const dim3 grid((unsigned)((m + 4 / wpr - 1) / (4 / wpr))), block(256);
    hipStream_t st = (hipStream_t)stream;
#define KEA_NQ(V, W)                                                                                             \
    hipLaunchKernelGGL((norm_quantize_kernel<V, W>), grid, block, 0, st, x, (long long)ldx, (int)m, (int)k,        \
                       norm0_w, norm0_b, eps0, x_out, (long long)ldo, norm1_w, norm1_b, eps1, parts, q,           \
                       (long long)ldq, qs)
    if (wpr == 1) KEA_NQ(1, 1);
    else if (vpt <= 1) KEA_NQ(1, 4);
    else if (vpt <= 2) KEA_NQ(2, 4);
    else KEA_NQ(4, 4);
#undef KEA_NQ
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("norm_quantize launch failed: ") + hipGetErrorString(e));
    return KEA_OK;
}

extern "C" int kea_attention_merge_quantize(const void *workspace, int64_t workspace_bytes, int64_t batch, int64_t t,
                                            int heads, int parts, int8_t *q, int64_t ldq, float *qs, void *stream) {
    if (parts < 1 || parts > 3) return kea::fail(KEA_EINVAL, "parts must be 1, 2 or 3");
    if (batch < 1 || t < 1 || heads < 1 || heads > 32 || batch > 65535)
        return kea::fail(KEA_EINVAL, "bad sizes (heads <= 32)");
    if (!kea::attention_splits(batch, t, heads))
        return kea::fail(KEA_EINVAL, "the key-split attention does not apply to this shape: no halves to merge");
    const long long rows = batch * t, k = (long long)heads * 128;
    if (rows > INT32_MAX) return kea::fail(KEA_EINVAL, "too many rows");
    if (workspace_bytes < 4 * kea::split_ws_floats(rows, heads))
        return kea::fail(KEA_ESPACE, "attention workspace too small");
    if (ldq < k) return kea::fail(KEA_EINVAL, "leading dimension too small");
    if (!workspace || !q || !qs) return kea::fail(KEA_EINVAL, "null pointer");
    if ((uintptr_t)workspace & 15 || ((uintptr_t)q | (uintptr_t)ldq) & 3)
        return kea::fail(KEA_EALIGN, "workspace needs 16-byte alignment, q rows 4-byte alignment");
    const kea::SplitWs sw = kea::split_ws(const_cast<void *>(workspace), rows, heads);
    const int wpr = k > 256 ? 4 : 1, vpt = (int)((k + 256 * wpr - 1) / (256 * wpr));
    if (!kea::fits_dispatch((rows + 4 / wpr - 1) / (4 / wpr), 256)) return kea::fail(KEA_EINVAL, "too large for one launch: split the call along M");
    const dim3 grid((unsigned)((rows + 4 / wpr - 1) / (4 / wpr))), block(256);
    hipStream_t st = (hipStream_t)stream;
#define KEA_MQ(V, W)                                                                                             \
    hipLaunchKernelGGL((attention_merge_quantize_kernel<V, W>), grid, block, 0, st, sw, rows, heads, parts, q,     \
                       (long long)ldq, qs)
    if (wpr == 1) KEA_MQ(1, 1);
    else if (vpt <= 1) KEA_MQ(1, 4);
    else if (vpt <= 2) KEA_MQ(2, 4);
    else KEA_MQ(4, 4);
#undef KEA_MQ
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("merge_quantize launch failed: ") + hipGetErrorString(e));
    return KEA_OK;
}

static int dwconv_quantize(bool glu, const float *x, int64_t ldx, const float *w, const float *bias, int64_t batch,
                           int64_t t, int64_t channels, int kernel, int parts, int8_t *q, int64_t ldq, float *qs,
                           void *stream) {
    if (parts < 1 || parts > 3) return kea::fail(KEA_EINVAL, "parts must be 1, 2 or 3");
    if (batch < 0 || t < 0 || batch > 65535 || t > INT32_MAX || channels < 4 || channels > 2048 || channels % 4 ||
        kernel < 1 || kernel % 2 == 0)
        return kea::fail(KEA_EINVAL, "bad sizes (channels in 4..2048, a multiple of 4; odd kernel width)");
    if (ldx < (glu ? 2 : 1) * channels || ldq < channels) return kea::fail(KEA_EINVAL, "leading dimension too small");
    if (batch == 0 || t == 0) return KEA_OK;
    if (!x || !w || !q || !qs) return kea::fail(KEA_EINVAL, "null pointer");
    if (((uintptr_t)x | (uintptr_t)bias) & 15 || ldx & 3 || ((uintptr_t)q | (uintptr_t)ldq) & 3)
        return kea::fail(KEA_EALIGN, "x rows and bias need 16-byte alignment, q rows 4-byte alignment");
    const int vpt = (int)((channels + 1023) / 1024);
    if (!kea::fits_dispatch(t, 256)) return kea::fail(KEA_EINVAL, "too large for one launch: split the call along T");
    const dim3 grid((unsigned)t, (unsigned)batch), block(256);
    hipStream_t st = (hipStream_t)stream;
#define KEA_GQ(V, W, G)                                                                                          \
    hipLaunchKernelGGL((glu_dwconv_quantize_kernel<V, W, G>), grid, block, 0, st, x, (long long)ldx, w, bias,    \
                       (int)t, (int)channels, kernel, parts, q, (long long)ldq, qs)
#define KEA_GQ_V(W, G)                 \
    do {                               \
        if (vpt <= 1) KEA_GQ(1, W, G); \
        else KEA_GQ(2, W, G);          \
    } while (0)
    if (glu) {
        if (kernel == 9) KEA_GQ_V(9, true);
        else KEA_GQ_V(0, true);
    } else {
        if (kernel == 9) KEA_GQ_V(9, false);
        else KEA_GQ_V(0, false);
    }
#undef KEA_GQ_V
#undef KEA_GQ
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("dwconv_quantize launch failed: ") + hipGetErrorString(e));
    return KEA_OK;
}

extern "C" int kea_glu_dwconv_quantize(const float *x, int64_t ldx, const float *w, const float *bias, int64_t batch,
                                       int64_t t, int64_t channels, int kernel, int parts, int8_t *q, int64_t ldq,
                                       float *qs, void *stream) {
    return dwconv_quantize(true, x, ldx, w, bias, batch, t, channels, kernel, parts, q, ldq, qs, stream);
}

extern "C" int kea_dwconv_quantize(const float *u, int64_t ldu, const float *w, const float *bias, int64_t batch,
                                   int64_t t, int64_t channels, int kernel, int parts, int8_t *q, int64_t ldq,
                                   float *qs, void *stream) {
    return dwconv_quantize(false, u, ldu, w, bias, batch, t, channels, kernel, parts, q, ldq, qs, stream);
}

extern "C" int kea_row_epilogue(const int32_t *slices, int split, int parts, int64_t m, int64_t n, const float *qs,
                                int64_t qs_stride, const void *wscale, int ws_dtype, const void *bias, int bias_dtype,
                                int flags, const float *residual, int64_t ldr, float factor, const float *out_norm_w,
                                const float *out_norm_b, float out_eps, float *y, int64_t ldy, const float *norm_w,
                                const float *norm_b, float eps, int q_parts, int8_t *q, int64_t ldq, float *q_scales,
                                void *stream) {
    if (split < 1 || parts < 1 || parts > 3) return kea::fail(KEA_EINVAL, "split must be >= 1 and parts 1, 2 or 3");
    if (m < 0 || n < 4 || n > 4096 || n % 4 || m > INT32_MAX)
        return kea::fail(KEA_EINVAL, "bad sizes (n in 4..4096, a multiple of 4)");
    if (flags & ~(KEA_FLAG_SILU | KEA_FLAG_ORDER)) return kea::fail(KEA_EINVAL, "unknown flags");
    if (ws_dtype != KEA_F32 && ws_dtype != KEA_F16) return kea::fail(KEA_EINVAL, "wscale dtype must be f32 or f16");
    if (bias && bias_dtype != KEA_F32 && bias_dtype != KEA_F16) return kea::fail(KEA_EINVAL, "bias dtype must be f32 or f16");
    if ((out_norm_w == nullptr) != (out_norm_b == nullptr) || (norm_w == nullptr) != (norm_b == nullptr))
        return kea::fail(KEA_EINVAL, "LayerNorm weight and bias go together");
    if (norm_w && !q) return kea::fail(KEA_EINVAL, "a LayerNorm for the next projection needs q");
    if (q && (q_parts < 1 || q_parts > 3 || !q_scales || ldq < n || ldq % 4))
        return kea::fail(KEA_EINVAL, "q needs q_parts 1..3, q_scales and ldq >= n, ldq % 4 == 0");
    if (ldy < n || (residual && ldr < n) || (parts > 1 && qs_stride < m)) return kea::fail(KEA_EINVAL, "leading dimension too small");
    if (m == 0) return KEA_OK;
    if (!slices || !qs || !wscale || !y) return kea::fail(KEA_EINVAL, "slices, qs, wscale and y are required");
    if (((uintptr_t)slices | (uintptr_t)y | (uintptr_t)residual | (uintptr_t)out_norm_w | (uintptr_t)out_norm_b |
         (uintptr_t)norm_w | (uintptr_t)norm_b) & 15 || (ldy | (residual ? ldr : 0)) & 3 || (uintptr_t)q & 3)
        return kea::fail(KEA_EALIGN, "slices, y, residual and LayerNorm weights need 16-byte alignment");
    RowParams rp = {};
    rp.slices = slices; rp.split = split; rp.M = (int)m; rp.N = (int)n; rp.flags = flags;
    rp.qs = qs; rp.qs_stride = qs_stride; rp.ws = wscale; rp.ws_dtype = ws_dtype;
    rp.bias = bias; rp.bias_dtype = bias_dtype;
    rp.res = residual; rp.ldr = ldr; rp.factor = factor;
    rp.ow = out_norm_w; rp.ob = out_norm_b; rp.oeps = out_eps;
    rp.y = y; rp.ldy = ldy;
    rp.nw = norm_w; rp.nb = norm_b; rp.eps = eps;
    rp.qparts = q_parts; rp.q = q; rp.ldq = ldq; rp.qsc = q_scales;
    const int wpr = n > 256 ? 4 : 1, vpt = (int)((n + 256 * wpr - 1) / (256 * wpr));
    if (!kea::fits_dispatch((m + 4 / wpr - 1) / (4 / wpr), 256)) return kea::fail(KEA_EINVAL, "too large for one launch: split the call along M");
    const dim3 grid((unsigned)((m + 4 / wpr - 1) / (4 / wpr))), block(256);
    hipStream_t st = (hipStream_t)stream;
#define KEA_RE(P_, V, W) hipLaunchKernelGGL((row_epilogue_kernel<P_, V, W>), grid, block, 0, st, rp)
#define KEA_RE_P(P_)                         \
    do {                                     \
        if (wpr == 1) KEA_RE(P_, 1, 1);      \
        else if (vpt <= 1) KEA_RE(P_, 1, 4); \
        else if (vpt <= 2) KEA_RE(P_, 2, 4); \
        else KEA_RE(P_, 4, 4);               \
    } while (0)
    if (parts == 1) KEA_RE_P(1);
    else if (parts == 2) KEA_RE_P(2);
    else KEA_RE_P(3);
#undef KEA_RE_P
#undef KEA_RE
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("row epilogue launch failed: ") + hipGetErrorString(e));
    return KEA_OK;
}
