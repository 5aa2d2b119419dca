// Residual int8 activation quantizer with optional fused LayerNorm and input SiLU (one wavefront per token row).
//
// Semantics follow the reference's quantizers (kk/binary/kernels.py:567-616 and the Triton `_quantize`,
// kk/ternary/fused_kernels.py:31-50):
//     z = x ; z = LayerNorm(z) * w + b (optional) ; z = z * sigmoid(z) (optional)
//     for c < P:  s_c = max(max|z| / 127, 1e-30) ; q_c = rint(z / s_c) ; z = z - q_c * s_c
// with IEEE division and round-half-even (the reference's `div.full` / `ex2.approx` NVIDIA approximations are not
// reproduced). Reductions that are not exact (the LayerNorm sums) use one fixed order that the CPU oracle restates:
// each lane sums its elements k = lane, lane + 64, ... in increasing k, then a xor butterfly over 64 lanes with
// offsets 32, 16, ..., 1. The max reductions are exact in any order. With fp16 scales the scale is rounded to fp16
// (kept >= the smallest fp16 subnormal, <= the largest finite fp16) before use and q is clamped to [-127, 127].
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "kea_internal.h"

namespace {

constexpr int kRowsPerBlock = 4;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ float load_x(const void *x, int dtype, long long i) {
    if (dtype == KEA_F16) return (float)(((const _Float16 *)x)[i]);
    return ((const float *)x)[i];
}

// CPL: elements per lane held in registers (K <= 64 * CPL).
template <int CPL>
__global__ void __launch_bounds__(64 * kRowsPerBlock)
quantize_kernel(const void *x, int x_dtype, long long xb, long long xt, long long xk, long long t, int M, int K,
                int parts, const float *nw, const float *nb, float eps, int input_silu, int8_t *q, long long ldq,
                void *qs, int qs_dtype) {
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (m >= M) return;
    const long long base = (long long)(m / t) * xb + (long long)(m % t) * xt;
    float z[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int k = lane + 64 * i;
        z[i] = k < K ? load_x(x, x_dtype, base + (long long)k * xk) : 0.f;
    }
    if (nw) {
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i)
            if (lane + 64 * i < K) sum = sum + z[i];
        const float mean = wave_sum(sum) / (float)K;
        float sq = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int k = lane + 64 * i;
            z[i] = k < K ? z[i] - mean : 0.f;
            sq = sq + z[i] * z[i];
        }
        const float var = wave_sum(sq) / (float)K;
        const float inv = 1.0f / sqrtf(var + eps);
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int k = lane + 64 * i;
            if (k < K) z[i] = z[i] * inv * nw[k] + nb[k];
        }
    }
    if (input_silu) {
#pragma unroll
        for (int i = 0; i < CPL; ++i) z[i] = z[i] * (1.0f / (1.0f + expf(-z[i])));
    }
    for (int c = 0; c < parts; ++c) {
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i)
            if (lane + 64 * i < K) amax = fmaxf(amax, fabsf(z[i]));
        amax = wave_max(amax);
        float s = fmaxf(amax / 127.0f, 1.0e-30f);
        if (qs_dtype == KEA_F16) {
            _Float16 h = (_Float16)s;
            float hs = (float)h;
            hs = fmaxf(hs, 5.9604644775390625e-08f);  // 2^-24, the smallest fp16 subnormal
            hs = fminf(hs, 65504.0f);
            s = hs;
            if (lane == 0) ((_Float16 *)qs)[(long long)c * M + m] = (_Float16)s;
        } else if (lane == 0) {
            ((float *)qs)[(long long)c * M + m] = s;
        }
        int8_t *row = q + ((long long)c * M + m) * ldq;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int k = lane + 64 * i;
            if (k < K) {
                float v = rintf(z[i] / s);
                v = fminf(fmaxf(v, -127.0f), 127.0f);
                row[k] = (int8_t)(int)v;
                z[i] = z[i] - v * s;
            }
        }
        for (long long k = K + lane; k < ldq; k += 64) row[k] = 0;
    }
}

}  // namespace

extern "C" int kea_quantize(const void *x, int x_dtype, int64_t xb, int64_t xt, int64_t xk, int64_t t, int64_t m,
                            int64_t k, int parts, const float *norm_w, const float *norm_b, float eps,
                            int input_silu, int8_t *q, int64_t ldq, void *qs, int qs_dtype, void *stream) {
    if (parts < 1 || parts > 3) return kea::fail(KEA_EINVAL, "parts must be 1, 2 or 3");
    if (m < 0 || k < 1 || m > INT32_MAX || k > 8192) return kea::fail(KEA_EINVAL, "bad sizes (k must be 1..8192)");
    if (t < 1) return kea::fail(KEA_EINVAL, "t must be >= 1");
    if (ldq < k) return kea::fail(KEA_EINVAL, "ldq < k");
    if (x_dtype != KEA_F32 && x_dtype != KEA_F16) return kea::fail(KEA_EINVAL, "x dtype must be f32 or f16");
    if (qs_dtype != KEA_F32 && qs_dtype != KEA_F16) return kea::fail(KEA_EINVAL, "qs dtype must be f32 or f16");
    if ((norm_w == nullptr) != (norm_b == nullptr)) return kea::fail(KEA_EINVAL, "norm weight and bias go together");
    if (m == 0) return KEA_OK;
    if (!x || !q || !qs) return kea::fail(KEA_EINVAL, "x, q and qs are required");
    const dim3 grid((unsigned)((m + kRowsPerBlock - 1) / kRowsPerBlock)), block(64 * kRowsPerBlock);
    hipStream_t st = (hipStream_t)stream;
    const int cpl = (int)((k + 63) / 64);
#define KEA_Q(N)                                                                                                  \
    hipLaunchKernelGGL(quantize_kernel<N>, grid, block, 0, st, x, x_dtype, xb, xt, xk, t, (int)m, (int)k, parts, \
                       norm_w, norm_b, eps, input_silu, q, ldq, qs, qs_dtype)
    if (cpl <= 4) KEA_Q(4);
    else if (cpl <= 16) KEA_Q(16);
    else if (cpl <= 64) KEA_Q(64);
    else KEA_Q(128);
#undef KEA_Q
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("quantize launch failed: ") + hipGetErrorString(e));
    return KEA_OK;
}
