// The FP32 epilogue arithmetic shared by the GEMM kernels and the row epilogue: one definition, so a value finished
// in either place is the same bits. Translation units that include it are built with -ffp-contract=off.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/kea_lowbit.h"

namespace kea {

__device__ __forceinline__ float load_scalar(const void *p, int dtype, long long i) {
    if (dtype == KEA_F16) return (float)(((const _Float16 *)p)[i]);
    return ((const float *)p)[i];
}

// The reference's P-part combination (comb<P>, kk/binary/kernels_parts.py:28-39): each * is one IEEE multiply, each
// fma an explicit fused multiply-add.
template <int P>
__device__ __forceinline__ float combine(const int *a, const float *s, int flags) {
    if constexpr (P == 1) {
        return (float)a[0] * s[0];
    } else {
        float r = (flags & KEA_FLAG_ORDER) ? __builtin_fmaf((float)a[1], s[1], (float)a[0] * s[0])
                                           : __builtin_fmaf((float)a[0], s[0], (float)a[1] * s[1]);
        if constexpr (P == 3) r = __builtin_fmaf((float)a[2], s[2], r);
        return r;
    }
}

// SiLU of the epilogue, r * sigmoid(r), on the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32, about 1 ulp
// each): the reference's epilogue SiLU is itself approximate (ex2.approx and div.full, kk/binary/kernels.py:82), so
// this value is held to a tolerance against an FP64 SiLU, not to bits. r = -inf gives NaN, as r / (1 + exp(-r)) does.
__device__ __forceinline__ float silu_epilogue(float r) {
    return r * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(r * -1.4426950408889634f));
}

// Weight scale and bias, then the optional SiLU (kk/binary/kernels.py:73-93): bias ? fma(r, alpha, bias) : r * alpha.
// Both forms are one fma here: `b` is the bias, or kNoBias (-0.0f) for none, and fma(r, alpha, -0) is bitwise r * alpha
// (the exact product plus -0 is the exact product, also when that is +0, -0, a denormal, an infinity or a NaN).
constexpr float kNoBias = -0.0f;
__device__ __forceinline__ float finish(float r, float alpha, float b, int flags) {
    r = __builtin_fmaf(r, alpha, b);
    if (flags & KEA_FLAG_SILU) r = silu_epilogue(r);
    return r;
}
// The same value with the two cases as written (a select between the fma and the product). Small GEMM tiles keep
// this form: their launches measured about 1% faster with it (instruction layout), the values are identical.
__device__ __forceinline__ float finish(float r, float alpha, bool has_bias, float b, int flags) {
    r = has_bias ? __builtin_fmaf(r, alpha, b) : r * alpha;
    if (flags & KEA_FLAG_SILU) r = silu_epilogue(r);
    return r;
}

}  // namespace kea
