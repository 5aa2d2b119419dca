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

// Weight scale and bias, then the optional SiLU (kk/binary/kernels.py:73-93).
__device__ __forceinline__ float finish(float r, float alpha, bool has_bias, float b, int flags) {
    r = has_bias ? __builtin_fmaf(r, alpha, b) : r * alpha;
    if (flags & KEA_FLAG_SILU) r = r / (1.0f + expf(-r));
    return r;
}

}  // namespace kea
