// The per-element step of the residual int8 activation quantizer, shared by the quantizer kernels of kea_quantize.hip
// (the plain row quantizer and the fused LayerNorm / GLU-convolution / attention-merge quantizers), so all of them
// produce the same codes.
// Translation units that include it are built with -ffp-contract=off.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace kea {

// rint(z / s) with z / s the IEEE quotient, without a division per element: q = z * inv (inv = 1 / s, correctly
// rounded) is corrected once with the residual, r = fma(-q, s, z), q' = fma(r, inv, q), which is the correctly rounded
// quotient (Markstein's correction step for division with a fused multiply-add). Where the residual would underflow,
// |z / s| < 1 / 4 and both round to 0.
__device__ __forceinline__ float round_quotient(float z, float s, float inv) {
    const float q = z * inv;
    return rintf(fmaf(fmaf(-q, s, z), inv, q));
}

// The int8 code of z in a part of scale s (inv = 1 / s), clamped to [-127, 127], as the low byte of the result; z
// becomes the residual z - code * s that the next part quantizes.
__device__ __forceinline__ uint32_t quantize_code(float &z, float s, float inv) {
    const float v = fminf(fmaxf(round_quotient(z, s, inv), -127.0f), 127.0f);
    z = z - v * s;
    return (uint32_t)(uint8_t)(int8_t)(int)v;
}

}  // namespace kea
