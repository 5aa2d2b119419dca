// Internal helpers shared by the library's translation units: the thread-local error message.
#pragma once

#include <string>

#include "../../include/kea_lowbit.h"

namespace kea {

// Records `message` as the calling thread's last error and returns `code` (a KEA_E* value or a hipError_t).
int fail(int code, const std::string &message);

// The 1-bit native layout is two parts (include/kea_lowbit.h): the word layout of 16-row n-tiles (read by the
// LDS-ring and per-group kernels), then the bit-plane layout of 128-row groups (read by the wave-split kernel).
// Word offset of the bit-plane part, and its size in words: 16 bytes per lane per group per k-step of 64.
inline long long b1_plane_offset(long long n, long long k) { return (n + 15) / 16 * ((k + 127) / 128) * 64; }
inline long long b1_plane_words(long long n, long long k) { return (n + 127) / 128 * ((k + 63) / 64) * 64 * 4; }

// A dispatch packet holds each grid dimension as a 32-bit count of work-items: `blocks` workgroups of `threads`
// work-items along one dimension must stay within it, or the launch would be truncated and leave work undone.
inline bool fits_dispatch(long long blocks, long long threads) {
    return blocks >= 0 && blocks * threads <= 0xFFFFFFFFLL;
}

// kea_quantize in two steps: the checks that depend on no pointer (KEA_OK or the error kea_quantize returns), and
// the launch for arguments that passed them with m >= 1 and x, q, qs present (kea_quantize.hip).
int quantize_check(int x_dtype, int64_t t, int64_t m, int64_t k, int parts, int64_t ldq, int qs_dtype,
                   const float *norm_w, const float *norm_b);
int quantize_enqueue(const void *x, int x_dtype, int64_t xb, int64_t xt, int64_t xk, int64_t t, int64_t m, int64_t k,
                     int parts, const float *norm_w, const float *norm_b, float eps, int input_silu, int8_t *q,
                     int64_t ldq, void *qs, int qs_dtype, void *stream);

}  // namespace kea
