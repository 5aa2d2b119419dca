// Host-side conversions between the export weight codes and the gfx950 native word layouts.
//
// The export layouts are the reference's on-disk formats (kk/binary/bits.py:3-5, kk/formats.py:5-7); the native
// layouts are this library's own (declared in include/kea_lowbit.h). Their role matches the reference's one-time
// `relayout` (kk/binary/kernels.py:730-742) and the ternary `packed_t` transposition (kk/ternary/runtime.py:33-35):
// rearrange the codes once so that the GEMM reads each wavefront's weights with one coalesced 128-bit load per lane
// and expands them to int8 MFMA operands with a mask and a byte permute (the word part) or with a mask alone (the
// bit-plane part of the 1-bit layout, which the wave-split kernel reads).
#include <cstdint>
#include <cstring>
#include <string>

#include "kea_internal.h"

namespace {

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Index of word j of lane l of n-tile t in the quad-major native layout.
inline int64_t word_index(int64_t t, int64_t j, int l, int64_t J) {
    const int64_t jq = j / 4;
    const int64_t wq = (J - 4 * jq) < 4 ? (J - 4 * jq) : 4;
    return t * J * 64 + jq * 256 + (int64_t)l * wq + (j - 4 * jq);
}

bool sizes_ok(int64_t n, int64_t k) { return n >= 1 && k >= 1 && n <= (int64_t(1) << 31) && k <= (int64_t(1) << 31); }

}  // namespace

extern "C" {

int64_t kea_b1_native_words(int64_t n, int64_t k) {
    if (!sizes_ok(n, k)) return 0;
    return kea::b1_plane_offset(n, k) + kea::b1_plane_words(n, k);
}

int64_t kea_t2_native_words(int64_t n, int64_t k) {
    if (!sizes_ok(n, k)) return 0;
    return cdiv(n, 16) * cdiv(k, 64) * 64;
}

int kea_b1_relayout_host(const uint8_t *codes, int64_t n, int64_t k, uint32_t *words) {
    if (!sizes_ok(n, k) || !codes || !words) return kea::fail(KEA_EINVAL, "kea_b1_relayout_host: bad arguments");
    const int64_t row_bytes = cdiv(k, 8), J = cdiv(k, 128), NT = cdiv(n, 16);
    const int tail = (int)(8 * row_bytes - k);
    if (tail) {
        const uint8_t mask = (uint8_t)(0xFFu << (8 - tail));
        for (int64_t r = 0; r < n; ++r)
            if (codes[r * row_bytes + row_bytes - 1] & mask)
                return kea::fail(KEA_ECODES, "invalid packed codes: nonzero tail padding (row " + std::to_string(r) + ")");
    }
    std::memset(words, 0, sizeof(uint32_t) * NT * J * 64);
    for (int64_t t = 0; t < NT; ++t)
        for (int64_t j = 0; j < J; ++j)
            for (int l = 0; l < 64; ++l) {
                const int64_t row = 16 * t + (l % 16);
                if (row >= n) continue;
                const uint8_t *src = codes + row * row_bytes;
                uint32_t word = 0;
                for (int h = 0; h < 2; ++h)
                    for (int d = 0; d < 4; ++d)
                        for (int i = 0; i < 4; ++i) {
                            const int64_t kk = 128 * j + 64 * h + 16 * (l / 16) + 4 * d + i;
                            // padding (kk >= K) stays 0, i.e. +1: the kernel masks activations there to 0
                            if (kk < k && !((src[kk >> 3] >> (kk & 7)) & 1)) word |= 1u << (8 * i + 4 * h + d);
                        }
                words[word_index(t, j, l, J)] = word;
            }
    // the bit-plane part: unit (group g, k-step s, lane l) = 4 words; bit p of byte 4d + i of the unit is the
    // inverted sign of w[128g + 16p + l%16][64s + 16(l/16) + 4d + i] (rows and k past the matrix: 0). A lane's 16 k of
    // one row are two code bytes; their inverted bits 4d .. 4d+3 spread to bits 0, 8, 16, 24 of word d.
    static const uint32_t spread4[16] = {0x00000000u, 0x00000001u, 0x00000100u, 0x00000101u, 0x00010000u, 0x00010001u,
                                         0x00010100u, 0x00010101u, 0x01000000u, 0x01000001u, 0x01000100u, 0x01000101u,
                                         0x01010000u, 0x01010001u, 0x01010100u, 0x01010101u};
    uint32_t *planes = words + kea::b1_plane_offset(n, k);
    const int64_t NG = cdiv(n, 128), KS = cdiv(k, 64);
    std::memset(planes, 0, sizeof(uint32_t) * kea::b1_plane_words(n, k));
    for (int64_t g = 0; g < NG; ++g)
        for (int64_t s = 0; s < KS; ++s)
            for (int l = 0; l < 64; ++l) {
                uint32_t *unit = planes + ((g * KS + s) * 64 + l) * 4;
                const int64_t k0 = 64 * s + 16 * (l / 16);  // the lane's first k (a multiple of 16)
                if (k0 >= k) continue;
                const uint32_t valid = k - k0 >= 16 ? 0xFFFFu : (1u << (k - k0)) - 1u;
                for (int p = 0; p < 8; ++p) {
                    const int64_t row = 128 * g + 16 * p + (l % 16);
                    if (row >= n) continue;
                    const uint8_t *src = codes + row * row_bytes + k0 / 8;
                    const uint32_t bits = src[0] | (k0 / 8 + 1 < row_bytes ? (uint32_t)src[1] << 8 : 0u);
                    const uint32_t inv = ~bits & valid;
                    for (int d = 0; d < 4; ++d) unit[d] |= spread4[(inv >> (4 * d)) & 15u] << p;
                }
            }
    return KEA_OK;
}

int kea_b1_unlayout_host(const uint32_t *words, int64_t n, int64_t k, uint8_t *codes) {
    if (!sizes_ok(n, k) || !codes || !words) return kea::fail(KEA_EINVAL, "kea_b1_unlayout_host: bad arguments");
    const int64_t row_bytes = cdiv(k, 8), J = cdiv(k, 128);
    std::memset(codes, 0, (size_t)(n * row_bytes));
    for (int64_t row = 0; row < n; ++row)
        for (int64_t kk = 0; kk < k; ++kk) {
            const int64_t j = kk / 128;
            const int r = (int)(kk % 128), h = r / 64, g = (r % 64) / 16, d = (r % 16) / 4, i = r % 4;
            const int l = (int)(row % 16) + 16 * g;
            const uint32_t word = words[word_index(row / 16, j, l, J)];
            if (!((word >> (8 * i + 4 * h + d)) & 1)) codes[row * row_bytes + (kk >> 3)] |= (uint8_t)(1u << (kk & 7));
        }
    return KEA_OK;
}

int kea_t2_relayout_host(const uint8_t *codes, int64_t n, int64_t k, uint32_t *words) {
    if (!sizes_ok(n, k) || !codes || !words) return kea::fail(KEA_EINVAL, "kea_t2_relayout_host: bad arguments");
    const int64_t row_bytes = cdiv(k, 4), J = cdiv(k, 64), NT = cdiv(n, 16);
    for (int64_t r = 0; r < n; ++r)
        for (int64_t b = 0; b < row_bytes; ++b) {
            const uint8_t v = codes[r * row_bytes + b];
            for (int f = 0; f < 4; ++f) {
                const int c = (v >> (2 * f)) & 3;
                if (c == 3 || (c != 0 && 4 * b + f >= k))
                    return kea::fail(KEA_ECODES, "invalid packed codes (row " + std::to_string(r) + ")");
            }
        }
    std::memset(words, 0, sizeof(uint32_t) * NT * J * 64);
    for (int64_t t = 0; t < NT; ++t)
        for (int64_t j = 0; j < J; ++j)
            for (int l = 0; l < 64; ++l) {
                const int64_t row = 16 * t + (l % 16);
                if (row >= n) continue;
                const uint8_t *src = codes + row * row_bytes;
                uint32_t word = 0;
                for (int d = 0; d < 4; ++d)
                    for (int i = 0; i < 4; ++i) {
                        const int64_t kk = 64 * j + 16 * (l / 16) + 4 * d + i;
                        if (kk >= k) continue;
                        const uint32_t c = (src[kk >> 2] >> (2 * (kk & 3))) & 3u;
                        word |= c << (8 * i + 2 * d);
                    }
                words[word_index(t, j, l, J)] = word;
            }
    return KEA_OK;
}

int kea_t2_unlayout_host(const uint32_t *words, int64_t n, int64_t k, uint8_t *codes) {
    if (!sizes_ok(n, k) || !codes || !words) return kea::fail(KEA_EINVAL, "kea_t2_unlayout_host: bad arguments");
    const int64_t row_bytes = cdiv(k, 4), J = cdiv(k, 64);
    std::memset(codes, 0, (size_t)(n * row_bytes));
    for (int64_t row = 0; row < n; ++row)
        for (int64_t kk = 0; kk < k; ++kk) {
            const int64_t j = kk / 64;
            const int r = (int)(kk % 64), g = r / 16, d = (r % 16) / 4, i = r % 4;
            const int l = (int)(row % 16) + 16 * g;
            const uint32_t c = (words[word_index(row / 16, j, l, J)] >> (8 * i + 2 * d)) & 3u;
            codes[row * row_bytes + (kk >> 2)] |= (uint8_t)(c << (2 * (kk & 3)));
        }
    return KEA_OK;
}

}  // extern "C"
