/*
 * kea_oracle.c - CPU restatement of the reference's low-bit GEMM arithmetic. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and only as the
 * checker (or the timed CPU baseline). The product path (libkea_hip.so) never calls it.
 *
 * Every function works on the reference's EXPORT layouts (never the GPU's native words) and follows:
 *   oracle_b1_gemm      b1_fallback's loop (kk/binary/kernels.py:619-637): sign = bit ? +1 : -1, int32 sums per part
 *   oracle_t2_gemm      the 2-bit decode (c & 1) - (c >> 1) (kk/ternary/fused_kernels.py:92-96, kk/formats.py:73-81)
 *   oracle_epilogue     comb<P> + epilogue (kk/binary/kernels_parts.py:28-39, kk/binary/kernels.py:76-93) with IEEE
 *                       fp32 ops in the written order (this file is built with -ffp-contract=off), SiLU as
 *                       r / (1 + expf(-r)) (the reference's ex2.approx / div.full are NVIDIA approximations that are
 *                       deliberately not reproduced), and the library's per-group rule for ws_group > 0
 *   oracle_quantize     the residual quantizer (kk/binary/kernels.py:567-616, kk/ternary/fused_kernels.py:31-50) with
 *                       IEEE division, rint (round half to even) and the library's fixed LayerNorm summation order
 *   oracle_f32_to_f16 / oracle_f32_to_bf16   IEEE round-to-nearest-even conversions, written out bit by bit
 * Groups: acc has layout [G][P][M][N] where G = ceil(K / group) and group = K gives one group.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define EXPORT __attribute__((visibility("default")))

EXPORT int oracle_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

static inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

/* int8 . int8 dot product of one activation row with one decoded weight row over [k0, k1). */
__attribute__((target_clones("avx2", "default")))
static int32_t dot_i8(const int8_t *a, const int8_t *w, int64_t k0, int64_t k1) {
    int32_t s = 0;
    for (int64_t k = k0; k < k1; ++k) s += (int32_t)a[k] * (int32_t)w[k];
    return s;
}

static void gemm_rows(const int8_t *q, int64_t part_stride, int64_t ldq, int parts, const int8_t *wrow, int64_t nidx,
                      int64_t n, int64_t k, int64_t m, int64_t group, int32_t *acc) {
    const int64_t G = cdiv(k, group);
    for (int64_t g = 0; g < G; ++g) {
        const int64_t k0 = g * group, k1 = (k0 + group < k) ? k0 + group : k;
        for (int c = 0; c < parts; ++c)
            for (int64_t r = 0; r < m; ++r) {
                const int8_t *a = q + c * part_stride + r * ldq;
                acc[((g * parts + c) * m + r) * n + nidx] = dot_i8(a, wrow, k0, k1);
            }
    }
}

/* 1-bit: codes uint8 [n][ceil(k/8)], bit k%8 of byte k/8, 1 = +1, 0 = -1. acc int32 [G][parts][m][n]. */
EXPORT int oracle_b1_gemm(const int8_t *q, int64_t part_stride, int64_t ldq, int parts, const uint8_t *codes,
                          int64_t n, int64_t k, int64_t m, int64_t group, int32_t *acc) {
    if (parts < 1 || parts > 3 || n < 1 || k < 1 || m < 0 || group < 1) return -1;
    const int64_t rb = cdiv(k, 8);
#pragma omp parallel
    {
        int8_t *wrow = (int8_t *)__builtin_alloca((size_t)k);
#pragma omp for schedule(static)
        for (int64_t j = 0; j < n; ++j) {
            const uint8_t *src = codes + j * rb;
            for (int64_t kk = 0; kk < k; ++kk) wrow[kk] = ((src[kk >> 3] >> (kk & 7)) & 1) ? 1 : -1;
            gemm_rows(q, part_stride, ldq, parts, wrow, j, n, k, m, group, acc);
        }
    }
    return 0;
}

/* 2-bit: codes uint8 [n][ceil(k/4)], code k at bits 2(k%4) of byte k/4: 00 = 0, 01 = +1, 10 = -1. */
EXPORT int oracle_t2_gemm(const int8_t *q, int64_t part_stride, int64_t ldq, int parts, const uint8_t *codes,
                          int64_t n, int64_t k, int64_t m, int64_t group, int32_t *acc) {
    if (parts < 1 || parts > 3 || n < 1 || k < 1 || m < 0 || group < 1) return -1;
    const int64_t rb = cdiv(k, 4);
#pragma omp parallel
    {
        int8_t *wrow = (int8_t *)__builtin_alloca((size_t)k);
#pragma omp for schedule(static)
        for (int64_t j = 0; j < n; ++j) {
            const uint8_t *src = codes + j * rb;
            for (int64_t kk = 0; kk < k; ++kk) {
                const int c = (src[kk >> 2] >> (2 * (kk & 3))) & 3;
                wrow[kk] = (int8_t)((c & 1) - (c >> 1));
            }
            gemm_rows(q, part_stride, ldq, parts, wrow, j, n, k, m, group, acc);
        }
    }
    return 0;
}

/* comb<P>: P = 1: f(a0)*s0; P = 2: fma(f(a0), s0, f(a1)*s1) (order 1: fma(f(a1), s1, f(a0)*s0)); P = 3: fma(f(a2), s2, .) */
static float combine(int parts, const int32_t *a, const float *s, int flags) {
    if (parts == 1) return (float)a[0] * s[0];
    float r = (flags & 2) ? fmaf((float)a[1], s[1], (float)a[0] * s[0]) : fmaf((float)a[0], s[0], (float)a[1] * s[1]);
    if (parts == 3) r = fmaf((float)a[2], s[2], r);
    return r;
}

/*
 * acc int32 [G][parts][m][n]; qs f32 [parts][m]; alpha f32 [n] (groups == 1 and group_scales == 0) or [n][G]
 * (group_scales != 0); bias f32 [n] or NULL; out f32 [m][n].
 *   per-channel: r = comb(acc); r = bias ? fma(r, alpha, bias) : r * alpha
 *   per-group:   r = 0; for g: r = fma(comb(acc_g), alpha[n][g], r); r = bias ? r + bias : r
 *   SiLU:        r = r / (1 + expf(-r))
 */
EXPORT int oracle_epilogue(const int32_t *acc, int64_t groups, int parts, int64_t m, int64_t n, const float *qs,
                           const float *alpha, int group_scales, const float *bias, int flags, float *out) {
    if (parts < 1 || parts > 3 || groups < 1 || (!group_scales && groups != 1)) return -1;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; ++r) {
        float s[3] = {0.f, 0.f, 0.f};
        for (int c = 0; c < parts; ++c) s[c] = qs[c * m + r];
        for (int64_t j = 0; j < n; ++j) {
            float v;
            if (!group_scales) {
                int32_t a[3] = {0, 0, 0};
                for (int c = 0; c < parts; ++c) a[c] = acc[(c * m + r) * n + j];
                v = combine(parts, a, s, flags);
                v = bias ? fmaf(v, alpha[j], bias[j]) : v * alpha[j];
            } else {
                v = 0.f;
                for (int64_t g = 0; g < groups; ++g) {
                    int32_t a[3] = {0, 0, 0};
                    for (int c = 0; c < parts; ++c) a[c] = acc[((g * parts + c) * m + r) * n + j];
                    v = fmaf(combine(parts, a, s, flags), alpha[j * groups + g], v);
                }
                if (bias) v = v + bias[j];
            }
            if (flags & 1) v = v / (1.0f + expf(-v));
            out[r * n + j] = v;
        }
    }
    return 0;
}

/* IEEE binary32 -> binary16, round to nearest, ties to even; overflow -> inf; NaN stays NaN. */
static uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu)); /* NaN */
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
    const int exp = (int)(ax >> 23) - 127;
    if (exp >= -14) { /* normal half */
        uint32_t mant = ax & 0x7FFFFFu;
        uint32_t h = ((uint32_t)(exp + 15) << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1; /* carries into the exponent correctly */
        return (uint16_t)(sign | h);
    }
    if (exp < -25) return (uint16_t)sign; /* below half the smallest subnormal: 0 (exactly half is exp == -25) */
    /* subnormal half: value / 2^-24 = mant24 * 2^(exp + 1), exp + 1 in [-24, -14]; a carry out of the
     * subnormal range yields the smallest normal encoding, which is correct */
    const uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
    const int sh = -(exp + 1);
    const uint32_t whole = mant >> sh;
    const uint32_t rem = mant & ((1u << sh) - 1u);
    const uint32_t half = 1u << (sh - 1);
    uint32_t res = whole;
    if (rem > half || (rem == half && (whole & 1u))) res += 1;
    return (uint16_t)(sign | res);
}

/* IEEE binary32 -> bfloat16, round to nearest, ties to even; NaN stays NaN. */
static uint16_t f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    const uint32_t lsb = (x >> 16) & 1u;
    x += 0x7FFFu + lsb;
    return (uint16_t)(x >> 16);
}

EXPORT void oracle_f32_to_f16(const float *src, uint16_t *dst, int64_t count) {
    for (int64_t i = 0; i < count; ++i) dst[i] = f32_to_f16(src[i]);
}

EXPORT void oracle_f32_to_bf16(const float *src, uint16_t *dst, int64_t count) {
    for (int64_t i = 0; i < count; ++i) dst[i] = f32_to_bf16(src[i]);
}

/* binary16 -> binary32 (exact) */
static float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, mant = h & 0x3FFu;
    uint32_t x;
    if (e == 0) {
        if (mant == 0) {
            x = sign;
        } else { /* subnormal: mant * 2^-24 */
            float v = (float)mant * 5.9604644775390625e-08f;
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7F800000u | (mant << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/*
 * The library's fixed LayerNorm summation order: a row is split over WPR wave64s (1 for k <= 256, else 4); thread th
 * of the row sums, in increasing k, its 4-element chunks k = 4 * (th + 64 * WPR * i) + j; each wave combines its 64
 * partial sums with a xor butterfly (offsets 1, 2, 4, ..., 32); the wave totals are then added in wave order.
 */
static float row_sum(const float *z, int64_t k) {
    const int wpr = k > 256 ? 4 : 1, tpr = 64 * wpr;
    float p[256];
    for (int th = 0; th < tpr; ++th) {
        float s = 0.f;
        for (int64_t c = 4 * (int64_t)th; c < k; c += 4 * (int64_t)tpr)
            for (int64_t kk = c; kk < c + 4 && kk < k; ++kk) s = s + z[kk];
        p[th] = s;
    }
    float total = 0.f;
    for (int w = 0; w < wpr; ++w) {
        float *v = p + 64 * w;
        for (int off = 1; off <= 32; off <<= 1) {
            float nxt[64];
            for (int l = 0; l < 64; ++l) nxt[l] = v[l] + v[l ^ off];
            memcpy(v, nxt, sizeof(nxt));
        }
        total = w == 0 ? v[0] : total + v[0];
    }
    return total;
}

/*
 * x: row m at x + (m / t) * xb + (m % t) * xt + kk * xk (f32 elements when x_f16 == 0, binary16 bits otherwise).
 * q int8 [parts][m][ldq] (zero padded), qs f32 [parts][m] (the fp16-rounded value when qs_f16 != 0).
 */
EXPORT int oracle_quantize(const void *x, int x_f16, int64_t xb, int64_t xt, int64_t xk, int64_t t, int64_t m,
                           int64_t k, int parts, const float *nw, const float *nb, float eps, int input_silu,
                           int8_t *q, int64_t ldq, float *qs, int qs_f16) {
    if (parts < 1 || parts > 3 || k < 1 || ldq < k || t < 1) return -1;
#pragma omp parallel
    {
        float *z = (float *)__builtin_alloca(sizeof(float) * (size_t)k);
        float *sq = (float *)__builtin_alloca(sizeof(float) * (size_t)k);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < m; ++r) {
            const int64_t base = (r / t) * xb + (r % t) * xt;
            for (int64_t kk = 0; kk < k; ++kk) {
                const int64_t i = base + kk * xk;
                z[kk] = x_f16 ? f16_to_f32(((const uint16_t *)x)[i]) : ((const float *)x)[i];
            }
            if (nw) {
                const float mean = row_sum(z, k) / (float)k;
                for (int64_t kk = 0; kk < k; ++kk) z[kk] = z[kk] - mean;
                for (int64_t kk = 0; kk < k; ++kk) sq[kk] = z[kk] * z[kk];
                const float var = row_sum(sq, k) / (float)k;
                const float inv = 1.0f / sqrtf(var + eps);
                for (int64_t kk = 0; kk < k; ++kk) z[kk] = z[kk] * inv * nw[kk] + nb[kk];
            }
            if (input_silu)
                for (int64_t kk = 0; kk < k; ++kk) z[kk] = z[kk] * (1.0f / (1.0f + expf(-z[kk])));
            for (int c = 0; c < parts; ++c) {
                float amax = 0.f;
                for (int64_t kk = 0; kk < k; ++kk) amax = fmaxf(amax, fabsf(z[kk]));
                float s = fmaxf(amax / 127.0f, 1.0e-30f);
                if (qs_f16) {
                    s = f16_to_f32(f32_to_f16(s));
                    s = fmaxf(s, 5.9604644775390625e-08f);
                    s = fminf(s, 65504.0f);
                }
                qs[c * m + r] = s;
                int8_t *row = q + (c * m + r) * ldq;
                for (int64_t kk = 0; kk < k; ++kk) {
                    float v = rintf(z[kk] / s);
                    v = fminf(fmaxf(v, -127.0f), 127.0f);
                    row[kk] = (int8_t)(int)v;
                    z[kk] = z[kk] - v * s;
                }
                for (int64_t kk = k; kk < ldq; ++kk) row[kk] = 0;
            }
        }
    }
    return 0;
}
