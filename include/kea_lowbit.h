/*
 * kea_lowbit.h - C ABI of libkea_hip.so, the MI355X (gfx950) low-bit GEMM library.
 *
 * 1-bit (sign) and 2-bit (ternary) weights x int8 activations, int32 accumulation on CDNA4 int8 MFMA,
 * fused FP32 epilogue (per-token and per-channel / per-group scales, bias, optional SiLU) to f32/f16/bf16.
 *
 * Conventions
 *   - Every pointer named *_dev is a device pointer (hipMalloc / torch CUDA tensor memory); *_host is host memory.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream). Calls are stream-ordered and never
 *     synchronize the host. No function allocates device memory: the caller passes every buffer.
 *   - Functions return KEA_OK (0) on success, a negative KEA_E* code for a contract violation (nothing is
 *     launched), or a positive hipError_t when the HIP runtime refused a launch. kea_last_error() returns a
 *     thread-local message describing the last failure of the calling thread.
 *   - A call whose grid would exceed one dispatch (2^32 work-items along a grid dimension) fails with KEA_EINVAL
 *     ("too large for one launch") instead of being truncated: split it along M (or N for the GEMM).
 *
 * Reference interfaces replaced (paths relative to the reference checkout, kk/ = src/kea_kernels/):
 *   kea_lowbit_gemm    <- the NVRTC kernel entry `b1_dot_*` (kk/binary/kernels.py:556-565) launched by
 *                         kk/binary/layer.py:182-201 and kk/binary/layer_parts.py:112-130, the fallback
 *                         `b1_fallback` (kk/binary/kernels.py:619-637), and the ternary Triton `_int8_dot` +
 *                         `_finish` pair (kk/ternary/fused_kernels.py:53-120, kk/ternary/kernels.py:122-137)
 *   kea_b1_relayout_host / kea_b1_unlayout_host
 *                      <- `relayout` / `unlayout` (kk/binary/kernels.py:730-752), re-targeted to the gfx950
 *                         native word layout described below
 *   kea_t2_relayout_host / kea_t2_unlayout_host
 *                      <- the int32 `packed_t` words of PackedLinear (kk/ternary/runtime.py:33-35) and the
 *                         one-time `_expand` (kk/ternary/encoder4.py:51-61): the 2-bit codes stay resident
 *   kea_quantize       <- `b1_quantize` (kk/binary/kernels.py:578-616) and the Triton `_quantize`
 *                         (kk/ternary/fused_kernels.py:31-50), with LayerNorm / input SiLU fused
 */
#ifndef KEA_LOWBIT_H
#define KEA_LOWBIT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define KEA_OK 0
#define KEA_EINVAL (-1)     /* bad argument value (sizes, flags, dtype enums) */
#define KEA_EALIGN (-2)     /* pointer or leading dimension not aligned as required */
#define KEA_ECODES (-3)     /* invalid packed weight codes (tail bits, the unused ternary 11 pattern) */
#define KEA_ESPACE (-4)     /* workspace missing or too small */
#define KEA_ENODEV (-5)     /* no usable gfx950 device */

/* element types of scales, bias and outputs */
#define KEA_F32 0
#define KEA_F16 1
#define KEA_BF16 2

/* epilogue flags */
#define KEA_FLAG_SILU 1     /* y = y * sigmoid(y) after scale and bias */
#define KEA_FLAG_ORDER 2    /* P = 2 / 3: first FP32 contraction fma(a1, s1, a0 * s0) instead of fma(a0, s0, a1 * s1) */
#define KEA_FLAG_GLU 4      /* kea_lowbit_gemm only: column pairs (2j, 2j + 1) -> y[j] = r[2j] * sigmoid(r[2j + 1]) */

/* ---------------------------------------------------------------------------------------------------------
 * Weight layouts
 *
 * Export layouts (the on-disk formats the library accepts; identical to the reference's):
 *   1-bit   uint8 [N][ceil(K/8)]: code k of row n is bit k%8 of byte k/8 (LSB first); 1 = +1, 0 = -1;
 *           unused tail bits 0 (kk/binary/bits.py:3-5).
 *   2-bit   uint8 [N][ceil(K/4)]: code k at bits 2*(k%4) of byte k/4; 00 = 0, 01 = +1, 10 = -1; 11 invalid;
 *           tail codes 0 (kk/formats.py:5-7, :62-81).
 *
 * Native layouts (device resident, built once by the relayout functions): uint32 words grouped per 16-row
 * "n-tile" t (rows 16t .. 16t+15, zero padded past N) and per lane l = 0..63 of a wavefront:
 *   1-bit   J = ceil(K/128) words per lane; word j of lane l holds, at bit 8*i + 4*h + d (i, d in 0..3,
 *           h in 0..1), the INVERTED sign (1 = -1) of w[n = 16t + l%16][k = 128j + 64h + 16(l/16) + 4d + i].
 *   2-bit   J = ceil(K/64) words per lane; word j of lane l holds, at bits 8*i + 2*d .. +1, the 2-bit code of
 *           w[n = 16t + l%16][k = 64j + 16(l/16) + 4d + i] (k >= K: code 00).
 *   Words are stored quad-major so that one 128-bit load per lane fetches 4 consecutive words: word j of lane
 *   l of tile t is at index  t*J*64 + (j/4)*256 + l*wq + j%4,  wq = min(4, J - 4*(j/4)).
 * --------------------------------------------------------------------------------------------------------- */

/* The 1-bit native layout has a second part after the words above, the bit-plane layout, which the wide wave-split
 * tiles read (one activation part on tiles of 4 or 8 n-tiles, two parts on 16x128 tiles; the LDS-ring GEMM, the
 * per-group kernel and the other wave-split tiles read the words), so a 1-bit weight takes 2 bits resident: rows in
 * groups of 128 (8 n-tiles, zero padded past N), k in steps of 64; for group g, k-step s and lane l, a 16-byte unit
 * of 4 words at word index
 *   P0 + ((g * ceil(K/64) + s) * 64 + l) * 4 + d,   P0 = ceil(N/16) * ceil(K/128) * 64 (the word part's size),
 * whose bit 8*i + p of word d is the INVERTED sign of w[n = 128g + 16p + l%16][k = 64s + 16(l/16) + 4d + i]. Masking
 * the unit with 0x01010101 << p gives the MFMA operand of n-tile p of the group with int8 values 0 / 2^p (p = 7:
 * -128): one AND per 4 weights instead of an AND and a byte permute. The kernel divides the exact sum by 2^p and
 * recovers sum q * w = sum q - 2 * sum q * bit from a row sum of q (an MFMA on an all-ones operand). */

/* Number of uint32 words of the native layout for an N x K weight matrix (0 on bad sizes). */
int64_t kea_b1_native_words(int64_t n, int64_t k);
int64_t kea_t2_native_words(int64_t n, int64_t k);

/* Export codes (host) -> native words (host). KEA_ECODES on nonzero tail bits (1-bit) or on the 11 pattern /
 * nonzero tail codes (2-bit). `words_host` must hold kea_*_native_words(n, k) words. */
int kea_b1_relayout_host(const uint8_t *codes_host, int64_t n, int64_t k, uint32_t *words_host);
int kea_t2_relayout_host(const uint8_t *codes_host, int64_t n, int64_t k, uint32_t *words_host);

/* Inverse: native words (host) -> export codes (host). */
int kea_b1_unlayout_host(const uint32_t *words_host, int64_t n, int64_t k, uint8_t *codes_host);
int kea_t2_unlayout_host(const uint32_t *words_host, int64_t n, int64_t k, uint8_t *codes_host);

/* ---------------------------------------------------------------------------------------------------------
 * The low-bit GEMM
 *
 *   acc_c[m][n] = sum_k q[c*part_stride + m*ldq + k] * w[n][k]        (exact int32, c = 0 .. parts-1)
 *   per-channel scales (ws_group == 0):
 *     r = comb_P(acc, qs[c*qs_stride + m])       P = 1: f(a0)*s0
 *                                                P = 2: fma(f(a0), s0, f(a1)*s1)   (ORDER: fma(f(a1), s1, f(a0)*s0))
 *                                                P = 3: fma(f(a2), s2, <P = 2 form>)
 *     r = bias ? fma(r, alpha[n], bias[n]) : r * alpha[n]
 *   per-group scales (ws_group = 64, 128 or 256; alpha is [N][ceil(K/ws_group)] row-major, group g covering
 *   k in [g*ws_group, (g+1)*ws_group); unsplit, split_k 0 or 1; config 0, ring tile 1 or 4, or a wave-split tile of
 *   16-row blocks and at most 64 columns whose one workgroup covers K exactly, K = waves x 64 x 2..16 with whole
 *   groups per wave):
 *     r = 0; for g in groups: r = fma(comb_P(acc_g, s), alpha[n][g], r);  r = bias ? r + bias[n] : r
 *   SiLU (flags & KEA_FLAG_SILU): r = r / (1 + exp(-r)); then y[m*ldy + n] = RN(r) in y_dtype.
 *   f() is int32 -> fp32 round-to-nearest; every FP32 operation is IEEE round-to-nearest-even, unfused
 *   except where an fma is written (kk/binary/kernels_parts.py:28-39, kk/binary/kernels.py:76-93).
 *
 *   q          int8, rows 16-byte aligned: q_dev % 16 == 0, ldq % 16 == 0, part_stride % 16 == 0, ldq >= k.
 *              Bytes at k .. ldq-1 are never read as data (they are masked to zero in-kernel).
 *   qs         per-token scales [parts][m] (stride qs_stride), dtype KEA_F32 or KEA_F16; qs, wscale and bias are
 *              aligned to their element size (KEA_EALIGN otherwise).
 *   w          native words (kea_b1_relayout_host / kea_t2_relayout_host), 16-byte aligned.
 *   wscale     alpha, dtype KEA_F32 or KEA_F16.  bias: NULL or [n] of bias_dtype (KEA_F32 / KEA_F16).
 *   y          NULL (no dequantized output) or [m][ldy] of y_dtype (KEA_F32 / KEA_F16 / KEA_BF16), ldy >= n.
 *   acc_out    NULL or int32 [parts][m][acc_ld] raw accumulators (acc_ld >= n); exact for every split.
 *   split_k    1 = one launch; > 1 = K split over split_k slices with an exact int32 reduction in a fixed
 *              order (a second, finishing launch). Needs workspace_dev of kea_lowbit_gemm_workspace() bytes.
 *              0 = the library chooses (a pure function of the shape).
 *   config     0 = the library's tile table (a pure function of wbits, parts, m, n, k); > 0 selects a tile
 *              configuration by id (results are identical for every config; see kea_config_count()).
 * --------------------------------------------------------------------------------------------------------- */
int kea_lowbit_gemm(int wbits,
                    const int8_t *q_dev, int64_t part_stride, int64_t ldq, int parts,
                    const void *qs_dev, int qs_dtype, int64_t qs_stride,
                    const uint32_t *w_dev, int64_t n, int64_t k,
                    const void *wscale_dev, int ws_dtype, int64_t ws_group,
                    const void *bias_dev, int bias_dtype,
                    void *y_dev, int y_dtype, int64_t ldy,
                    int32_t *acc_out_dev, int64_t acc_ld,
                    int64_t m, int flags, int split_k, int config,
                    void *workspace_dev, int64_t workspace_bytes, void *stream);

/* kea_lowbit_gemm plus a residual stream: y[m*ldy + n] = residual[m*ldr + n] + r * factor (an IEEE multiply, then an
 * IEEE add), with r the epilogue value above (after bias and SiLU). residual is FP32 [m][ldr], ldr >= n; y may be
 * the residual itself (in place, with ldy == ldr and y_dtype KEA_F32). Replaces the residual step of the reference's
 * row epilogue, x = R + value * FACTOR (kk/ternary/row_fusion.py:28-39, :90-113). */
int kea_lowbit_gemm_residual(int wbits,
                             const int8_t *q_dev, int64_t part_stride, int64_t ldq, int parts,
                             const void *qs_dev, int qs_dtype, int64_t qs_stride,
                             const uint32_t *w_dev, int64_t n, int64_t k,
                             const void *wscale_dev, int ws_dtype, int64_t ws_group,
                             const void *bias_dev, int bias_dtype,
                             void *y_dev, int y_dtype, int64_t ldy,
                             int32_t *acc_out_dev, int64_t acc_ld,
                             int64_t m, int flags, int split_k, int config,
                             void *workspace_dev, int64_t workspace_bytes,
                             const float *residual_dev, int64_t ldr, float factor, void *stream);

/* Exact deferred split-K: the K range is cut into `split` slices (split >= 1, at most ceil(J/4) where J is the number
 * of native words per lane) and slice z writes its exact int32 partial accumulators to
 * slices_dev[((z * parts + c) * m + row) * n + col] (int32 [split][parts][m][n], 16-byte aligned). No scale is read.
 * Replaces the XCHG 5 slice kernels (kk/binary/kernels_exact.py:24-54) driven by hybrid_exact.dot_slices
 * (kk/binary/hybrid_exact.py:53-72), whose slices are packed int64 words instead. */
int kea_lowbit_gemm_slices(int wbits, const int8_t *q_dev, int64_t part_stride, int64_t ldq, int parts,
                           const uint32_t *w_dev, int64_t n, int64_t k, int64_t m, int split, int config,
                           int32_t *slices_dev, void *stream);

/* Sums slices int32 [split][parts][m][n] in slice order (exact) and applies the epilogue of kea_lowbit_gemm (same
 * scale, bias, flag and output arguments); bitwise the unsplit kea_lowbit_gemm result. Replaces the integer finish
 * of the reference's exact row epilogue (kk/binary/row_exact.py:69-96) for the projection value. */
int kea_lowbit_slices_finish(const int32_t *slices_dev, int split, int parts, int64_t m, int64_t n,
                             const void *qs_dev, int qs_dtype, int64_t qs_stride,
                             const void *wscale_dev, int ws_dtype, const void *bias_dev, int bias_dtype,
                             void *y_dev, int y_dtype, int64_t ldy, int32_t *acc_out_dev, int64_t acc_ld,
                             int flags, void *stream);

/* The exact row epilogue, one launch per projection: for every row m of the [m][n] output,
 *   value = kea_lowbit_slices_finish's value (slices summed in slice order, then the unsplit epilogue: bitwise
 *           the unsplit kea_lowbit_gemm result; qs f32 [parts][qs_stride], wscale / bias f32 or f16 [n])
 *   x     = residual ? residual[m*ldr + j] + value * factor : value      (an IEEE multiply, then an IEEE add)
 *   x     = LayerNorm(x; out_norm_w, out_norm_b, out_eps)                 when out_norm_w != NULL
 *   y[m*ldy + j] = x                                                      (FP32; y may be the residual itself)
 *   q, q_scales = the q_parts-part quantization of LayerNorm(x; norm_w, norm_b, eps) (or of x when norm_w is NULL),
 *                 bitwise what kea_quantize returns for y's rows (q int8 [q_parts][m][ldq] zero padded, q_scales f32
 *                 [q_parts][m]); skipped when q is NULL.
 * n in 4..4096 with n % 4 == 0; slices, y, residual and the LayerNorm weights 16-byte aligned, ldy and ldr multiples
 * of 4, ldq >= n a multiple of 4. LayerNorm sums follow kea_quantize's fixed order. Replaces the reference's
 * _row_epilogue_exact / _row_epilogue (kk/binary/row_exact.py:62-122, kk/ternary/row_fusion.py:27-52) behind
 * finish_residual_exact / finish_residual (kk/binary/row_exact.py:125-156, kk/ternary/row_fusion.py:90-111). */
int kea_row_epilogue(const int32_t *slices_dev, int split, int parts, int64_t m, int64_t n,
                     const float *qs_dev, int64_t qs_stride, const void *wscale_dev, int ws_dtype,
                     const void *bias_dev, int bias_dtype, int flags,
                     const float *residual_dev, int64_t ldr, float factor,
                     const float *out_norm_w_dev, const float *out_norm_b_dev, float out_eps,
                     float *y_dev, int64_t ldy,
                     const float *norm_w_dev, const float *norm_b_dev, float eps,
                     int q_parts, int8_t *q_dev, int64_t ldq, float *q_scales_dev, void *stream);

/* GLU pairs (flags & KEA_FLAG_GLU; kea_lowbit_gemm and kea_lowbit_gemm_residual without a residual; per-channel
 * scales, no SiLU, n even): after scale and bias, y[m*ldy + j] = RN(r[2j] * (1 / (1 + exp(-r[2j+1])))) for
 * j < n/2, ldy >= n/2; acc_out still receives all n accumulators. A GLU whose value / gate halves are separate row
 * blocks (NeMo's conv module, GLU over [value; gate]) runs with the weight rows interleaved value, gate, value, ...
 * (scale and bias rows alike). Replaces the GLU of the reference's _glu_pad (kk/ternary/layer_fusions4.py:9-22). */

/* Workspace bytes kea_lowbit_gemm needs for these arguments (0 when split_k resolves to 1). */
int64_t kea_lowbit_gemm_workspace(int wbits, int parts, int64_t m, int64_t n, int64_t k, int64_t ws_group,
                                  int split_k, int config);

/* Plans: kea_lowbit_gemm's checks and its tile / split / kernel resolution done once, for callers that launch the
 * same GEMM on the same buffers many times (serving loops, benchmarks): kea_lowbit_gemm_plan takes kea_lowbit_gemm's
 * arguments (without the stream) plus kea_lowbit_gemm_residual's residual, ldr and factor (residual NULL: none) and
 * returns a host-side plan, or NULL with kea_last_error() set on any argument kea_lowbit_gemm would refuse. The plan
 * records the pointers: their buffers must stay allocated, with the same contents layout, while it is launched.
 * kea_lowbit_gemm_plan_launch enqueues the GEMM (and its split-K finish) on `stream` exactly as kea_lowbit_gemm would;
 * kea_lowbit_gemm_plan_free releases the plan (host memory only). No counterpart in the reference, whose launches
 * re-validate on every call (kk/binary/layer.py:182-201). */
typedef struct kea_gemm_plan kea_gemm_plan;
kea_gemm_plan *kea_lowbit_gemm_plan(int wbits,
                                    const int8_t *q_dev, int64_t part_stride, int64_t ldq, int parts,
                                    const void *qs_dev, int qs_dtype, int64_t qs_stride,
                                    const uint32_t *w_dev, int64_t n, int64_t k,
                                    const void *wscale_dev, int ws_dtype, int64_t ws_group,
                                    const void *bias_dev, int bias_dtype,
                                    void *y_dev, int y_dtype, int64_t ldy,
                                    int32_t *acc_out_dev, int64_t acc_ld,
                                    int64_t m, int flags, int split_k, int config,
                                    void *workspace_dev, int64_t workspace_bytes,
                                    const float *residual_dev, int64_t ldr, float factor);
int kea_lowbit_gemm_plan_launch(const kea_gemm_plan *plan, void *stream);
void kea_lowbit_gemm_plan_free(kea_gemm_plan *plan);

/* The plan's GEMM on other activation and output buffers of the same layout: q (16-byte aligned), qs, y, acc_out and
 * residual replace the pointers the plan was made with (each present exactly where the plan has one; their shapes,
 * strides and dtypes are the plan's), the weights and scales stay the plan's. workspace: kea_lowbit_gemm_plan_workspace
 * bytes (0: none needed). The plan is not modified, so one plan may be launched from several threads. This is the
 * per-call path of the operators' cached dot() launches on caller-made parts (an operator resolves a plan once per
 * call layout, then binds each call's buffers; its quantize-and-GEMM calls use the projection plan below), which
 * replaces the reference's per-call validation and launch (kk/binary/layer.py:182-209,
 * kk/ternary/fused_kernels.py:139-160). */
int kea_lowbit_gemm_plan_launch_with(const kea_gemm_plan *plan, const int8_t *q_dev, const void *qs_dev, void *y_dev,
                                     int32_t *acc_out_dev, const float *residual_dev, void *workspace_dev,
                                     int64_t workspace_bytes, void *stream);
int64_t kea_lowbit_gemm_plan_workspace(const kea_gemm_plan *plan);

/* One operator call in one C call: kea_quantize of x's rows into int8 parts, then a plan's GEMM on those parts, both
 * enqueued on `stream`. kea_lowbit_project_plan takes a GEMM plan made on a quantizer layout (y only, no acc_out or
 * residual; part_stride = m * ldq, qs_stride = m; the plan's parts, m, k, ldq and qs dtype are the quantizer's) and
 * kea_quantize's row mapping and LayerNorm / SiLU arguments; it copies what it needs, so the GEMM plan may be freed
 * afterwards, and returns NULL with kea_last_error() set on any argument kea_quantize or the launch would refuse.
 * The norm pointers are recorded and read on every launch. kea_lowbit_project_launch takes x (the plan's dtype and
 * row mapping), y (the plan's dtype and row stride) and a 16-byte aligned device workspace of at least
 * kea_lowbit_project_workspace bytes, which holds the int8 parts from its first byte, then their scales and any
 * split-K slices (calls that share a workspace must be ordered on one stream). Results are the bits of kea_quantize
 * followed by kea_lowbit_gemm. Replaces the reference's two per-call launches of an operator call, b1_quantize and
 * b1_dot (kk/binary/layer.py:154-165 and :182-209). */
typedef struct kea_project_plan kea_project_plan;
kea_project_plan *kea_lowbit_project_plan(const kea_gemm_plan *plan, int x_dtype, int64_t xb, int64_t xt,
                                          int64_t xk, int64_t t, const float *norm_w_dev, const float *norm_b_dev,
                                          float eps, int input_silu);
int64_t kea_lowbit_project_workspace(const kea_project_plan *pp);
int kea_lowbit_project_launch(const kea_project_plan *pp, const void *x_dev, void *y_dev, void *workspace_dev,
                              int64_t workspace_bytes, void *stream);
void kea_lowbit_project_plan_free(kea_project_plan *pp);

/* kea_lowbit_gemm without the workspace arguments, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). It has no counterpart in the reference. The
 * split-K slices live in a library-owned device array of KEA_NOALLOC_SCRATCH_BYTES per GPU (a file-scope __device__
 * array, held until the process ends); a call whose kea_lowbit_gemm_workspace() exceeds that returns KEA_ESPACE
 * with nothing launched. The call allocates nothing (no hipMalloc, hipFree or allocating library routine). Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU (on different streams, or in graphs
 * replayed concurrently) race on it; calls ordered on one stream do not. Results are identical to kea_lowbit_gemm's
 * for the same arguments. */
#define KEA_NOALLOC_SCRATCH_BYTES (8LL << 20)
int kea_lowbit_gemm_noalloc(int wbits,
                            const int8_t *q_dev, int64_t part_stride, int64_t ldq, int parts,
                            const void *qs_dev, int qs_dtype, int64_t qs_stride,
                            const uint32_t *w_dev, int64_t n, int64_t k,
                            const void *wscale_dev, int ws_dtype, int64_t ws_group,
                            const void *bias_dev, int bias_dtype,
                            void *y_dev, int y_dtype, int64_t ldy,
                            int32_t *acc_out_dev, int64_t acc_ld,
                            int64_t m, int flags, int split_k, int config, void *stream);

/* The tile configuration id config == 0 resolves to for this shape (-1 on bad arguments). */
int kea_lowbit_gemm_tile(int wbits, int parts, int64_t m, int64_t n, int64_t k);

/* The split factor split_k == 0 resolves to for this shape (results are identical for every split). */
int kea_lowbit_gemm_split(int wbits, int parts, int64_t m, int64_t n, int64_t k, int64_t ws_group, int config);

/* Number of tile configurations (valid ids are 1 .. count) and a description of one ("BMxBN waves ..."). */
int kea_config_count(void);
const char *kea_config_name(int config);

/* ---------------------------------------------------------------------------------------------------------
 * Residual int8 activation quantizer (optional fused LayerNorm and input SiLU), one row per token:
 *   x[m][k] at x_dev + (m / t) * xb + (m % t) * xt + k * xk   (elements of x_dtype, KEA_F32 / KEA_F16)
 *   z = LayerNorm(x) * norm_w + norm_b   if norm_w_dev != NULL (FP32 weights, eps)
 *   z = z * sigmoid(z)                   if input_silu
 *   for c < parts:  s_c = max(max|z| / 127, 1e-30);  q_c = rint(z / s_c);  z = z - q_c * s_c
 * q_dev int8 [parts][m][ldq] (zero padded from k to ldq), qs_dev [parts][m] of qs_dtype. With qs_dtype ==
 * KEA_F16 the scale is rounded to fp16 first (floored at the smallest fp16 subnormal) and q is clamped to
 * [-127, 127] (kk/binary/kernels.py:567-616, kk/ternary/fused_kernels.py:31-50).
 * --------------------------------------------------------------------------------------------------------- */
int kea_quantize(const void *x_dev, int x_dtype, int64_t xb, int64_t xt, int64_t xk, int64_t t,
                 int64_t m, int64_t k, int parts,
                 const float *norm_w_dev, const float *norm_b_dev, float eps, int input_silu,
                 int8_t *q_dev, int64_t ldq, void *qs_dev, int qs_dtype, void *stream);

/* Message of the calling thread's last failure ("" if none). */
const char *kea_last_error(void);

/* Library ABI version (major * 100 + minor). */
int kea_version(void);

#ifdef __cplusplus
}
#endif
#endif /* KEA_LOWBIT_H */
