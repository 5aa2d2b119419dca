/*
 * kea_encoder.h - fused FastConformer encoder kernels of libkea_hip.so (MI355X / gfx950), FP32.
 *
 * Conventions as in kea_lowbit.h: device pointers, int64 sizes and strides (in elements), a hipStream_t as void*,
 * KEA_OK / negative KEA_E* (nothing launched) / positive hipError_t, message in kea_last_error(). No allocation, no
 * host synchronisation: both entry points are HIP-graph capturable.
 */
#ifndef KEA_ENCODER_H
#define KEA_ENCODER_H

#include <stdint.h>

#include "kea_lowbit.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Relative-position multi-head self-attention (Transformer-XL form of NeMo's RelPositionMultiHeadAttention):
 *   for batch b, head h, query i, key j (T tokens, heads x head_dim = d):
 *     s[i][j] = ((q_i + u_h) . k_j + (q_i + v_h) . p_{T-1-i+j}) * scale,  out_i = sum_j softmax_j(s)[i][j] v_j
 *   q, k, v of token t: qkv[(b*T + t)*ld + {0, d, 2d} + h*head_dim + 0 .. head_dim-1]   (the fused QKV projection)
 *   p_r (relative position T-1-r, r = 0 .. 2T-2): pos[r*ldp + h*head_dim + ...]        (W_pos applied, [2T-1][>= d])
 *   bias_u, bias_v: [heads][head_dim];  out: out[(b*T + t)*ldo + h*head_dim + ...].
 * head_dim must be 128 and T <= 256; qkv, pos and out 16-byte aligned with ld, ldp, ldo multiples of 4.
 * Replaces the reference's relative_attention + Triton _attention / _position_scores
 * (kk/ternary/fused_kernels.py:163-240). */
int kea_relpos_attention(const float *qkv_dev, int64_t ld, const float *pos_dev, int64_t ldp,
                         const float *bias_u_dev, const float *bias_v_dev, float *out_dev, int64_t ldo,
                         int64_t batch, int64_t t, int heads, int head_dim, float scale, void *stream);

/* kea_relpos_attention with a workspace that lets small grids split every (clip, query tile, head) over two key
 * halves on two workgroups. Each half stores its unnormalised partial output O_s and its rows' softmax statistics
 * (m_s, l_s) in the workspace; a second launch merges them into out:
 *   out = (O0 exp(m0 - m) + O1 exp(m1 - m)) / (l0 exp(m0 - m) + l1 exp(m1 - m)),  m = max(m0, m1),
 * which equals the unsplit attention up to FP32 rounding. With out == NULL the merge is left to
 * kea_attention_merge_quantize, which quantizes the merged rows directly. kea_relpos_attention_workspace gives the
 * workspace size: 0 where the split does not apply (t > 128, an odd number of 16-key tiles, or a grid that already
 * fills the GPU); there workspace may be NULL, out is required and the call equals kea_relpos_attention. Same
 * reference function as kea_relpos_attention (kk/ternary/fused_kernels.py:163-240). */
int64_t kea_relpos_attention_workspace(int64_t batch, int64_t t, int heads);
int kea_relpos_attention_ws(const float *qkv_dev, int64_t ld, const float *pos_dev, int64_t ldp,
                            const float *bias_u_dev, const float *bias_v_dev, float *out_dev, int64_t ldo,
                            int64_t batch, int64_t t, int heads, int head_dim, float scale, void *workspace_dev,
                            int64_t workspace_bytes, void *stream);

/* The P-part int8 quantization (as kea_quantize, f32 scales, no LayerNorm) of the attention output that a
 * kea_relpos_attention_ws call with out == NULL left as two halves in `workspace_dev`: bitwise what kea_quantize
 * gives on that call's merged out, without writing it. The same batch, t and heads as that call (the split must
 * apply); q [parts][batch * t][ldq] (zero padded past heads * 128), qs [parts][batch * t]. The quantizer in front of
 * the attention output projection (kk/ternary/row_fusion.py:121-152 quantizes the attention output for it). */
int kea_attention_merge_quantize(const void *workspace_dev, int64_t workspace_bytes, int64_t batch, int64_t t,
                                 int heads, int parts, int8_t *q_dev, int64_t ldq, float *qs_dev, void *stream);

/* GLU + depthwise convolution (BatchNorm folded into w and bias by the caller):
 *   y[(b*T + t)*ldy + c] = bias[c] + sum_{j<kernel} w[c*kernel + j] * glu(b, t + j - kernel/2, c)
 *   glu(b, t, c) = x[(b*T + t)*ldx + c] * sigmoid(x[(b*T + t)*ldx + channels + c]), 0 outside [0, T).
 * kernel odd; bias may be NULL. Replaces the reference's _glu_pad + depthwise Conv1d + batch_norm of the patched
 * convolution module (kk/ternary/layer_fusions4.py:10-30, :62-72). */
int kea_glu_dwconv(const float *x_dev, int64_t ldx, const float *w_dev, const float *bias_dev, float *y_dev,
                   int64_t ldy, int64_t batch, int64_t t, int64_t channels, int kernel, void *stream);

/* x_out = LayerNorm0(x) (stored, FP32), then the P-part residual int8 quantization of LayerNorm1(x_out) exactly as
 * kea_quantize (f32 scales): one encoder layer's output LayerNorm fused with the normalised quantizer of the next
 * layer's first projection. Rows contiguous: x [m][ldx], x_out [m][ldo], 4 <= k <= 4096, k % 4 == 0; q [parts][m][ldq]
 * (zero padded), qs f32 [parts][m]. Replaces the reference's row epilogue LayerNorm + INT8x3 quantization
 * (kk/ternary/row_fusion.py:28-53, kk/binary/row_exact.py:98-156). */
int kea_norm_quantize(const float *x_dev, int64_t ldx, int64_t m, int64_t k, const float *norm0_w_dev,
                      const float *norm0_b_dev, float eps0, float *x_out_dev, int64_t ldo, const float *norm1_w_dev,
                      const float *norm1_b_dev, float eps1, int parts, int8_t *q_dev, int64_t ldq, float *qs_dev,
                      void *stream);

/* GLU + depthwise convolution as kea_glu_dwconv, then SiLU, then the P-part quantization of each token row (as
 * kea_quantize, f32 scales): the middle of the convolution module fused with the quantizer of its second pointwise
 * convolution (the reference's glu_pad + depthwise conv + BatchNorm + input SiLU of pointwise_conv2,
 * kk/ternary/layer_fusions4.py:62-72). channels % 4 == 0, channels <= 2048; q [parts][batch * t][ldq]. */
int kea_glu_dwconv_quantize(const float *x_dev, int64_t ldx, const float *w_dev, const float *bias_dev,
                            int64_t batch, int64_t t, int64_t channels, int kernel, int parts, int8_t *q_dev,
                            int64_t ldq, float *qs_dev, void *stream);

/* kea_glu_dwconv_quantize on GLU values already formed (u [batch*t][ldu], channels columns, rows 16-byte aligned):
 * the depthwise convolution, SiLU and quantization only. The GLU comes from the producing projection's epilogue
 * (kea_lowbit_gemm with KEA_FLAG_GLU and interleaved value / gate weight rows), which computes it with the same
 * formula, so the result is bitwise kea_glu_dwconv_quantize's. The reference's _glu_pad + depthwise Conv1d +
 * quantization of the next projection (kk/ternary/layer_fusions4.py:9-30, :62-72). */
int kea_dwconv_quantize(const float *u_dev, int64_t ldu, const float *w_dev, const float *bias_dev, int64_t batch,
                        int64_t t, int64_t channels, int kernel, int parts, int8_t *q_dev, int64_t ldq, float *qs_dev,
                        void *stream);

/* dw-striding subsampling (x8) of NeMo's ConvSubsampling, as the reference runs it inside its encoder (NeMo
 * modules, not part of kk/): conv 3x3 stride 2 (1 -> C channels, padding 1) + ReLU, then twice [depthwise 3x3 stride 2
 * + pointwise 1x1 + ReLU], then a linear layer over the flattened (channel, frequency) features. The pointwise
 * convolutions and the linear layer are matrix products left to the caller; these three launches are the rest.
 *
 * kea_subsample_front: x [batch][f][t] (f <= 128 mel bins of t frames) -> y [batch][C][t2][f2] =
 *   depthwise(relu(conv(x) + b1)) + b2, t1 = (t-1)/2+1, t2 = (t1-1)/2+1 (same for f); w1, w2 [C][9] (3x3, row-major).
 * kea_dwconv2d_s2: y [batch][C][(h-1)/2+1][(wd-1)/2+1] = depthwise3x3s2(relu(x + in_bias)) + bias, padding 1
 *   (in_bias NULL: a zero bias; the ReLU applies either way).
 * kea_bias_relu_flatten: y [batch][h][C * wd] = relu(x [batch][C][h][wd] + bias[c]). */
int kea_subsample_front(const float *x_dev, int64_t batch, int64_t t, int64_t f, const float *w1_dev,
                        const float *b1_dev, const float *w2_dev, const float *b2_dev, int64_t channels, float *y_dev,
                        void *stream);
int kea_dwconv2d_s2(const float *x_dev, const float *in_bias_dev, const float *w_dev, const float *bias_dev,
                    float *y_dev, int64_t batch, int64_t channels, int64_t h, int64_t wd, void *stream);
int kea_bias_relu_flatten(const float *x_dev, const float *bias_dev, float *y_dev, int64_t batch, int64_t channels,
                          int64_t h, int64_t wd, void *stream);

/* Normalised log-mel features from an STFT (the preprocessor of NeMo's AudioToMelSpectrogramPreprocessor, which
 * the reference's encoder runs in front of its layers): spec interleaved complex [batch][bins][ld_t] (ld_t >= frames),
 * fb [mels][bins] with row m nonzero only in [lo[m], hi[m]) (0 <= lo <= hi <= bins), y [batch][mels][frames] =
 *   v = log(sum_k fb[m][k] * |spec[k][t]|^2 + log_eps);  y = (v - mean_t v) / (std_t v + std_eps)  (std: n - 1). */
int kea_logmel_normalize(const float *spec_dev, int64_t batch, int64_t bins, int64_t frames, int64_t ld_t,
                         const float *fb_dev, const int32_t *lo_dev, const int32_t *hi_dev, int64_t mels, float log_eps,
                         float std_eps, float *y_dev, void *stream);

/* kea_logmel_normalize on a frame-major spectrum: spec interleaved complex [batch][ld_f][bins] (ld_f >= frames), as a
 * real FFT along the last dimension of kea_stft_frames' output leaves it. */
int kea_logmel_normalize_frames(const float *spec_dev, int64_t batch, int64_t bins, int64_t frames, int64_t ld_f,
                                const float *fb_dev, const int32_t *lo_dev, const int32_t *hi_dev, int64_t mels,
                                float log_eps, float std_eps, float *y_dev, void *stream);

/* The frames torch.stft transforms for center = True, pad_mode "constant", with NeMo's pre-emphasis applied first:
 * audio [batch][samples] -> frames [batch][1 + samples / hop][n_fft],
 *   frames[b][f][j] = window[j] * x[b][f * hop + j - n_fft / 2],
 *   x[b][0] = audio[b][0], x[b][i] = audio[b][i] - preemph * audio[b][i - 1], zero outside [0, samples),
 * window [n_fft] (the analysis window zero-padded to n_fft, as torch.stft pads it). Even n_fft <= 65536. */
int kea_stft_frames(const float *audio_dev, int64_t batch, int64_t samples, float preemph, const float *window_dev,
                    int64_t n_fft, int64_t hop, float *frames_dev, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* KEA_ENCODER_H */
