"""A Parakeet-TDT-0.6B-shaped FastConformer encoder on the 1-bit layers (the workload of BASELINE.json config 5).

The reference runs NeMo's encoder with its 264 quantized linears swapped for provider-backed modules
(kk/binary/provider.py:212-262) and a set of offline fusions (kk/ternary/layer_fusions4.py,
kk/ternary/transforms.py). NeMo is not part of this build, so this module is the build's own encoder with the same
layer arithmetic (NeMo ConformerLayer with relative-position attention, as patched by
kk/ternary/layer_fusions4.py:60-80):

    x   = audio -> log-mel (128 bins) -> dw-striding subsampling x8 (Conv2d 3x3/2 + 2 x [depthwise 3x3/2 +
          pointwise 1x1], ReLU) -> Linear(256 * 16 -> d) -> x * sqrt(d)
    per layer (24):
      r = x + 0.5 * FF1(LN(x))                      FF(z) = W2 silu(W1 z)
      r = r + W_out RelPosMHSA(LN(r))               q, k, v = W_qkv z (fused), p = W_pos pos_emb (frozen per T)
      r = r + W_pw2 silu(BN(dwconv9(GLU(W_pw1 LN(r)))))
      r = r + 0.5 * FF2(LN(r))
      x = LN_out(r)

All 11 linears of a layer (W1, W2 of both FFs, W_q, W_k, W_v, W_out, W_pos, W_pw1, W_pw2; formats.PER_LAYER) are
1-bit x int8 GEMMs through the provider seam (binary.provider.BinaryProjection over Int8MmaPartsLayer), with the
LayerNorms in front of W1 / W_qkv / W_pw1 fused into the quantizer, SiLU after W1 fused into the GEMM epilogue and
the SiLU in front of W_pw2 fused into the quantizer (the reference's norm_quant / silu transforms). The attention core
(relative-position scores, softmax, P.V) and GLU + depthwise convolution (BatchNorm folded into its weights) are the
fused HIP kernels of include/kea_encoder.h (the reference's Triton relative_attention and glu_pad); the GLU kernel
also applies the SiLU and quantizes for W_pw2 (kea_glu_dwconv_quantize). The four residual projections (W2 of both
FFs, W_out, W_pw2) add the residual in their GEMM epilogue, in place (the reference's row_fusions,
kk/ternary/row_fusion.py:121-152); the quantizers run as row kernels between the GEMMs (kea_quantize,
kea_norm_quantize, kea_attention_merge_quantize), 17 launches a layer. The subsampling convolutions are PyTorch on
the GPU.
With fused=False the same model runs with separate quantizers, the residual in the GEMM epilogue
(kea_lowbit_gemm_residual) and PyTorch attention, GLU and convolution. The quantized linears have no bias
(Q/K/V must be bias-free to fuse, kk/binary/provider.py:230-244).

`EncoderGraph` captures preprocessing + encoder for a fixed (batch, samples) into one HIP graph, as the reference
captures its encoder (kk/ternary/graphs.py). `dense=True` builds the same model with the quantized linears replaced by
FP32 matmuls on the dense weights (signs * alpha): the parity reference for the quantized encoder.
"""
from __future__ import annotations

import contextlib
import math
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F
from torch import Tensor

from kea_kernels import _hip, formats, lowbit
from kea_kernels.binary import bits, layer_parts, provider


@dataclass(frozen=True)
class EncoderConfig:
    layers: int = 24
    d_model: int = 1024
    heads: int = 8
    ff_mult: int = 4
    conv_kernel: int = 9
    feat_in: int = 128
    sub_channels: int = 256
    xscaling: bool = True
    sample_rate: int = 16000
    n_fft: int = 512
    win_length: int = 400
    hop_length: int = 160
    preemph: float = 0.97
    eps: float = 1e-5

    @property
    def d_ff(self) -> int:
        return self.ff_mult * self.d_model


def quantized_shapes(cfg: EncoderConfig) -> dict:
    """{suffix: (N, K, kind)} of the 11 quantized linears of one layer."""
    d, f = cfg.d_model, cfg.d_ff
    return {"feed_forward1.linear1": (f, d, "linear"), "feed_forward1.linear2": (d, f, "linear"),
            "feed_forward2.linear1": (f, d, "linear"), "feed_forward2.linear2": (d, f, "linear"),
            "self_attn.linear_q": (d, d, "linear"), "self_attn.linear_k": (d, d, "linear"),
            "self_attn.linear_v": (d, d, "linear"), "self_attn.linear_out": (d, d, "linear"),
            "self_attn.linear_pos": (d, d, "linear"), "conv.pointwise_conv1": (2 * d, d, "conv"),
            "conv.pointwise_conv2": (d, d, "conv")}


def synthetic_weights(cfg: EncoderConfig, seed: int = 0) -> dict:
    """Random-init parameters on the CPU (seeded torch.Generator). Quantized linears as export codes + FP32 scales
    (alpha ~ U(0.5, 1.5) / sqrt(K), which keeps activations O(1) through the stack)."""
    g = torch.Generator().manual_seed(seed)
    d, c, h = cfg.d_model, cfg.sub_channels, cfg.heads

    def randn(*shape, std=1.0):
        return torch.randn(*shape, generator=g) * std

    w = {}
    shapes = quantized_shapes(cfg)
    assert tuple(shapes) == tuple(sorted(shapes, key=formats.PER_LAYER.index))
    for layer in range(cfg.layers):
        pre = f"encoder.layers.{layer}."
        for suffix, (n, k, _) in shapes.items():
            signs = torch.where(torch.rand(n, k, generator=g) < 0.5, -1, 1).to(torch.int8)
            w[pre + suffix + ".codes"] = bits.pack_signs(signs)
            w[pre + suffix + ".scale"] = (torch.rand(n, generator=g) + 0.5) / math.sqrt(k)
        for norm in ("norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2", "norm_out"):
            w[pre + norm + ".weight"] = 1.0 + randn(d, std=0.05)
            w[pre + norm + ".bias"] = randn(d, std=0.02)
        w[pre + "self_attn.pos_bias_u"] = randn(h, d // h, std=0.02)
        w[pre + "self_attn.pos_bias_v"] = randn(h, d // h, std=0.02)
        w[pre + "conv.depthwise_conv.weight"] = randn(d, 1, cfg.conv_kernel, std=1.0 / 3.0)
        w[pre + "conv.batch_norm.weight"] = 1.0 + randn(d, std=0.05)
        w[pre + "conv.batch_norm.bias"] = randn(d, std=0.02)
        w[pre + "conv.batch_norm.running_mean"] = randn(d, std=0.1)
        w[pre + "conv.batch_norm.running_var"] = 1.0 + torch.rand(d, generator=g)
    pre = "encoder.pre_encode."
    w[pre + "conv.0.weight"] = randn(c, 1, 3, 3, std=1.0 / 3.0)
    w[pre + "conv.0.bias"] = randn(c, std=0.02)
    for i in (2, 5):
        w[pre + f"conv.{i}.weight"] = randn(c, 1, 3, 3, std=1.0 / 3.0)
        w[pre + f"conv.{i}.bias"] = randn(c, std=0.02)
        w[pre + f"conv.{i + 1}.weight"] = randn(c, c, 1, 1, std=1.0 / math.sqrt(c))
        w[pre + f"conv.{i + 1}.bias"] = randn(c, std=0.02)
    sub_out = c * (cfg.feat_in // 8)
    w[pre + "out.weight"] = randn(d, sub_out, std=1.0 / math.sqrt(sub_out))
    w[pre + "out.bias"] = randn(d, std=0.02)
    return w


# --- preprocessing ---------------------------------------------------------------------------------------------------

def mel_filterbank(cfg: EncoderConfig) -> np.ndarray:
    """[n_mels, n_fft // 2 + 1] triangular filters on the Slaney mel scale with Slaney area normalisation (the
    librosa default NeMo's preprocessor uses), FP64."""
    def hz_to_mel(f):
        f = np.asarray(f, np.float64)
        lin = f / (200.0 / 3)
        logstep = math.log(6.4) / 27.0
        return np.where(f >= 1000.0, 15.0 + np.log(np.maximum(f, 1e-10) / 1000.0) / logstep, lin)

    def mel_to_hz(m):
        m = np.asarray(m, np.float64)
        logstep = math.log(6.4) / 27.0
        return np.where(m >= 15.0, 1000.0 * np.exp(logstep * (m - 15.0)), m * (200.0 / 3))

    n_bins = cfg.n_fft // 2 + 1
    fft_freqs = np.linspace(0, cfg.sample_rate / 2, n_bins)
    mel_pts = mel_to_hz(np.linspace(hz_to_mel(0.0), hz_to_mel(cfg.sample_rate / 2), cfg.feat_in + 2))
    fdiff = np.diff(mel_pts)
    ramps = mel_pts[:, None] - fft_freqs[None, :]
    lower = -ramps[:-2] / fdiff[:-1, None]
    upper = ramps[2:] / fdiff[1:, None]
    fb = np.maximum(0.0, np.minimum(lower, upper))
    fb *= (2.0 / (mel_pts[2:cfg.feat_in + 2] - mel_pts[:cfg.feat_in]))[:, None]
    return fb


def frames_for(cfg: EncoderConfig, samples: int) -> int:
    """Feature frames of a clip: samples / hop (the centred STFT's final frame is dropped: 160,000 -> 1000)."""
    return samples // cfg.hop_length


def encoded_length(frames: int) -> int:
    for _ in range(3):
        frames = (frames + 2 - 3) // 2 + 1
    return frames


class Preprocessor:
    """audio [B, S] FP32 -> normalised log-mel [B, n_mels, frames]: pre-emphasis, |STFT|^2 (Hann 400 / hop 160 /
    n_fft 512, centred), mel projection, log(x + 2^-24), per-feature mean / std normalisation over time.
    fused: the pre-emphasised, windowed frames in one kernel (kea_stft_frames, the frames torch.stft transforms),
    torch's real FFT of them, then everything after the FFT in one kernel reading the frame-major spectrum
    (kea_logmel_normalize_frames, each filter's nonzero bins only)."""

    def __init__(self, cfg: EncoderConfig, device, *, fused: bool = False):
        self.cfg = cfg
        self.fused = fused
        self.window = torch.hann_window(cfg.win_length, periodic=False, dtype=torch.float32, device=device)
        left = (cfg.n_fft - cfg.win_length) // 2                 # torch.stft centres a short window in n_fft
        self.window_nfft = torch.zeros(cfg.n_fft, dtype=torch.float32, device=device)
        self.window_nfft[left:left + cfg.win_length] = self.window
        fb = mel_filterbank(cfg)
        self.fb = torch.from_numpy(fb).float().to(device)
        nz = fb != 0
        lo = np.where(nz.any(1), nz.argmax(1), 0)
        hi = np.where(nz.any(1), fb.shape[1] - nz[:, ::-1].argmax(1), 0)
        self.lo = torch.from_numpy(lo.astype(np.int32)).to(device)
        self.hi = torch.from_numpy(hi.astype(np.int32)).to(device)

    def stft_frames(self, audio: Tensor) -> Tensor:
        """audio [B, S] FP32 -> the windowed frames [B, 1 + S // hop, n_fft] that torch.stft (center = True,
        constant padding) transforms, of the pre-emphasised audio (kea_stft_frames)."""
        cfg = self.cfg
        if audio.dim() != 2 or audio.dtype != torch.float32 or not audio.is_contiguous():
            raise ValueError("audio must be a contiguous FP32 tensor [batch, samples]")
        if audio.device != self.window_nfft.device:
            raise ValueError(f"audio is on {audio.device}, the preprocessor on {self.window_nfft.device}")
        b, samples = audio.shape
        out = torch.empty(b, 1 + samples // cfg.hop_length, cfg.n_fft, device=audio.device, dtype=torch.float32)
        rc = _hip.lib().kea_stft_frames(audio.data_ptr(), b, samples, cfg.preemph, self.window_nfft.data_ptr(),
                                        cfg.n_fft, cfg.hop_length, out.data_ptr(), _hip.stream_handle(audio.device))
        _hip.check(rc, "kea_stft_frames")
        return out

    def __call__(self, audio: Tensor) -> Tensor:
        cfg = self.cfg
        frames = frames_for(cfg, audio.shape[1])
        if self.fused:
            spec = torch.fft.rfft(self.stft_frames(audio.contiguous()), dim=-1)   # [B, frames', bins]
            b, ld_f, bins = spec.shape
            y = torch.empty(b, cfg.feat_in, frames, device=audio.device, dtype=torch.float32)
            rc = _hip.lib().kea_logmel_normalize_frames(torch.view_as_real(spec).data_ptr(), b, bins, frames, ld_f,
                                                        self.fb.data_ptr(), self.lo.data_ptr(), self.hi.data_ptr(),
                                                        cfg.feat_in, 2.0 ** -24, 1e-5, y.data_ptr(),
                                                        _hip.stream_handle(audio.device))
            _hip.check(rc, "kea_logmel_normalize_frames")
            return y
        x = torch.cat([audio[:, :1], audio[:, 1:] - cfg.preemph * audio[:, :-1]], dim=1)
        spec = torch.stft(x, n_fft=cfg.n_fft, hop_length=cfg.hop_length, win_length=cfg.win_length,
                          window=self.window, center=True, pad_mode="constant", return_complex=True)
        power = torch.view_as_real(spec[:, :, :frames]).pow(2).sum(-1)          # [B, bins, frames]
        mel = torch.matmul(self.fb, power)                                     # [B, mels, frames]
        logmel = torch.log(mel + 2.0 ** -24)
        mean = logmel.mean(dim=2, keepdim=True)
        std = logmel.std(dim=2, keepdim=True) + 1e-5
        return (logmel - mean) / std


def relative_positions(cfg: EncoderConfig, t: int, device) -> Tensor:
    """Sinusoidal encodings of relative positions t-1 .. -(t-1): [2t-1, d] (NeMo RelPositionalEncoding)."""
    pos = torch.arange(t - 1, -t, -1, dtype=torch.float32, device=device)[:, None]
    div = torch.exp(torch.arange(0, cfg.d_model, 2, dtype=torch.float32, device=device)
                    * (-math.log(10000.0) / cfg.d_model))
    pe = torch.zeros(2 * t - 1, cfg.d_model, device=device)
    pe[:, 0::2] = torch.sin(pos * div)
    pe[:, 1::2] = torch.cos(pos * div)
    return pe


def rel_shift(x: Tensor) -> Tensor:
    """[B, H, T, 2T-1] scores against relative positions -> [B, H, T, T] (Transformer-XL shift, NeMo rel_shift)."""
    b, h, t, p = x.shape
    x = F.pad(x, (1, 0)).view(b, h, p + 1, t)[:, :, 1:].reshape(b, h, t, p)
    return x[..., :t]


# --- fused HIP kernels (include/kea_encoder.h) ----------------------------------------------------------------------

def _f32(name: str, t: Tensor | None, device, numel: int | None = None) -> None:
    """The kernels read FP32 parameters as dense arrays of a known length on the launch device."""
    if t is None:
        return
    if t.dtype != torch.float32 or t.device != device or not t.is_contiguous() or \
            (numel is not None and t.numel() != numel):
        what = f" of {numel} elements" if numel is not None else ""
        raise ValueError(f"{name} must be a contiguous FP32 tensor{what} on {device}")


def _f32_rows(name: str, t: Tensor, device) -> None:
    if t.dtype != torch.float32 or t.device != device:
        raise ValueError(f"{name} must be FP32 on {device}")


def attention_workspace(batch: int, t: int, heads: int, device) -> Tensor | None:
    """A workspace for relpos_attention's key-split form at this shape, or None where it does not apply
    (kea_relpos_attention_workspace). Each call writes both halves' partial outputs and row statistics before they
    are merged, so the buffer is reusable by every later call of the same shape that does not overlap it (it is
    zero-filled once here, which no call relies on)."""
    nbytes = _hip.lib().kea_relpos_attention_workspace(batch, t, heads)
    return torch.zeros(nbytes, dtype=torch.uint8, device=device) if nbytes > 0 else None


def relpos_attention(qkv: Tensor, pos: Tensor, bias_u: Tensor, bias_v: Tensor, heads: int, *,
                     workspace: Tensor | None = None, merged: bool = True) -> Tensor | None:
    """qkv [B, T, 3d] (rows contiguous), pos [2T-1, d] (W_pos of the relative encodings), biases [H, dk] ->
    attention output [B, T, d] (kea_relpos_attention). With `workspace` (from attention_workspace) small grids split
    the keys over two workgroups (kea_relpos_attention_ws); merged=False then leaves the two halves in the workspace
    for attention_merge_quantize and returns None."""
    b, t, three_d = qkv.shape
    d = three_d // 3
    if not merged and workspace is None:
        raise ValueError("merged=False needs the key-split workspace")
    out = torch.empty(b, t, d, device=qkv.device, dtype=torch.float32) if merged else None
    if qkv.stride(2) != 1 or pos.stride(1) != 1 or qkv.stride(0) != t * qkv.stride(1):
        raise ValueError("qkv and pos need contiguous rows")
    if three_d % 3 or d % heads:
        raise ValueError(f"qkv width {three_d} is not 3 x heads x head_dim for {heads} heads")
    if pos.dim() != 2 or pos.shape[0] < 2 * t - 1 or pos.shape[1] < d:
        raise ValueError(f"pos must be [>= {2 * t - 1}, >= {d}] (relative positions t-1 .. -(t-1))")
    _f32_rows("qkv", qkv, qkv.device)
    _f32_rows("pos", pos, qkv.device)
    _f32("bias_u", bias_u, qkv.device, d)
    _f32("bias_v", bias_v, qkv.device, d)
    args = (qkv.data_ptr(), qkv.stride(1), pos.data_ptr(), pos.stride(0), bias_u.data_ptr(), bias_v.data_ptr(),
            _hip.ptr(out), d, b, t, heads, d // heads, 1.0 / math.sqrt(d // heads))
    if workspace is None:
        rc = _hip.lib().kea_relpos_attention(*args, _hip.stream_handle(qkv.device))
    else:
        rc = _hip.lib().kea_relpos_attention_ws(*args, workspace.data_ptr(), workspace.numel(),
                                                _hip.stream_handle(qkv.device))
    _hip.check(rc, "kea_relpos_attention")
    return out


def attention_merge_quantize(workspace: Tensor, batch: int, t: int, heads: int, parts: int) -> tuple[Tensor, Tensor]:
    """The P-part quantization (f32 scales) of the attention output a relpos_attention(..., merged=False) call left
    in `workspace`: bitwise lowbit.quantize of the merged output (kea_attention_merge_quantize). Returns q int8
    [parts, B*T, ldq] (zero padded to ldq = round_up(heads * 128, 16)) and qs [parts, B*T]."""
    m, k = batch * t, heads * 128
    ldq = -(-k // 16) * 16
    q = torch.empty(parts, m, ldq, device=workspace.device, dtype=torch.int8)
    qs = torch.empty(parts, m, device=workspace.device, dtype=torch.float32)
    rc = _hip.lib().kea_attention_merge_quantize(workspace.data_ptr(), workspace.numel(), batch, t, heads, parts,
                                                 q.data_ptr(), ldq, qs.data_ptr(), _hip.stream_handle(workspace.device))
    _hip.check(rc, "kea_attention_merge_quantize")
    return q, qs


def glu_dwconv(x: Tensor, weight: Tensor, bias: Tensor | None) -> Tensor:
    """x [B, T, 2C] (rows contiguous) -> depthwise_conv(GLU(x)) [B, T, C] with weight [C, 1, KW] (kea_glu_dwconv)."""
    b, t, two_c = x.shape
    c, kw = two_c // 2, weight.shape[-1]
    if x.stride(2) != 1 or x.stride(0) != t * x.stride(1) or not weight.is_contiguous():
        raise ValueError("x needs contiguous rows and a contiguous weight")
    _f32_rows("x", x, x.device)
    _f32("weight", weight, x.device, c * kw)
    _f32("bias", bias, x.device, c)
    y = torch.empty(b, t, c, device=x.device, dtype=torch.float32)
    rc = _hip.lib().kea_glu_dwconv(x.data_ptr(), x.stride(1), weight.data_ptr(), _hip.ptr(bias), y.data_ptr(), c,
                                   b, t, c, kw, _hip.stream_handle(x.device))
    _hip.check(rc, "kea_glu_dwconv")
    return y


def norm_quantize(x: Tensor, norm0, norm1, parts: int, *, out: Tensor | None = None) -> tuple[Tensor, Tensor, Tensor]:
    """x [B, T, K] contiguous -> (LayerNorm0(x), q, qs): q / qs the P-part quantization of LayerNorm1(LayerNorm0(x))
    (kea_norm_quantize). `out` (contiguous like x, may be x itself) receives LayerNorm0(x)."""
    b, t, k = x.shape
    m = b * t
    ldq = lowbit.round_up(k, 16)
    if not x.is_contiguous() or (out is not None and (not out.is_contiguous() or out.shape != x.shape)):
        raise ValueError("x and out must be contiguous [B, T, K]")
    _f32_rows("x", x, x.device)
    if out is not None:
        _f32_rows("out", out, x.device)
    for name, v in (("norm0.weight", norm0.weight), ("norm0.bias", norm0.bias), ("norm1.weight", norm1.weight),
                    ("norm1.bias", norm1.bias)):
        _f32(name, v, x.device, k)
    out = torch.empty_like(x) if out is None else out
    q = torch.empty(parts, m, ldq, device=x.device, dtype=torch.int8)
    qs = torch.empty(parts, m, device=x.device, dtype=torch.float32)
    rc = _hip.lib().kea_norm_quantize(x.data_ptr(), k, m, k, norm0.weight.data_ptr(), norm0.bias.data_ptr(),
                                      float(norm0.eps), out.data_ptr(), k, norm1.weight.data_ptr(),
                                      norm1.bias.data_ptr(), float(norm1.eps), parts, q.data_ptr(), ldq,
                                      qs.data_ptr(), _hip.stream_handle(x.device))
    _hip.check(rc, "kea_norm_quantize")
    return out, q, qs


def glu_dwconv_quantize(x: Tensor, weight: Tensor, bias: Tensor | None, parts: int) -> tuple[Tensor, Tensor]:
    """x [B, T, 2C] (rows contiguous) -> the P-part quantization (q, qs) of silu(depthwise_conv(GLU(x)))
    (kea_glu_dwconv_quantize)."""
    b, t, two_c = x.shape
    c, kw = two_c // 2, weight.shape[-1]
    if x.stride(2) != 1 or x.stride(0) != t * x.stride(1) or not weight.is_contiguous():
        raise ValueError("x needs contiguous rows and a contiguous weight")
    _f32_rows("x", x, x.device)
    _f32("weight", weight, x.device, c * kw)
    _f32("bias", bias, x.device, c)
    ldq = lowbit.round_up(c, 16)
    q = torch.empty(parts, b * t, ldq, device=x.device, dtype=torch.int8)
    qs = torch.empty(parts, b * t, device=x.device, dtype=torch.float32)
    rc = _hip.lib().kea_glu_dwconv_quantize(x.data_ptr(), x.stride(1), weight.data_ptr(), _hip.ptr(bias), b, t, c, kw,
                                            parts, q.data_ptr(), ldq, qs.data_ptr(), _hip.stream_handle(x.device))
    _hip.check(rc, "kea_glu_dwconv_quantize")
    return q, qs


def dwconv_quantize(u: Tensor, weight: Tensor, bias: Tensor | None, parts: int) -> tuple[Tensor, Tensor]:
    """u [B, T, C] GLU values (rows contiguous) -> the P-part quantization (q, qs) of silu(depthwise_conv(u))
    (kea_dwconv_quantize)."""
    b, t, c = u.shape
    kw = weight.shape[-1]
    if u.stride(2) != 1 or u.stride(0) != t * u.stride(1) or not weight.is_contiguous():
        raise ValueError("u needs contiguous rows and a contiguous weight")
    _f32_rows("u", u, u.device)
    _f32("weight", weight, u.device, c * kw)
    _f32("bias", bias, u.device, c)
    ldq = lowbit.round_up(c, 16)
    q = torch.empty(parts, b * t, ldq, device=u.device, dtype=torch.int8)
    qs = torch.empty(parts, b * t, device=u.device, dtype=torch.float32)
    rc = _hip.lib().kea_dwconv_quantize(u.data_ptr(), u.stride(1), weight.data_ptr(), _hip.ptr(bias), b, t, c, kw,
                                        parts, q.data_ptr(), ldq, qs.data_ptr(), _hip.stream_handle(u.device))
    _hip.check(rc, "kea_dwconv_quantize")
    return q, qs


def glu_interleave(rows: Tensor) -> Tensor:
    """Rows [2C, ...] of a GLU input projection (value half, then gate half) -> value, gate, value, ... order, the
    pair layout of the GEMM's GLU epilogue."""
    c = rows.shape[0] // 2
    idx = torch.stack([torch.arange(c), torch.arange(c) + c], 1).reshape(-1)
    return rows[idx.to(rows.device)].contiguous()


# --- the encoder -----------------------------------------------------------------------------------------------------

class _DenseLinear:
    """FP32 dense stand-in for a quantized linear: signs * alpha (exact in FP32), y = z W^T."""

    def __init__(self, codes: Tensor, scale: Tensor, k: int, device):
        self.w = bits.dense_weight(codes, scale, k, dtype=torch.float32).to(device)
        self.out_features, self.in_features = self.w.shape

    def __call__(self, x, *, activation="", norm=None, input_activation=""):
        z = x
        if norm is not None:
            z = F.layer_norm(z, norm[0].shape, norm[0], norm[1], norm[2])
        if input_activation == "silu":
            z = F.silu(z)
        y = torch.matmul(z, self.w.t())
        return F.silu(y) if activation == "silu" else y


class _Norm:
    """LayerNorm parameters in the shape the quantizer's fused LayerNorm reads (weight, bias, eps)."""

    def __init__(self, weight: Tensor, bias: Tensor, eps: float):
        self.weight, self.bias, self.eps = weight, bias, eps
        self.normalized_shape = (weight.numel(),)


class FastConformerEncoder:
    """audio [B, S] -> encoder output [B, T', d]. parts = int8 activation parts of every quantized linear (1 = the
    Kea-B x1 mode); dense=True swaps the quantized linears for FP32 dense matmuls (the parity reference);
    fused=False runs attention and the GLU + depthwise convolution as PyTorch ops instead of the fused HIP kernels
    (the dense twin always does)."""

    def __init__(self, weights: dict, cfg: EncoderConfig = EncoderConfig(), device="cuda", *, parts: int = 1,
                 dense: bool = False, fused: bool = True):
        self.cfg, self.parts, self.dense = cfg, parts, dense
        self.fused = fused and not dense
        self._sub_out = None
        self.device = device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            self.device = device = torch.device("cuda", torch.cuda.current_device())
        self.pre = Preprocessor(cfg, device, fused=fused and not dense)
        dev = lambda t: t.to(device=device, dtype=torch.float32)  # noqa: E731
        p = "encoder.pre_encode."
        self.sub = {k[len(p):]: dev(v) for k, v in weights.items() if k.startswith(p)}
        self.layers = []
        self._pos_cache: dict = {}
        self._att_ws: dict = {}  # (batch, t) -> key-split attention workspace (or None)
        shapes = quantized_shapes(cfg)
        quantized = {}
        for layer in range(cfg.layers):
            pre = f"encoder.layers.{layer}."
            fp = {}
            for norm in ("norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2", "norm_out"):
                fp[norm] = _Norm(dev(weights[pre + norm + ".weight"]), dev(weights[pre + norm + ".bias"]), cfg.eps)
            fp["u"] = dev(weights[pre + "self_attn.pos_bias_u"])
            fp["v"] = dev(weights[pre + "self_attn.pos_bias_v"])
            # BatchNorm (inference) folded into the depthwise convolution: w' = w * g / sqrt(var + eps),
            # b' = beta - mean * g / sqrt(var + eps)
            gain = weights[pre + "conv.batch_norm.weight"] / torch.sqrt(weights[pre + "conv.batch_norm.running_var"]
                                                                         + cfg.eps)
            fp["dw_w"] = dev(weights[pre + "conv.depthwise_conv.weight"] * gain[:, None, None])
            fp["dw_b"] = dev(weights[pre + "conv.batch_norm.bias"] - weights[pre + "conv.batch_norm.running_mean"] * gain)
            self.layers.append(fp)
            for suffix, (n, k, kind) in shapes.items():
                codes, scale = weights[pre + suffix + ".codes"], weights[pre + suffix + ".scale"]
                if self.fused and suffix == "conv.pointwise_conv1":  # value / gate row pairs for the GLU epilogue
                    codes, scale = glu_interleave(codes), glu_interleave(scale)
                quantized[pre + suffix] = (codes, scale, None, kind, k)
        if dense:
            self.linears = {name: _DenseLinear(codes, scale, k, device)
                            for name, (codes, scale, _, _, k) in quantized.items()}
            for layer in range(cfg.layers):
                pre = f"encoder.layers.{layer}.self_attn."
                parts = [self.linears[pre + x] for x in provider.QKV]
                fused = _DenseLinear.__new__(_DenseLinear)
                fused.w = torch.cat([x.w for x in parts])
                fused.out_features, fused.in_features = fused.w.shape
                self.linears[pre + "qkv"] = fused
            self.table = None
        else:
            self.table, modules = provider.prepare_table(quantized, layer_parts.LAYERS[parts], device)
            self.project = provider.PartCount(provider.BinaryProjection(self.table), parts)
            self.modules = modules
            self._fused = {}
            for layer in range(cfg.layers):
                pre = f"encoder.layers.{layer}.self_attn."
                handle = torch.cat([modules[pre + x].packed_t for x in provider.QKV], 1)
                self._fused[pre + "qkv"] = type("FusedQKV", (), {"packed_t": handle})()

    # one quantized linear through the provider seam (or its dense stand-in)
    def _linear(self, name: str, x: Tensor, *, activation="", norm=None, input_activation="") -> Tensor:
        if self.dense:
            nt = None if norm is None else (norm.weight, norm.bias, norm.eps)
            return self.linears[name](x, activation=activation, norm=nt, input_activation=input_activation)
        mod = self._fused.get(name) or self.modules[name]
        return self.project(x, mod, False, self.parts, activation, norm, None, input_activation)

    def _residual(self, name: str, z: Tensor, r: Tensor, factor: float, *, input_activation="") -> Tensor:
        """r + factor * linear(z). Quantized: the residual add runs in the GEMM epilogue, in place into r
        (kea_lowbit_gemm_residual; r is not used afterwards). Dense: PyTorch."""
        if self.dense:
            return torch.add(r, self._linear(name, z, input_activation=input_activation), alpha=factor)
        layer = self.modules[name]._segment.layer
        b, t, k = z.shape
        m, n = b * t, layer.out_features
        q, qs, _ = lowbit.quantize(z, (z.stride(0), z.stride(1), z.stride(2), t), m, k, self.parts,
                                   input_activation=input_activation)
        r2 = r.view(m, n)
        lowbit.gemm(layer.WBITS, q, qs, layer.words, n, k, layer.scale, layer.bias, r2, None, residual=r2,
                    residual_factor=factor)
        return r

    def _layer(self, name: str):
        """The prepared layer behind `name` (the fused QKV handle resolves through the provider's table)."""
        mod = self._fused.get(name)
        if mod is None:
            return self.modules[name]._segment.layer
        segment, offset, count = self.project.resolve(mod)
        if offset or count != segment.out_features:
            raise ValueError(f"{name} does not cover a whole prepared layer")
        return segment.layer

    def _gemm(self, name: str, q: Tensor, qs: Tensor, m: int, *, silu: bool = False, glu: bool = False) -> Tensor:
        """The quantized linear `name` on pre-quantized activations (q, qs): FP32 [m, N] (glu: [m, N/2])."""
        layer = self._layer(name)
        n = layer.out_features
        y = torch.empty(m, n // 2 if glu else n, device=self.device, dtype=torch.float32)
        lowbit.gemm(layer.WBITS, q, qs, layer.words, n, layer.in_features, layer.scale, layer.bias, y, None,
                    silu=silu, glu=glu)
        return y

    def weight_bytes(self) -> int:
        return 0 if self.table is None else self.table.weight_bytes()

    def subsample(self, feats: Tensor) -> Tensor:
        """[B, mels, frames] -> [B, T', d] (dw-striding x8, then the output linear).

        Fused (quantized) path: the first convolution + ReLU + first depthwise convolution in one kernel
        (kea_subsample_front), the pointwise convolutions as batched matrix products whose bias + ReLU are applied
        by the next kernel on load, the second depthwise convolution (kea_dwconv2d_s2), the last bias + ReLU with the
        (channel, frequency) flatten (kea_bias_relu_flatten), and the output linear as one matrix product. Otherwise
        PyTorch's own convolution kernels (the library-convolution path is switched off: its algorithm choice varied
        from box to box, by up to 10x on the first 3x3 convolution)."""
        s = self.sub
        c = self.cfg.sub_channels
        if self.fused:
            return self._subsample_fused(feats)
        with torch.backends.cudnn.flags(enabled=False):
            x = feats.transpose(1, 2).unsqueeze(1)                                    # [B, 1, frames, mels]
            x = F.relu(F.conv2d(x, s["conv.0.weight"], s["conv.0.bias"], stride=2, padding=1))
            for i in (2, 5):
                x = F.conv2d(x, s[f"conv.{i}.weight"], s[f"conv.{i}.bias"], stride=2, padding=1, groups=c)
                x = F.relu(F.conv2d(x, s[f"conv.{i + 1}.weight"], s[f"conv.{i + 1}.bias"]))
        b, _, t, f = x.shape
        x = x.transpose(1, 2).reshape(b, t, c * f)
        return F.linear(x, s["out.weight"], s["out.bias"])

    def _subsample_fused(self, feats: Tensor) -> Tensor:
        s, c = self.sub, self.cfg.sub_channels
        feats = feats.contiguous()
        b, f, t = feats.shape
        t1, f1 = (t - 1) // 2 + 1, (f - 1) // 2 + 1
        t2, f2 = (t1 - 1) // 2 + 1, (f1 - 1) // 2 + 1
        t3, f3 = (t2 - 1) // 2 + 1, (f2 - 1) // 2 + 1
        L = _hip.lib()
        st = _hip.stream_handle(feats.device)
        x1 = torch.empty(b, c, t2, f2, device=feats.device, dtype=torch.float32)
        _hip.check(L.kea_subsample_front(feats.data_ptr(), b, t, f, s["conv.0.weight"].data_ptr(),
                                         s["conv.0.bias"].data_ptr(), s["conv.2.weight"].data_ptr(),
                                         s["conv.2.bias"].data_ptr(), c, x1.data_ptr(), st), "kea_subsample_front")
        p1 = torch.matmul(s["conv.3.weight"].view(c, c), x1.view(b, c, t2 * f2))           # [B, C, t2*f2]
        x2 = torch.empty(b, c, t3, f3, device=feats.device, dtype=torch.float32)
        _hip.check(L.kea_dwconv2d_s2(p1.data_ptr(), s["conv.3.bias"].data_ptr(), s["conv.5.weight"].data_ptr(),
                                     s["conv.5.bias"].data_ptr(), x2.data_ptr(), b, c, t2, f2, st), "kea_dwconv2d_s2")
        p2 = torch.matmul(s["conv.6.weight"].view(c, c), x2.view(b, c, t3 * f3))           # [B, C, t3*f3]
        flat = torch.empty(b, t3, c * f3, device=feats.device, dtype=torch.float32)
        _hip.check(L.kea_bias_relu_flatten(p2.data_ptr(), s["conv.6.bias"].data_ptr(), flat.data_ptr(), b, c, t3,
                                           f3, st), "kea_bias_relu_flatten")
        if self._sub_out is None:  # the x sqrt(d) scaling folded into the output linear
            g = math.sqrt(self.cfg.d_model) if self.cfg.xscaling else 1.0
            self._sub_out = ((s["out.weight"] * g).contiguous(), (s["out.bias"] * g).contiguous())
        return F.linear(flat, *self._sub_out)

    def positions(self, t: int) -> list:
        """W_pos applied to the relative encodings, per layer, for length t: [2t-1, d] each. Frozen per length
        (the reference freezes them for graph capture too, kk/ternary/transforms.py:18-21); computed with the same
        quantized GEMM as every other call."""
        hit = self._pos_cache.get(t)
        if hit is None:
            cfg = self.cfg
            pe = relative_positions(cfg, t, self.device).unsqueeze(0)
            hit = [self._linear(f"encoder.layers.{layer}.self_attn.linear_pos", pe)[0].contiguous()
                   for layer in range(cfg.layers)]
            self._pos_cache[t] = hit
        return hit

    @contextlib.contextmanager
    def attention_workspaces(self, table: dict):
        """Forward calls inside the block take their key-split attention workspaces from `table` ((batch, t) ->
        workspace, filled on first use) instead of the encoder's shared table. EncoderGraph gives each graph its own,
        so graphs replayed on different streams, and eager calls, never share one. Eager calls of one encoder that
        overlap on different streams must each run inside their own table."""
        saved = self._att_ws
        self._att_ws = table
        try:
            yield
        finally:
            self._att_ws = saved

    def _attention_ws(self, b: int, t: int) -> Tensor | None:
        """The key-split attention workspace of this shape (None where the split does not apply), allocated on the
        first forward of the shape (the eager warm-up, before any graph capture)."""
        key = (b, t)
        if key not in self._att_ws:
            self._att_ws[key] = attention_workspace(b, t, self.cfg.heads, self.device)
        return self._att_ws[key]

    def _attention_quantized(self, qkv: Tensor, pos: Tensor, u: Tensor, v_bias: Tensor) -> tuple[Tensor, Tensor]:
        """The attention output as the P-part input of the output projection. Where the key split applies its two
        halves are merged inside the quantizer (the merged FP32 output is never written)."""
        b, t, _ = qkv.shape
        ws = self._attention_ws(b, t) if self.cfg.d_model // self.cfg.heads == 128 else None
        if ws is None:
            return self._quantize(self.attention(qkv, pos, u, v_bias))
        relpos_attention(qkv, pos, u, v_bias, self.cfg.heads, workspace=ws, merged=False)
        return attention_merge_quantize(ws, b, t, self.cfg.heads, self.parts)

    def attention(self, qkv: Tensor, pos: Tensor, u: Tensor, v_bias: Tensor) -> Tensor:
        b, t, _ = qkv.shape
        h = self.cfg.heads
        dk = self.cfg.d_model // h
        if self.fused and t <= 256 and dk == 128:
            return relpos_attention(qkv, pos, u, v_bias, h, workspace=self._attention_ws(b, t))
        pos_t = pos.view(2 * t - 1, h, dk).permute(1, 2, 0).contiguous()  # [H, dk, 2t-1]
        q, k, v = qkv.view(b, t, 3, h, dk).unbind(2)
        qu = (q + u).transpose(1, 2).contiguous()                                   # [B, H, T, dk]
        qv = (q + v_bias).transpose(1, 2).contiguous()
        kt = k.permute(0, 2, 3, 1).contiguous()                                     # [B, H, dk, T]
        ac = torch.matmul(qu, kt)
        bd = rel_shift(torch.matmul(qv, pos_t))                                     # [B, H, T, T]
        attn = torch.softmax((ac + bd) * (1.0 / math.sqrt(dk)), dim=-1)
        out = torch.matmul(attn, v.transpose(1, 2).contiguous())                    # [B, H, T, dk]
        return out.transpose(1, 2).reshape(b, t, h * dk)

    def _quantize(self, z: Tensor, *, norm=None) -> tuple[Tensor, Tensor]:
        """The P-part quantization of the rows of z ([B, T, K] or [M, K], unit element stride)."""
        z3 = z if z.dim() == 3 else z.unsqueeze(0)
        b, t, k = z3.shape
        q, qs, _ = lowbit.quantize(z3, (z3.stride(0), z3.stride(1), z3.stride(2), t), b * t, k, self.parts, norm=norm)
        return q, qs

    def _block(self, name: str, q: Tensor, qs: Tensor, r: Tensor, factor: float, *, norm=None, out_norm=None):
        """r <- out_norm(r + factor * linear(q)) in place; with `norm`, returns the next projection's (q, qs) = the
        P-part quantization of norm(r). The residual add runs in the GEMM epilogue, the LayerNorm(s) + quantization
        in one row kernel (kea_norm_quantize / kea_quantize)."""
        layer = self._layer(name)
        b, t, n = r.shape
        r2 = r.view(b * t, n)
        lowbit.gemm(layer.WBITS, q, qs, layer.words, n, layer.in_features, layer.scale, layer.bias, r2, None,
                    residual=r2, residual_factor=factor)
        if out_norm is not None:
            # the output LayerNorm in the library's summation order; after the last layer (no next LayerNorm) the
            # quantization that comes with it is not used
            _, q2, qs2 = norm_quantize(r, out_norm, norm or out_norm, self.parts, out=r)
            return (q2, qs2) if norm is not None else None
        return self._quantize(r, norm=norm) if norm is not None else None

    def _layer_rows(self, i: int, x: Tensor, pos: Tensor, xq=None):
        """The fused layer: each residual block ends in one row epilogue that also quantizes the next block's
        input (the reference's row_fusions forward, kk/ternary/row_fusion.py:121-152). x is updated in place."""
        fp = self.layers[i]
        pre = f"encoder.layers.{i}."
        b, t, _ = x.shape
        m = b * t
        if xq is None:
            xq = self._quantize(x, norm=fp["norm_feed_forward1"])
        y = self._gemm(pre + "feed_forward1.linear1", *xq, m, silu=True)
        xq = self._block(pre + "feed_forward1.linear2", *self._quantize(y), x, 0.5, norm=fp["norm_self_att"])
        qkv = self._gemm(pre + "self_attn.qkv", *xq, m).view(b, t, -1)
        xq = self._block(pre + "self_attn.linear_out", *self._attention_quantized(qkv, pos, fp["u"], fp["v"]), x, 1.0,
                         norm=fp["norm_conv"])
        u = self._gemm(pre + "conv.pointwise_conv1", *xq, m, glu=True).view(b, t, -1)   # GLU in the epilogue
        xq = self._block(pre + "conv.pointwise_conv2", *dwconv_quantize(u, fp["dw_w"], fp["dw_b"], self.parts),
                         x, 1.0, norm=fp["norm_feed_forward2"])
        y = self._gemm(pre + "feed_forward2.linear1", *xq, m, silu=True)
        following = self.layers[i + 1]["norm_feed_forward1"] if i + 1 < self.cfg.layers else None
        xq = self._block(pre + "feed_forward2.linear2", *self._quantize(y), x, 0.5, norm=following,
                         out_norm=fp["norm_out"])
        return x, xq

    def layer(self, i: int, x: Tensor, pos: Tensor, xq=None) -> Tensor | tuple:
        """One layer. Fused (quantized, fused=True): returns (x, xq) with x updated in place and xq = (q, qs) the
        next layer's quantized input (None after the last layer). Otherwise returns the layer output."""
        if self.fused:
            return self._layer_rows(i, x, pos, xq)
        fp = self.layers[i]
        pre = f"encoder.layers.{i}."
        y = self._linear(pre + "feed_forward1.linear1", x, norm=fp["norm_feed_forward1"], activation="silu")
        r = self._residual(pre + "feed_forward1.linear2", y, x, 0.5)
        qkv = self._linear(pre + "self_attn.qkv", r, norm=fp["norm_self_att"])
        r = self._residual(pre + "self_attn.linear_out", self.attention(qkv, pos, fp["u"], fp["v"]), r, 1.0)
        z = self._linear(pre + "conv.pointwise_conv1", r, norm=fp["norm_conv"])
        z = F.glu(z, dim=-1)                                                    # a * sigmoid(g)
        z = F.conv1d(z.transpose(1, 2), fp["dw_w"], fp["dw_b"], padding=self.cfg.conv_kernel // 2,
                     groups=self.cfg.d_model).transpose(1, 2)
        r = self._residual(pre + "conv.pointwise_conv2", z, r, 1.0, input_activation="silu")
        y = self._linear(pre + "feed_forward2.linear1", r, norm=fp["norm_feed_forward2"], activation="silu")
        r = self._residual(pre + "feed_forward2.linear2", y, r, 0.5)
        n = fp["norm_out"]
        return F.layer_norm(r, n.normalized_shape, n.weight, n.bias, n.eps)

    def encode(self, feats: Tensor) -> Tensor:
        x = self.subsample(feats)
        if self.cfg.xscaling and not self.fused:  # the fused subsampling applies it in its output linear
            x = x * math.sqrt(self.cfg.d_model)
        pos = self.positions(x.shape[1])
        xq = None
        for i in range(self.cfg.layers):
            out = self.layer(i, x, pos[i], xq)
            x, xq = out if isinstance(out, tuple) else (out, None)
        return x

    @torch.inference_mode()
    def __call__(self, audio: Tensor) -> Tensor:
        return self.encode(self.pre(audio))


class EncoderGraph:
    """One HIP graph of preprocessing + encoder for a fixed (batch, samples); __call__ copies the audio into the
    graph's input buffer, replays and returns the graph's output buffer (overwritten by the next call). The graph owns
    its input, its key-split attention workspace (FastConformerEncoder.attention_workspaces) and its output."""

    def __init__(self, encoder: FastConformerEncoder, batch: int, samples: int, *, warmup: int = 2):
        self.encoder = encoder
        dev = encoder.device
        self.audio = torch.zeros(batch, samples, device=dev)
        self.stream = torch.cuda.Stream(dev)
        self.workspaces: dict = {}
        with torch.inference_mode(), encoder.attention_workspaces(self.workspaces):
            encoder.positions(encoded_length(frames_for(encoder.cfg, samples)))
            self.stream.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(self.stream):
                for _ in range(warmup):
                    encoder(self.audio)
            torch.cuda.synchronize(dev)
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph, stream=self.stream):
                self.out = encoder(self.audio)
        torch.cuda.synchronize(dev)

    def replay(self) -> Tensor:
        """Replays on the graph's stream, ordered after the caller's current stream and before its later work."""
        caller = torch.cuda.current_stream(self.audio.device)
        self.stream.wait_stream(caller)
        with torch.cuda.stream(self.stream):
            self.graph.replay()
        caller.wait_stream(self.stream)
        return self.out

    def __call__(self, audio: Tensor) -> Tensor:
        caller = torch.cuda.current_stream(self.audio.device)
        self.stream.wait_stream(caller)
        with torch.cuda.stream(self.stream):
            self.audio.copy_(audio)
            self.graph.replay()
        caller.wait_stream(self.stream)
        return self.out


class EncoderGraphCache:
    """Up to max_graphs HIP graphs of one encoder, one per (audio shape, dtype, device, caller stream): the
    reference's bounded encoder graph cache (kk/ternary/graphs.py:11-65). The first call of a key warms up and captures
    an EncoderGraph (its own input, attention workspace and output); later calls copy the audio in and replay it.
    Keys past the limit, CPU audio, calls with grad enabled and calls made while the current stream is capturing run
    the encoder eagerly. Every call returns a tensor the caller owns (a copy of the graph's output)."""

    def __init__(self, encoder: FastConformerEncoder, max_graphs: int = 4, *, warmup: int = 2):
        if max_graphs < 1:
            raise ValueError("max_graphs must be positive")
        self.encoder, self.max_graphs, self.warmup = encoder, max_graphs, warmup
        self.entries: dict = {}

    def __call__(self, audio: Tensor) -> Tensor:
        if (not audio.is_cuda or audio.dim() != 2 or torch.is_grad_enabled()
                or torch.cuda.is_current_stream_capturing()):
            return self.encoder(audio)
        stream = torch.cuda.current_stream(audio.device)
        key = (tuple(audio.shape), audio.dtype, audio.device, stream.cuda_stream)
        graph = self.entries.get(key)
        if graph is None:
            if len(self.entries) >= self.max_graphs:
                return self.encoder(audio)
            graph = self.entries[key] = EncoderGraph(self.encoder, audio.shape[0], audio.shape[1], warmup=self.warmup)
        return graph(audio).clone()

    def clear(self) -> None:
        """Releases the graphs after the work queued on their devices has finished."""
        for device in {graph.audio.device for graph in self.entries.values()}:
            torch.cuda.synchronize(device)
        self.entries.clear()
