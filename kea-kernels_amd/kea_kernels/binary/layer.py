"""Int8MmaLayer: 1-bit weights resident in the gfx950 native layout, residual int8 activations, int8 MFMA.

Drop-in for the reference's operator (kk/binary/layer.py:29-209): the same prepare / linear / conv / dot / project
methods with the same argument meaning and errors, plus gfx950 extras as keyword arguments (fp16/bf16 outputs via the
dtype of `y`, fp16 per-token scales via the dtype of `qs`, raw int32 accumulators via `acc_out`). Two launches per
call, both on the current stream and both graph-capturable (no allocation inside the library, no host sync):
  1. kea_quantize: x (any strides) -> q int8 [P, M, ldq] + qs [P, M] (LayerNorm / input SiLU fused for `project`);
  2. kea_lowbit_gemm: the 1-bit x int8 GEMM with the fused epilogue.
The layer resolves each call layout once (lowbit.Launches: a projection plan per layout, the buffers bound per call),
so a repeated linear / conv call with the same input shape, strides, dtype and output dtype pays one C call that
enqueues both launches and two allocations (output and workspace), not the argument checks.
There is no slow fallback layout: every shape runs the MFMA kernel (the native layout pads N to 16 and K to 128).
"""
from __future__ import annotations

import math

import torch
from torch import Tensor

from kea_kernels import _hip, lowbit
from kea_kernels.binary import bits as api
from kea_kernels.binary import kernels

round_up = lowbit.round_up


class Int8MmaLayer:
    """One layer resident as native 1-bit words plus FP32 scale / bias. Calls use three activation parts (x3), as
    the reference's Int8MmaLayer; Int8MmaPartsLayer (layer_parts.py) makes the part count a class attribute."""

    PARTS = 3
    WBITS = 1

    def __init__(self, n: int, k: int, device: torch.device, words: Tensor, scale: Tensor, bias: Tensor | None):
        self.out_features, self.in_features, self.device = n, k, device
        self.words, self.scale, self.bias = words, scale, bias
        self.codes = None  # the reference keeps raw codes only for its fallback layout; this build has none

    @classmethod
    def prepare(cls, codes: Tensor, scale: Tensor, bias: Tensor | None, in_features: int, device) -> "Int8MmaLayer":
        """Validate export codes uint8 [N, ceil(K/8)] and FP32 scale / bias [N]; make the only GPU copies."""
        n, k = api.validate_weights(codes, scale, bias, in_features)
        device = torch.device(device)
        if device.type != "cuda":
            raise ValueError("Int8MmaLayer runs on GPU devices only")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        with torch.no_grad():
            words = kernels.relayout_codes(codes, k, 1).to(device)
            scale = scale.to(device=device, dtype=torch.float32, copy=True).contiguous()
            bias = None if bias is None else bias.to(device=device, dtype=torch.float32, copy=True).contiguous()
        return cls(n, k, device, words, scale, bias)

    @property
    def fast(self) -> bool:
        return True

    @property
    def launches(self) -> lowbit.Launches:
        """The layer's launches resolved once per call layout (lowbit.Launches), rebuilt if the weights change."""
        cache = self.__dict__.get("_launches")
        if (cache is None or cache.words is not self.words or cache.wscale is not self.scale
                or cache.bias is not self.bias):
            cache = lowbit.Launches(self.WBITS, self.words, self.out_features, self.in_features, self.scale,
                                    self.bias)
            self.__dict__["_launches"] = cache
        return cache

    def weight_bytes(self) -> int:
        return api.resident_bytes(self.words, self.scale, self.bias)

    # --- calls ------------------------------------------------------------------------------------------------
    def _check(self, x: Tensor, kind: str) -> None:
        if not isinstance(x, Tensor):
            raise ValueError("input must be a tensor")
        if x.dtype not in (torch.float32, torch.float16):
            raise ValueError(f"expected FP32 input, got {x.dtype}")
        if x.device != self.device:
            raise ValueError(f"input on {x.device}, layer on {self.device}")
        if kind == "linear" and (x.dim() < 1 or x.shape[-1] != self.in_features):
            raise ValueError(f"expected [..., {self.in_features}] input, got {tuple(x.shape)}")
        if kind == "conv" and (x.dim() != 3 or x.shape[1] != self.in_features):
            raise ValueError(f"expected [B, {self.in_features}, T] input, got {tuple(x.shape)}")
        if torch.is_grad_enabled() and x.requires_grad:
            raise RuntimeError("Int8MmaLayer is inference only: input requires grad")

    def linear(self, x: Tensor, *, out_dtype: torch.dtype = torch.float32) -> Tensor:
        """[..., K] -> [..., N] (FP32 unless out_dtype says otherwise)."""
        launches, key = self.launches, _call_key(x, out_dtype, "linear")
        hit = launches.recall(key)
        if hit is not None and not (x.requires_grad and torch.is_grad_enabled()):
            # a layout checked and resolved before: everything checked derives from the key
            y = torch.empty(hit[1], device=self.device, dtype=out_dtype)
            launches.launch(hit[0], x, y)
            return y
        self._check(x, "linear")
        lead = tuple(x.shape[:-1])
        m = math.prod(lead)
        y = torch.empty(*lead, self.out_features, device=self.device, dtype=out_dtype)
        if m:
            xr = x
            if x.dim() == 1:
                rows = (0, 0, x.stride(0), 1)
            elif x.dim() == 2:
                rows = (0, x.stride(0), x.stride(1), m)
            else:
                xr = x.reshape(-1, x.shape[-2], x.shape[-1])
                rows = (xr.stride(0), xr.stride(1), xr.stride(2), xr.shape[1])
            e = self._run(xr, rows, m, y.view(m, self.out_features))
            if e and key is not None and xr.data_ptr() == x.data_ptr():  # not where the reshape copied x
                launches.remember(key, e, y.shape)
        return y

    def conv(self, x: Tensor, *, out_dtype: torch.dtype = torch.float32) -> Tensor:
        """Pointwise convolution [B, K, T] -> [B, N, T] (a transposed view of a [B, T, N] result)."""
        launches, key = self.launches, _call_key(x, out_dtype, "conv")
        hit = launches.recall(key)
        if hit is not None and not (x.requires_grad and torch.is_grad_enabled()):
            y = torch.empty(hit[1], device=self.device, dtype=out_dtype)
            launches.launch(hit[0], x, y)
            return y.transpose(1, 2)
        self._check(x, "conv")
        b, _, t = x.shape
        y = torch.empty(b, t, self.out_features, device=self.device, dtype=out_dtype)
        if b * t:
            e = self._run(x, (x.stride(0), x.stride(2), x.stride(1), t), b * t, y.view(b * t, self.out_features))
            if e and key is not None:
                launches.remember(key, e, y.shape)
        return y.transpose(1, 2)

    def _run(self, x: Tensor, rows: tuple, m: int, y: Tensor):
        """The layer's parts of x's rows into y [m, N]; returns the cached launch entry used, or None."""
        e = self.launches.project(x, rows, m, self.PARTS, y)
        if not e:
            q, qs, ldq = quantize(x, rows, m, self.in_features, parts=self.PARTS)
            self.dot(q, qs, ldq, m, y)
            return None
        return e

    def dot(self, q: Tensor, qs: Tensor, ldq: int, m: int, y: Tensor | None, *, silu: bool = False, config=None,
            order: int = 0, acc_out: Tensor | None = None) -> None:
        """y[:m] (row-major, row stride y.stride(0); f32, f16 or bf16) from q int8 [P, m, ldq] and qs [P, m]."""
        dot(self, q, qs, ldq, m, y, silu=silu, config=config, order=order, acc_out=acc_out)

    def project(self, x: Tensor, *, conv: bool = False, components: int = 3, activation: str = "", norm=None,
                input_activation: str = "") -> Tensor:
        """The fused provider op: quantize (LayerNorm / input SiLU fused) + GEMM (+ SiLU epilogue), FP32 out.

        Semantics of the reference's provider seam (kk/binary/provider.py:3-15): x [B, T, K] (or [T, K]), or
        [B, K, T] with conv=True (returns a [B, N, T] view)."""
        if components != self.PARTS and type(self) is Int8MmaLayer:
            raise ValueError("Int8MmaLayer implements INT8x3 arithmetic only (components=3)")
        return _project(self, x, conv, components, activation, norm, input_activation)


def _call_key(x, out_dtype, kind: str):
    """A linear / conv call's layout: x's shape, strides, dtype and device and the output dtype determine every
    argument the call checks and launches with (the rows are x's own); None for a non-tensor (the checks raise)."""
    try:
        return (kind, x.shape, x.stride(), x.dtype, x.device, out_dtype)
    except (AttributeError, TypeError, RuntimeError):  # not a strided tensor
        return None


def _project(layer: Int8MmaLayer, x: Tensor, conv: bool, parts: int, activation: str, norm,
             input_activation: str) -> Tensor:
    if activation not in ("", "silu") or input_activation not in ("", "silu"):
        raise ValueError(f"unsupported activation {activation!r} / {input_activation!r}")
    xx = x.transpose(1, 2) if conv else x
    layer._check(xx, "linear")
    if xx.dim() == 2:
        xx = xx.unsqueeze(0)
    if xx.dim() != 3:
        raise ValueError("project expects [B, T, K] (or [T, K]) input")
    b, t, k = xx.shape
    m, n = b * t, layer.out_features
    y = torch.empty(b, t, n, device=layer.device, dtype=torch.float32)
    if m:
        rows = (xx.stride(0), xx.stride(1), xx.stride(2), t)
        if not layer.launches.project(xx, rows, m, parts, y.view(m, n), silu=activation == "silu", norm=norm,
                                      input_activation=input_activation):
            q, qs, ldq = lowbit.quantize(xx, rows, m, k, parts, norm=norm, input_activation=input_activation)
            layer.dot(q, qs, ldq, m, y.view(m, n), silu=activation == "silu")
    if conv:
        return y.transpose(1, 2)
    return y if x.dim() == 3 else y.view(*x.shape[:-1], n)


def quantize(x: Tensor, rows: tuple, m: int, k: int, parts: int = 3) -> tuple[Tensor, Tensor, int]:
    """(x, (XB, XT, XK, T)) -> q int8 [parts, m, ldq] (zero padded), qs FP32 [parts, m], ldq = round_up(k, 16).

    The reference's b1_quantize contract (kk/binary/layer.py:154-165); its first P parts equal the P-part quantizer."""
    return lowbit.quantize(x, rows, m, k, parts)


def m1_quantize(xx: Tensor, norm=None, input_activation: str = "") -> tuple[Tensor, Tensor]:
    """The three-part quantizer with LayerNorm / input SiLU fused, on [B, T, K] (kk/binary/layer.py:168-179).
    Returns q int8 [3, M, K'] (K' = round_up(K, 16)) and qs FP32 [3, M]."""
    b, t, k = xx.shape
    q, qs, _ = lowbit.quantize(xx, (xx.stride(0), xx.stride(1), xx.stride(2), t), b * t, k, 3, norm=norm,
                               input_activation=input_activation)
    return q, qs


def dot(layer: Int8MmaLayer, q: Tensor, qs: Tensor, ldq: int, m: int, y: Tensor | None, *, silu: bool = False,
        config=None, order: int = 0, acc_out: Tensor | None = None) -> None:
    """The launch (kk/binary/layer.py:182-209). `order` selects the epilogue's first FP32 contraction for P >= 2."""
    n, k = layer.out_features, layer.in_features
    if q.dim() != 3 or q.shape[2] != ldq or ldq % 16 or q.stride(1) != ldq or q.stride(2) != 1 or q.data_ptr() % 16:
        raise ValueError("fast path needs 16-byte aligned rows of q")
    if order not in (0, 1):
        raise ValueError("order must be 0 or 1")
    layer.launches.dot(q, qs, m, y, acc_out, silu=silu, order=order, config=config)
