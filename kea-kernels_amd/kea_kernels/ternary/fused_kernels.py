"""The ternary int8 projection (drop-in for the int8 path of kk/ternary/fused_kernels.py).

`int8_matmul(x, mod, conv, components, activation, norm, config, input_activation)` keeps the reference's provider
signature and semantics (kk/ternary/fused_kernels.py:139-160): quantize x into `components` residual int8 parts (with
LayerNorm / input SiLU fused), multiply by the module's 2-bit codes, scale by alpha, add bias, optional SiLU, FP32
[B, T, N] (or a [B, N, T] view for conv). The reference decodes the codes in a Triton kernel and reduces split-K
partials in FP32 (`_int8_dot` + `_finish`, kk/ternary/fused_kernels.py:53-120, kk/ternary/kernels.py:122-137); here
both steps are the library's int8-MFMA GEMM, whose split-K reduction is exact int32, so every split gives the
unsplit result bit for bit.
"""
from __future__ import annotations

import torch

from kea_kernels import lowbit
from kea_kernels.binary import configs
from kea_kernels.ternary.runtime import native_words


def integer_configuration(m: int, n: int, k: int, parts: int = 3):
    """The library's tile / split choice for this shape (a pure function of the shape, as the reference's table;
    kk/ternary/fused_kernels.py:123-136)."""
    return configs.choose(m, n, k, parts=parts, wbits=2)


def _quantize(xx: torch.Tensor, parts: int, norm=None, input_activation: str = ""):
    """The residual quantizer on [B, T, K] (any strides); returns q int8 [parts, M, ldq], qs FP32 [parts, M], ldq."""
    b, t, k = xx.shape
    return lowbit.quantize(xx, (xx.stride(0), xx.stride(1), xx.stride(2), t), b * t, k, parts, norm=norm,
                           input_activation=input_activation)


def int8_matmul(x, mod, conv=False, components=1, activation="", norm=None, config=None, input_activation=""):
    if activation not in ("", "silu") or input_activation not in ("", "silu"):
        raise ValueError(f"unsupported activation {activation!r} / {input_activation!r}")
    if components not in (1, 2, 3):
        raise ValueError(f"components must be 1, 2 or 3, got {components!r}")
    xx = x.transpose(1, 2) if conv else x
    if xx.ndim == 2:
        xx = xx.unsqueeze(0)
    if xx.ndim != 3 or xx.shape[-1] != mod.in_features:
        raise ValueError(f"expected [B, T, {mod.in_features}] input, got {tuple(xx.shape)}")
    if xx.dtype not in (torch.float32, torch.float16):
        raise ValueError(f"expected FP32 input, got {xx.dtype}")
    b, t, k = xx.shape
    m, n = b * t, mod.out_features
    y = torch.empty((b, t, n), dtype=torch.float32, device=x.device)
    if m:
        launches = _launches(mod)
        rows = (xx.stride(0), xx.stride(1), xx.stride(2), t)
        if not launches.project(xx, rows, m, components, y.view(m, n), silu=activation == "silu", norm=norm,
                                input_activation=input_activation, config=config):
            q, qs, _ = _quantize(xx, components, norm, input_activation)
            lowbit.gemm(2, q, qs, native_words(mod), n, k, mod.scale, mod.bias, y.view(m, n), None,
                        silu=activation == "silu", config=config)
    return y.transpose(1, 2) if conv else y.reshape(*x.shape[:-1], n)


def _launches(mod) -> lowbit.Launches:
    """The module's launches resolved once per call layout (lowbit.Launches), kept on the module and rebuilt if its
    codes, scale or bias change."""
    words = native_words(mod)
    cache = mod.__dict__.get("_kea_launches")
    if cache is None or cache.words is not words or cache.wscale is not mod.scale or cache.bias is not mod.bias:
        cache = lowbit.Launches(2, words, mod.out_features, mod.in_features, mod.scale, mod.bias)
        mod.__dict__["_kea_launches"] = cache
    return cache
