"""The exact row epilogue: finish deferred integer K-slices straight into the next layer's input (row F2).

Drop-in for kk/binary/row_exact.py's `finish_residual_exact` (:125-156) and the row_fusion protocol it serves
(kk/ternary/row_fusion.py:90-111): one launch per residual block computes, per row,

    value = the unsplit GEMM epilogue of the slices (bitwise the SPLIT == 1 result)
    x     = residual + value * factor ; x = out_norm(x) if given ; y = x
    q, qs = the 3-part int8 quantization of norm(y) for the next projection (when `norm` is given)

and leaves (q, qs) in provider.prequantized under the reference's key (y.data_ptr(), m, n, id(norm)), where the next
provider call with that LayerNorm picks it up instead of quantizing again. The kernel is kea_row_epilogue
(include/kea_lowbit.h): its LayerNorm sums and quantization are the library quantizer's, so q / qs are bitwise
what kea_quantize returns for y's rows.
"""
from __future__ import annotations

import torch
from torch import Tensor

from kea_kernels import lowbit
from kea_kernels.binary.hybrid_exact import ExactDeferredProjection


def finish_residual_exact(provider, value: ExactDeferredProjection, residual: Tensor, factor: float, norm=None,
                          out_norm=None, *, components: int = 3) -> Tensor:
    """y [B, T, N] = out_norm(residual + factor * value); with `norm`, the next input's int8 parts are cached in
    provider.prequantized (kk/binary/row_exact.py:125-156)."""
    if not isinstance(value, ExactDeferredProjection):
        raise TypeError("finish_residual_exact needs an ExactDeferredProjection")
    if not residual.is_contiguous() or tuple(residual.shape) != tuple(value.shape):
        raise ValueError("expected contiguous B,T,C residual")
    n = residual.shape[-1]
    m = residual.numel() // n
    if value.slices.dtype != torch.int32 or value.slices.dim() != 4 or tuple(value.slices.shape[2:]) != (m, n) \
            or not value.slices.is_contiguous():
        raise ValueError("expected contiguous int32 slices [split, P, M, N]")
    y = torch.empty_like(residual)
    out = lowbit.row_epilogue(value.slices, value.xs, value.scale, value.bias, y.view(m, n),
                              residual=residual.view(m, n), factor=factor, out_norm=out_norm, norm=norm,
                              quantize_parts=components if norm is not None else 0, order=value.order)
    if norm is not None:
        key = (y.data_ptr(), m, n, id(norm))
        cache = getattr(provider, "prequantized", None)
        if cache is None:
            raise TypeError("the provider keeps no prequantized cache")
        if key in cache:
            raise RuntimeError("unconsumed fused activation")
        cache[key] = out
    return y
