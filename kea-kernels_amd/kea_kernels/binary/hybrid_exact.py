"""Exact deferred split-K for the 1-bit layers (drop-in for the slice half of kk/binary/hybrid_exact.py).

The reference's deferred path cuts K across a thread-block cluster, writes each slice's three INT32 part sums packed
into 21-bit lanes of an int64 word ([C, 2, M, N] int32 word planes, kk/binary/kernels_exact.py:1-12), and finishes
them in integers inside the next row epilogue (kk/binary/row_exact.py:69-96), so the projection value is bitwise the
unsplit result. Here every slice keeps its P exact int32 sums in their own plane, slices int32 [C, P, M, N]: no
packing and no K limit from 21-bit lanes (|acc| <= 127 K fits int32 for any K this library accepts).

  dot_slices(layer, q, qs, ldq, m, slices, config, order)   one launch: the K-slice sums (no scale is read)
  finish_slices(deferred | slices, ...)                     one launch: sum in slice order + the unsplit epilogue
  choose_exact_deferred(m, n, k)                            the slice count worth deferring for this shape, or None

ExactDeferredProjection carries the slices, scales and output shape to whoever finishes them; like the reference's,
its FP32 `partial` view raises, so integer slices can never be consumed as FP32 partials.
"""
from __future__ import annotations

import torch
from torch import Tensor

from kea_kernels import _hip, lowbit
from kea_kernels.binary.kernels import GemmConfig


def choose_exact_deferred(m: int, n: int, k: int, parts: int = 3, wbits: int = 1) -> GemmConfig | None:
    """A config with split > 1 when the library's chooser splits K for (M, N, K), else None (the unsplit in-kernel
    epilogue is then the faster exact path). A pure function of the shape, as the reference's tuned table
    (kk/binary/hybrid_exact.py:41-50)."""
    if m < 1:
        return None
    L = _hip.lib()
    tile = L.kea_lowbit_gemm_tile(wbits, parts, m, n, k)
    split = L.kea_lowbit_gemm_split(wbits, parts, m, n, k, 0, 0)
    if tile < 1 or split < 1:
        raise ValueError(f"no configuration for m={m} n={n} k={k}: {_hip.last_error()}")
    if split == 1 or k % 16:
        return None
    return GemmConfig(tile, split)


def dot_slices(layer, q: Tensor, qs: Tensor, ldq: int, m: int, slices: Tensor, config: GemmConfig | None = None,
               order: int = 0) -> None:
    """slices int32 [C, P, m, N] <- exact K-slice sums of the layer's GEMM (kk/binary/hybrid_exact.py:53-72).

    `qs` and `order` are accepted for the reference's signature; they are applied by finish_slices."""
    del qs, order
    n, k = layer.out_features, layer.in_features
    if q.dim() != 3 or q.shape[2] != ldq or ldq % 16 or q.stride(1) != ldq or q.stride(2) != 1 or q.data_ptr() % 16:
        raise ValueError("fast path needs q [P, M, ldq] with 16-byte aligned rows")
    if config is not None and int(getattr(config, "split", slices.shape[0]) or slices.shape[0]) != slices.shape[0]:
        raise ValueError(f"slices hold {slices.shape[0]} slices, config asks for {config.split}")
    lowbit.gemm_slices(layer.WBITS, q, layer.words, n, k, slices, m=m, config=config)


class ExactDeferredProjection:
    """Integer K-slices of one projection waiting for their epilogue: slices int32 [C, P, M, N], the layer's scale
    and bias, the part scales xs [P, M], the epilogue order and the [B, T, N] output shape."""

    def __init__(self, slices: Tensor, scale: Tensor, bias: Tensor | None, split: int, shape: tuple, xs: Tensor,
                 order: int = 0):
        self.slices, self.scale, self.bias, self.split, self.shape, self.xs, self.order = \
            slices, scale, bias, split, shape, xs, order

    @property
    def partial(self):
        raise RuntimeError("ExactDeferredProjection holds integer slices, not FP32 partials: finish it with "
                           "kea_kernels.binary.hybrid_exact.finish_slices")

    def finish(self, *, silu: bool = False, out_dtype: torch.dtype = torch.float32) -> Tensor:
        y = torch.empty(self.shape, device=self.slices.device, dtype=out_dtype)
        finish_slices(self, y.view(-1, self.shape[-1]), silu=silu)
        return y

    def __repr__(self) -> str:
        return f"ExactDeferredProjection(split={self.split}, shape={self.shape}, order={self.order})"


def finish_slices(deferred: ExactDeferredProjection, y: Tensor | None = None, acc_out: Tensor | None = None, *,
                  silu: bool = False) -> None:
    """y [M, N] (f32 / f16 / bf16 rows) and/or acc_out int32 [P, M, N] from the slices: bitwise the unsplit GEMM."""
    lowbit.slices_finish(deferred.slices, deferred.xs, deferred.scale, deferred.bias, y, acc_out, silu=silu,
                         order=deferred.order)


def project_deferred(layer, x: Tensor, *, components: int = 3, norm=None, input_activation: str = "",
                     config: GemmConfig | None = None) -> ExactDeferredProjection | Tensor:
    """Quantize x [B, T, K] and run the layer: an ExactDeferredProjection when the shape is worth splitting (or
    `config` asks for split > 1), else the finished FP32 [B, T, N] result of the unsplit GEMM."""
    xx = x.unsqueeze(0) if x.dim() == 2 else x
    b, t, k = xx.shape
    m, n = b * t, layer.out_features
    q, qs, ldq = lowbit.quantize(xx, (xx.stride(0), xx.stride(1), xx.stride(2), t), m, k, components, norm=norm,
                                 input_activation=input_activation)
    cfg = config if config is not None else choose_exact_deferred(m, n, k, components, layer.WBITS)
    if cfg is None or m == 0 or cfg.split in (0, 1):
        y = torch.empty(b, t, n, device=x.device, dtype=torch.float32)
        if m:
            lowbit.gemm(layer.WBITS, q, qs, layer.words, n, k, layer.scale, layer.bias, y.view(m, n), None, m=m)
        return y
    slices = torch.empty(cfg.split, components, m, n, device=x.device, dtype=torch.int32)
    dot_slices(layer, q, qs, ldq, m, slices, cfg)
    return ExactDeferredProjection(slices, layer.scale, layer.bias, cfg.split, (b, t, n), qs)
