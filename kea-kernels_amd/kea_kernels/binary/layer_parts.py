"""Int8MmaLayer with 1, 2 or 3 activation parts (drop-in for kk/binary/layer_parts.py).

`Int8MmaPartsLayer` is Int8MmaLayer (layer.py) with
  * project(x, *, conv, components, activation, norm, input_activation) honouring components in {1, 2, 3} (the
    provider's PartCount sets it on every call): the residual quantizer at P = components (fused LayerNorm / input
    SiLU), then the P-part GEMM;
  * dot(q, qs, ldq, m, y, ..., parts=None): the P-part GEMM, P = q.shape[0] unless given;
  * linear / conv at the class's fixed part count PARTS (the first PARTS parts of the three-part quantizer, which are
    bitwise the PARTS-part quantizer: its loop over parts is sequential, kk/binary/layer_parts.py:93-99).
The P-part epilogue combines the parts as the reference's comb<P> (kk/binary/kernels_parts.py:28-39):
    P = 1: acc0 * s0;  P = 2: fma(acc0, s0, acc1 * s1) (order 1: fma(acc1, s1, acc0 * s0));  P = 3: fma(acc2, s2, <P=2>)
then * alpha (+ bias) and optional SiLU. Unlike the reference there is no separate source transform per P: the kernel
is instantiated for P = 1, 2 and 3 ahead of time.
"""
from __future__ import annotations

import torch
from torch import Tensor

from kea_kernels import lowbit
from kea_kernels.binary.layer import Int8MmaLayer, _project, quantize

round_up = lowbit.round_up


def m1_quantize_parts(xx: Tensor, parts: int, norm=None, input_activation: str = "") -> tuple[Tensor, Tensor]:
    """The residual int8 quantizer at P = parts on [B, T, K] with LayerNorm / input SiLU fused.
    Returns q int8 [parts, M, K'] (K' = round_up(K, 16), zero padded) and qs FP32 [parts, M]."""
    b, t, k = xx.shape
    q, qs, _ = lowbit.quantize(xx, (xx.stride(0), xx.stride(1), xx.stride(2), t), b * t, k, parts, norm=norm,
                               input_activation=input_activation)
    return q, qs


class Int8MmaPartsLayer(Int8MmaLayer):
    PARTS = 3

    def dot(self, q: Tensor, qs: Tensor, ldq: int, m: int, y: Tensor | None, *, silu: bool = False, config=None,
            order: int = 0, parts: int | None = None, acc_out: Tensor | None = None) -> None:
        parts = q.shape[0] if parts is None else parts
        if parts not in (1, 2, 3) or q.shape[0] != parts or qs.shape[0] != parts:
            raise ValueError(f"q / qs must hold {parts} parts")
        dot_parts(self, q, qs, ldq, m, y, silu=silu, config=config, order=order, parts=parts, acc_out=acc_out)

    def project(self, x: Tensor, *, conv: bool = False, components: int | None = None, activation: str = "",
                norm=None, input_activation: str = "") -> Tensor:
        parts = self.PARTS if components is None else components
        if parts not in (1, 2, 3):
            raise ValueError(f"components must be 1, 2 or 3, got {components!r}")
        return _project(self, x, conv, parts, activation, norm, input_activation)

    def _run(self, x: Tensor, rows: tuple, m: int, y: Tensor):
        """linear / conv: the first PARTS residual parts (bitwise the PARTS-part quantizer); returns the cached
        launch entry used, or None."""
        e = self.launches.project(x, rows, m, self.PARTS, y)
        if not e:
            q, qs, ldq = quantize(x, rows, m, self.in_features, parts=self.PARTS)
            self.dot(q, qs, ldq, m, y, parts=self.PARTS)
            return None
        return e


def _aligned(q: Tensor, k: int) -> tuple[Tensor, int]:
    """q [P, M, K] -> rows padded with zeros to a multiple of 16 bytes (the GEMM's row alignment) if needed."""
    if k % 16 == 0 and q.data_ptr() % 16 == 0 and q.stride(1) == k:
        return q, k
    ldq = round_up(k, 16)
    padded = q.new_zeros(q.shape[0], q.shape[1], ldq)
    padded[:, :, :k] = q[:, :, :k]
    return padded, ldq


def dot_parts(layer: Int8MmaLayer, q: Tensor, qs: Tensor, ldq: int, m: int, y: Tensor | None, *, silu: bool = False,
              config=None, order: int = 0, parts: int = 3, acc_out: Tensor | None = None) -> None:
    """The P-part launch (kk/binary/layer_parts.py:112-130): y[:m] from q int8 [P, m, ldq] and qs [P, m]."""
    n, k = layer.out_features, layer.in_features
    if q.shape[0] != parts:
        raise ValueError(f"q must hold {parts} parts")
    if ldq % 16 or q.stride(1) != ldq or q.stride(2) != 1 or q.data_ptr() % 16:
        raise ValueError("fast path needs 16-byte aligned rows of q")
    if order not in (0, 1):
        raise ValueError("order must be 0 or 1")
    layer.launches.dot(q, qs, m, y, acc_out, silu=silu, order=order, config=config)


def variant(parts: int):
    """The layer class whose linear / conv run at `parts` activation parts."""
    return type(f"Int8MmaX{parts}Layer", (Int8MmaPartsLayer,), {"PARTS": parts})


LAYERS = {parts: variant(parts) for parts in (1, 2, 3)}
