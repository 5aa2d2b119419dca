"""1-bit weight codes: the export layout, its validation and dequantization (drop-in for kk/binary/bits.py).

Export layout (parakeet-binary-v1, kk/binary/bits.py:3-5): uint8 [N, ceil(K/8)]; weight k of a row is bit k % 8 of
byte k // 8 (least significant bit first); a set bit is +1, a clear bit -1; bits past K are 0. One FP32 scale per
row, so W = alpha * sign. Runs on any device (CPU included); validation syncs when the tensors live on a GPU.
"""
from __future__ import annotations

import math

import torch
from torch import Tensor

_BIT = 1 << torch.arange(8, dtype=torch.int32)  # weight of bit j inside a byte


def packed_row_bytes(in_features: int) -> int:
    return math.ceil(in_features / 8)


def validate_weights(codes: Tensor, scale: Tensor, bias: Tensor | None, in_features: int) -> tuple[int, int]:
    """(N, K) after the checks Int8MmaLayer.prepare needs; ValueError otherwise (kk/binary/bits.py:21-38)."""
    if isinstance(in_features, bool) or not isinstance(in_features, int) or in_features < 1:
        raise ValueError(f"in_features must be a positive int, got {in_features!r}")
    width = packed_row_bytes(in_features)
    if codes.dtype != torch.uint8 or codes.dim() != 2 or codes.shape[0] < 1 or codes.shape[1] != width:
        raise ValueError(f"codes must be uint8 [N, {width}], got {codes.dtype} {tuple(codes.shape)}")
    n = codes.shape[0]
    spare = 8 * width - in_features
    if spare and bool((codes[:, -1].to(torch.int32) >> (8 - spare)).ne(0).any()):
        raise ValueError("invalid packed codes: nonzero tail padding")
    if scale.dtype != torch.float32 or tuple(scale.shape) != (n,) or not bool(torch.isfinite(scale).all()):
        raise ValueError("scale must be finite FP32 [N]")
    if bias is not None and (bias.dtype != torch.float32 or tuple(bias.shape) != (n,)
                             or not bool(torch.isfinite(bias).all())):
        raise ValueError("bias must be None or finite FP32 [N]")
    if scale.device != codes.device or (bias is not None and bias.device != codes.device):
        raise ValueError("codes, scale and bias must be on one device")
    return n, in_features


def unpack_bits(codes: Tensor, in_features: int) -> Tensor:
    """uint8 [N, ceil(K/8)] -> uint8 {0, 1} [N, K] (1 = +1); nonzero tail bits raise ValueError."""
    width = packed_row_bytes(in_features)
    if codes.dtype != torch.uint8 or codes.dim() != 2 or codes.shape[1] != width:
        raise ValueError(f"expected uint8 [N, {width}], got {codes.dtype} {tuple(codes.shape)}")
    expanded = (codes.to(torch.int32).unsqueeze(-1) & _BIT.to(codes.device)).ne(0)
    flat = expanded.reshape(codes.shape[0], 8 * width)
    if bool(flat[:, in_features:].any()):
        raise ValueError("invalid packed codes: nonzero tail padding")
    return flat[:, :in_features].to(torch.uint8).contiguous()


def unpack_signs(codes: Tensor, in_features: int) -> Tensor:
    """uint8 [N, ceil(K/8)] -> int8 {-1, +1} [N, K]."""
    return unpack_bits(codes, in_features).to(torch.int8).mul_(2).sub_(1)


def pack_signs(signs: Tensor) -> Tensor:
    """int8 {-1, +1} [N, K] -> uint8 codes [N, ceil(K/8)]."""
    if signs.dtype != torch.int8 or signs.dim() != 2 or bool(((signs != 1) & (signs != -1)).any()):
        raise ValueError("expected 2-D int8 signs in {-1, +1}")
    rows, k = signs.shape
    width = packed_row_bytes(k)
    positive = torch.zeros(rows, 8 * width, dtype=torch.int32, device=signs.device)
    positive[:, :k] = signs.eq(1).to(torch.int32)
    weighted = positive.view(rows, width, 8) * _BIT.to(signs.device)
    return weighted.sum(dim=2).to(torch.uint8)


def dense_weight(codes: Tensor, scale: Tensor, in_features: int, dtype: torch.dtype = torch.float64) -> Tensor:
    """Dequantized [N, K] = sign * scale[:, None] (exact in FP32 and FP64), on codes.device."""
    signs = unpack_signs(codes, in_features).to(dtype)
    return signs * scale.to(device=codes.device, dtype=dtype).unsqueeze(1)


def resident_bytes(*tensors: Tensor | None) -> int:
    """Bytes of the distinct GPU storages behind `tensors` (a view counts its whole storage once)."""
    storages = {(s.data_ptr(), s.nbytes()) for s in (t.untyped_storage() for t in tensors if t is not None and t.is_cuda)}
    largest: dict[int, int] = {}
    for ptr, nbytes in storages:
        largest[ptr] = max(nbytes, largest.get(ptr, 0))
    return sum(largest.values())
