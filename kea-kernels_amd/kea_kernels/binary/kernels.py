"""gfx950 native weight layout and tile configurations of the low-bit GEMM (the role of kk/binary/kernels.py).

The reference rearranges the 1-bit codes once into the B-fragment layout of SM120's mma.m16n8k32
(kk/binary/kernels.py:18-23, :730-752). This build keeps its own wavefront-native layout (include/kea_lowbit.h):
per 16-row n-tile and per lane of a 64-wide wavefront, one 32-bit word per 128 weights (1-bit, inverted signs at
bit 8i + 4h + d) or per 64 weights (2-bit codes at bits 8i + 2d), stored so that a lane's four consecutive words
arrive with one 128-bit load. Built on the host by the library (kea_b1_relayout_host / kea_t2_relayout_host).

GemmConfig is the counterpart of DotConfig: a tile id of the library's table plus the split-K factor. Every tile and
every split produces bitwise the same outputs (exact int32 accumulation and reduction); they only change speed.
"""
from __future__ import annotations

import ctypes
import dataclasses

import numpy as np
import torch

from kea_kernels import _hip


def native_words(n: int, k: int, wbits: int = 1) -> int:
    """Number of uint32 words of the native layout of an N x K weight matrix."""
    fn = _hip.lib().kea_b1_native_words if wbits == 1 else _hip.lib().kea_t2_native_words
    count = fn(n, k)
    if count <= 0:
        raise ValueError(f"bad weight shape {n} x {k}")
    return count


def relayout_codes(codes: torch.Tensor, k: int, wbits: int = 1) -> torch.Tensor:
    """Export codes uint8 [N, ceil(K*wbits/8)] (any device) -> native words int32 (flat, on the CPU).

    ValueError on invalid codes (nonzero tail bits, the ternary 11 pattern)."""
    if codes.dtype != torch.uint8 or codes.dim() != 2:
        raise ValueError("codes must be a 2-D uint8 tensor")
    n = codes.shape[0]
    host = np.ascontiguousarray(codes.detach().cpu().numpy())
    words = np.zeros(native_words(n, k, wbits), np.uint32)
    fn = _hip.lib().kea_b1_relayout_host if wbits == 1 else _hip.lib().kea_t2_relayout_host
    _hip.check(fn(host.ctypes.data_as(ctypes.c_void_p), n, k, words.ctypes.data_as(ctypes.c_void_p)), "relayout")
    return torch.from_numpy(words.view(np.int32))


def unlayout_codes(words: torch.Tensor, n: int, k: int, wbits: int = 1) -> torch.Tensor:
    """Inverse of relayout_codes: native words -> export codes uint8 (on the CPU)."""
    host = np.ascontiguousarray(words.detach().cpu().numpy().view(np.uint32))
    if host.size != native_words(n, k, wbits):
        raise ValueError("word count does not match the shape")
    width = -(-k * wbits // 8)
    codes = np.zeros((n, width), np.uint8)
    fn = _hip.lib().kea_b1_unlayout_host if wbits == 1 else _hip.lib().kea_t2_unlayout_host
    _hip.check(fn(host.ctypes.data_as(ctypes.c_void_p), n, k, codes.ctypes.data_as(ctypes.c_void_p)), "unlayout")
    return torch.from_numpy(codes)


def relayout(bits: torch.Tensor) -> torch.Tensor:
    """uint8 {0, 1} [N, K] (1 = +1) -> native words (the counterpart of the reference's relayout)."""
    from kea_kernels.binary import bits as api
    signs = bits.to(torch.int8).mul(2).sub(1)
    return relayout_codes(api.pack_signs(signs.cpu()), bits.shape[1], 1)


def unlayout(words: torch.Tensor, n: int, k: int) -> torch.Tensor:
    """Inverse of relayout: native words -> uint8 {0, 1} [N, K]."""
    from kea_kernels.binary import bits as api
    return api.unpack_bits(unlayout_codes(words, n, k, 1), k)


@dataclasses.dataclass(frozen=True)
class GemmConfig:
    """A tile of the library's table (1-based id) and a split-K factor (0 = the library's choice)."""
    tile: int
    split: int = 0

    def label(self) -> str:
        name = _hip.lib().kea_config_name(self.tile).decode()
        return f"t{self.tile}[{name}]" + (f"_s{self.split}" if self.split else "")

    def validate(self) -> None:
        count = _hip.lib().kea_config_count()
        if not (1 <= self.tile <= count) or self.split < 0:
            raise ValueError(f"invalid config {self} (tiles 1..{count}, split >= 0)")


def tile_count() -> int:
    return _hip.lib().kea_config_count()


def config_name(tile: int) -> str:
    """The library's name of tile id `tile` ("" for an unknown id)."""
    return _hip.lib().kea_config_name(tile).decode()
