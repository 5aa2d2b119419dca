"""Tile choice for the gfx950 low-bit GEMM (the role of kk/binary/configs.py).

As in the reference (kk/binary/configs.py:1-7), the choice is a pure function of the shape, with no inference-time
autotuning. The table itself lives in the library (kea_lowbit_gemm_tile / kea_lowbit_gemm_split), so the Python
layer, the C ABI and the benchmarks all agree on it. Results never depend on it.
"""
from __future__ import annotations

from kea_kernels import _hip
from kea_kernels.binary.kernels import GemmConfig

CUS = 256  # MI355X compute units (8 XCDs x 32)


def choose(m: int, n: int, k: int, parts: int = 1, wbits: int = 1) -> GemmConfig:
    tile = _hip.lib().kea_lowbit_gemm_tile(wbits, parts, max(m, 1), n, k)
    split = _hip.lib().kea_lowbit_gemm_split(wbits, parts, max(m, 1), n, k, 0, 0)
    if tile < 1 or split < 1:
        raise ValueError(f"no configuration for m={m} n={n} k={k} parts={parts} wbits={wbits}: {_hip.last_error()}")
    return GemmConfig(tile, split)
