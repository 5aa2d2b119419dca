"""The Kea-T projection provider (drop-in for ExpandedProjection, kk/ternary/encoder4.py:77-149).

The reference's x2 / x3 provider expands every layer's 2-bit codes once into an int8 [N, K] copy (about 604 MB per
model, kk/ternary/encoder4.py:104-110) so its Triton kernel can read dense int8 weights. On gfx950 the GEMM expands
2-bit codes to int8 inside the registers that feed the MFMA, so this provider keeps the codes 2-bit resident and
allocates no expanded copy (`bytes` is 0); otherwise it has the reference's call signature and semantics
(kk/binary/provider.py:3-15).
"""
from __future__ import annotations

from kea_kernels.ternary.fused_kernels import int8_matmul, integer_configuration


def expanded_configuration(m: int, n: int, k: int, parts: int = 3):
    """The library's tile / split choice (the reference's RTX 5090 table, kk/ternary/encoder4.py:9-20, re-measured as a
    pure function of the shape on MI355X)."""
    return integer_configuration(m, n, k, parts)


class ExpandedProjection:
    """Provider for the ternary modules: quantize + 2-bit x int8 GEMM, no expanded weight copy."""

    def __init__(self, backend: str = "triton", config=None):
        self.backend, self.config = backend, config
        self.weights: dict = {}

    @property
    def bytes(self) -> int:
        return 0

    def __call__(self, x, mod, conv=False, components=3, activation="", norm=None, config=None, input_activation=""):
        return int8_matmul(x, mod, conv, components, activation, norm, self.config or config, input_activation)
