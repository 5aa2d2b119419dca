"""GPU parity of the row-quantizing GEMM (kea_lowbit_gemm_rows) against the two-launch path and the oracle.

The bar is bitwise: the codes and scales quantized inside the GEMM are those of kea_quantize / kea_norm_quantize /
kea_attention_merge_quantize, so y (and NORM2's stored x_out) must equal the quantizer-then-GEMM result bit for bit,
for every mode, part count, tile, output dtype and epilogue. One case per mode is also checked against the oracle
directly (its quantizer, GEMM and epilogue on the CPU).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from kea_kernels import encoder as E
from kea_kernels import lowbit
from kea_kernels.binary import kernels
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"

# wave-split tile ids whose blocks are 16 rows (kea_config_name: 13 16x128 k/4, 15 16x64 k/4, 16 16x128 k/8,
# 18 16x32 k/4, 20 16x64 k/8)
TILES_K1024 = (13, 15, 18)


class Weights:
    """Seeded n x k weights (1-bit signs or ternary) with f32 scales, on the CPU and in the native layout."""

    def __init__(self, wbits: int, n: int, k: int, seed: int, *, bias: bool = False, glu: bool = False):
        g = torch.Generator().manual_seed(seed)
        self.wbits, self.n, self.k = wbits, n, k
        if wbits == 1:
            signs = torch.where(torch.rand(n, k, generator=g) < 0.5, -1, 1).to(torch.int8).numpy()
            self.codes = O.pack_signs(signs)
        else:
            self.codes = O.pack_ternary(torch.randint(-1, 2, (n, k), generator=g, dtype=torch.int8).numpy())
        self.alpha = (torch.rand(n, generator=g) + 0.5) / math.sqrt(k)
        self.bias = torch.randn(n, generator=g) * 0.1 if bias else None
        self.words = kernels.relayout_codes(torch.from_numpy(self.codes), k, wbits).to(DEV)
        self.dalpha = self.alpha.to(DEV)
        self.dbias = None if self.bias is None else self.bias.to(DEV)

    def gemm(self, q, qs, y, m, **kw):
        lowbit.gemm(self.wbits, q, qs, self.words, self.n, self.k, self.dalpha, self.dbias, y, None, m=m, **kw)

    def rows(self, x, y, m, **kw):
        lowbit.gemm_rows(self.wbits, x, self.words, self.n, self.k, self.dalpha, self.dbias, y, m=m, **kw)


def _rows(m: int, k: int, seed: int, *, ld: int | None = None) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, ld or k, generator=g) * (1.0 + torch.rand(m, 1, generator=g) * 3)
    return x.to(DEV)


def _norm(k: int, seed: int) -> torch.nn.LayerNorm:
    g = torch.Generator().manual_seed(seed)
    ln = torch.nn.LayerNorm(k)
    with torch.no_grad():
        ln.weight.copy_(torch.rand(k, generator=g) + 0.5)
        ln.bias.copy_(torch.randn(k, generator=g) * 0.1)
    return ln.to(DEV)


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    return (t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.int16)).numpy()


def _nan(m: int, n: int, dtype=torch.float32) -> torch.Tensor:
    return torch.full((m, n), float("nan"), device=DEV, dtype=dtype)


@pytest.mark.parametrize("wbits,parts,m,n,k", [(1, 1, 125, 4096, 1024), (1, 1, 125, 1024, 4096), (2, 1, 17, 1024, 2048),
                                               (1, 2, 1, 3072, 1024), (2, 3, 300, 1024, 1024), (1, 2, 33, 96, 2048),
                                               (1, 1, 1000, 1024, 4096), (2, 2, 125, 2048, 1024)])
@torch.inference_mode()
def test_plain_rows_bitwise_two_launch_path(wbits, parts, m, n, k):
    w = Weights(wbits, n, k, seed=m + n + k, bias=True)
    x = _rows(m, k, seed=m + k)
    q, qs, _ = lowbit.quantize(x, (0, k, 1, m), m, k, parts)
    want, got = _nan(m, n), _nan(m, n)
    w.gemm(q, qs, want, m)
    w.rows(x, got, m, parts=parts)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("tile", TILES_K1024)
@pytest.mark.parametrize("parts", [1, 2, 3])
@torch.inference_mode()
def test_norm_rows_every_tile_and_part_count(tile, parts):
    m, n, k = 125, 1024, 1024
    w = Weights(1, n, k, seed=tile + parts)
    x, ln = _rows(m, k, seed=7), _norm(k, seed=8)
    q, qs, _ = lowbit.quantize(x, (0, k, 1, m), m, k, parts, norm=ln)
    want, got = _nan(m, n), _nan(m, n)
    w.gemm(q, qs, want, m)
    w.rows(x, got, m, parts=parts, norm=ln, config=tile)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("m", [1, 16, 125, 250])
@pytest.mark.parametrize("parts", [1, 3])
@torch.inference_mode()
def test_norm2_rows_store_the_first_layernorm_bitwise(m, parts):
    n, k = 4096, 1024
    w = Weights(1, n, k, seed=m, bias=False)
    x, ln0, ln1 = _rows(m, k, seed=m + 1), _norm(k, seed=2), _norm(k, seed=3)
    out_want, q, qs = E.norm_quantize(x.view(1, m, k), ln0, ln1, parts)
    want, got = _nan(m, n), _nan(m, n)
    w.gemm(q, qs, want, m, silu=True)
    x_out = _nan(m, k)
    w.rows(x, got, m, parts=parts, norm=ln0, next_norm=ln1, x_out=x_out, silu=True)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(x_out), _bits(out_want.view(m, k)))
    assert np.array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("batch", [1, 2])
@torch.inference_mode()
def test_merge_rows_equal_merge_quantize_then_gemm(batch):
    t, heads, d, n = 125, 8, 1024, 1024
    m = batch * t
    g = torch.Generator().manual_seed(batch)
    qkv = (torch.randn(batch, t, 3 * d, generator=g)).to(DEV)
    pos = (torch.randn(2 * t - 1, d, generator=g) * 0.5).to(DEV)
    bu, bv = (torch.randn(heads, d // heads, generator=g) * 0.02).to(DEV), (torch.randn(heads, d // heads, generator=g) * 0.02).to(DEV)
    ws = E.attention_workspace(batch, t, heads, DEV)
    assert ws is not None, "the key split applies at this shape"
    E.relpos_attention(qkv, pos, bu, bv, heads, workspace=ws, merged=False)
    q, qs = E.attention_merge_quantize(ws, batch, t, heads, 1)
    w = Weights(1, n, d, seed=11)
    res = _rows(m, n, seed=12)
    want, got = res.clone(), res.clone()
    w.gemm(q, qs, want, m, residual=want)
    w.rows(ws, got, m, merge_heads=heads, residual=got)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16, torch.bfloat16])
@torch.inference_mode()
def test_epilogue_variants(out_dtype):
    m, n, k = 77, 2048, 1024
    w = Weights(1, n, k, seed=5, bias=True)
    x, ln = _rows(m, k, seed=6), _norm(k, seed=9)
    q, qs, _ = lowbit.quantize(x, (0, k, 1, m), m, k, 2, norm=ln)
    for kw in ({"silu": True}, {"glu": True}, {"order": 1}):
        ny = n // 2 if kw.get("glu") else n
        want, got = _nan(m, ny, out_dtype), _nan(m, ny, out_dtype)
        w.gemm(q, qs, want, m, **kw)
        w.rows(x, got, m, parts=2, norm=ln, **kw)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(got), _bits(want)), kw


@torch.inference_mode()
def test_residual_in_place_and_strided_rows():
    m, n, k = 130, 1024, 4096
    w = Weights(1, n, k, seed=21)
    x = _rows(m, k, seed=22, ld=k + 64)
    r = _rows(m, n, seed=23)
    q, qs, _ = lowbit.quantize(x, (0, k + 64, 1, m), m, k, 1)
    want, got = r.clone(), r.clone()
    w.gemm(q, qs, want, m, residual=want, residual_factor=0.5)
    w.rows(x, got, m, residual=got, residual_factor=0.5)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("mode", ["plain", "norm"])
@torch.inference_mode()
def test_against_the_oracle(mode):
    m, n, k, parts = 19, 256, 1024, 2
    w = Weights(1, n, k, seed=31, bias=True)
    x, ln = _rows(m, k, seed=32), _norm(k, seed=33)
    norm = (ln.weight.detach().cpu().numpy(), ln.bias.detach().cpu().numpy()) if mode == "norm" else None
    q, qs = O.quantize(x.cpu().numpy(), parts, norm=norm, eps=ln.eps)
    want = O.epilogue(O.b1_gemm(q, w.codes, k), qs, w.alpha.numpy(), w.bias.numpy())
    got = _nan(m, n)
    w.rows(x, got, m, parts=parts, norm=ln if mode == "norm" else None)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))


@torch.inference_mode()
def test_refusals():
    w = Weights(1, 1024, 1024, seed=41)
    x = _rows(32, 1024, seed=42)
    with pytest.raises(ValueError, match="must not overlap"):
        w.rows(x, x, 32)                                        # y would overwrite rows other workgroups still read
    w4 = Weights(1, 1024, 4096, seed=43)
    with pytest.raises(ValueError, match="no row-quantizing kernel"):
        w4.rows(_rows(8, 4096, seed=44), _nan(8, 1024), 8, parts=3)  # registers do not fit three parts at k = 4096
    w5 = Weights(1, 256, 512, seed=45)
    with pytest.raises(ValueError, match="k must be 1024"):
        w5.rows(_rows(8, 512, seed=46), _nan(8, 256), 8)
    ln = _norm(1024, seed=47)
    with pytest.raises(ValueError, match="x_out must not overlap"):
        w.rows(x, _nan(32, 1024), 32, norm=ln, next_norm=ln, x_out=x)
