"""GPU parity of the exact row epilogue (kea_row_epilogue) against the pinned oracle and the library's own paths.

The bar: y bitwise the oracle's epilogue value plus the residual (IEEE multiply, then add) for every slice count;
with a LayerNorm in front of the next projection, q / q_scales bitwise the oracle quantizer applied to y; an output
LayerNorm within FP32 rounding of an FP64 LayerNorm (its summation order is the library's own).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from kea_kernels import lowbit
from kea_kernels.binary import hybrid_exact, row_exact
from oracle import oracle as O
from test_gemm_gpu import DEV, Case

pytestmark = pytest.mark.gpu


def _slices(case: Case, split: int) -> torch.Tensor:
    s = torch.full((split, case.p, case.m, case.n), -5, device=DEV, dtype=torch.int32)
    lowbit.gemm_slices(case.wbits, case.dq, case.words, case.n, case.k, s)
    return s


def _layer_norm(n: int, seed: int) -> torch.nn.LayerNorm:
    g = torch.Generator().manual_seed(seed)
    ln = torch.nn.LayerNorm(n)
    with torch.no_grad():
        ln.weight.copy_(torch.rand(n, generator=g) + 0.5)
        ln.bias.copy_(torch.randn(n, generator=g) * 0.1)
    return ln


SHAPES = [(1, 3, 37, 1024, 4096, 4), (1, 1, 125, 1024, 1024, 1), (2, 3, 9, 96, 512, 2), (1, 1, 40, 2048, 1024, 2),
          (1, 2, 64, 4096, 1024, 2), (1, 3, 1, 516, 640, 1), (2, 1, 100, 1024, 4096, 8)]


@pytest.mark.parametrize("wbits,p,m,n,k,split", SHAPES)
@torch.inference_mode()
def test_residual_value_bitwise(wbits, p, m, n, k, split):
    case = Case(wbits, p, m, n, k, seed=m + n + split, bias=True, scale_dtype=torch.float32)
    res = torch.randn(m, n, generator=torch.Generator().manual_seed(k + m))
    y = torch.full((m, n), float("nan"), device=DEV)
    out = lowbit.row_epilogue(_slices(case, split), case.dqs, case.dalpha, case.dbias, y, residual=res.to(DEV),
                              factor=0.5)
    torch.cuda.synchronize()
    assert out is None
    want = (res.numpy() + case.oracle_y(case.oracle_acc()) * np.float32(0.5)).astype(np.float32)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("order", [0, 1])
@torch.inference_mode()
def test_value_without_residual_equals_unsplit_gemm(order):
    case = Case(1, 2, 50, 1024, 2048, seed=3, bias=False, scale_dtype=torch.float32)
    y = torch.empty(50, 1024, device=DEV)
    lowbit.row_epilogue(_slices(case, 4), case.dqs, case.dalpha, None, y, order=order)
    ref = torch.empty(50, 1024, device=DEV)
    lowbit.gemm(1, case.dq, case.dqs, case.words, 1024, 2048, case.dalpha, None, ref, None, order=order)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), ref.view(torch.int32))


@pytest.mark.parametrize("n,parts,out_norm", [(1024, 3, True), (1024, 1, False), (96, 3, True), (4096, 2, False),
                                              (516, 3, True)])
@torch.inference_mode()
def test_norms_and_next_quantization(n, parts, out_norm):
    m, k = 33, 1024
    case = Case(1, 3, m, n, k, seed=n + parts, bias=True, scale_dtype=torch.float32)
    res = torch.randn(m, n, generator=torch.Generator().manual_seed(n)) * 2
    ln0, ln1 = _layer_norm(n, 1), _layer_norm(n, 2)
    dres = res.to(DEV)
    y = dres  # in place, as the encoder runs it
    q, qs = lowbit.row_epilogue(_slices(case, 2), case.dqs, case.dalpha, case.dbias, y, residual=dres, factor=1.0,
                                out_norm=ln0 if out_norm else None, norm=ln1, quantize_parts=parts)
    torch.cuda.synchronize()
    x = (res.numpy() + case.oracle_y(case.oracle_acc())).astype(np.float32)
    got = y.cpu()
    if out_norm:
        ref = F.layer_norm(torch.from_numpy(x).double(), (n,), ln0.weight.double(), ln0.bias.double(), ln0.eps)
        assert float((got.double() - ref).abs().max()) < 2e-5
    else:
        assert np.array_equal(got.numpy().view(np.uint32), x.view(np.uint32))
    rq, rqs = O.quantize(got.numpy(), parts, ldq=q.shape[2], norm=(ln1.weight.detach().numpy(),
                                                                     ln1.bias.detach().numpy()), eps=ln1.eps)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(qs.cpu().numpy(), rqs)
    # and bitwise the library's own quantizer on y
    lq, lqs, _ = lowbit.quantize(y, (0, n, 1, m), m, n, parts, norm=ln1.to(DEV))
    assert torch.equal(lq, q) and torch.equal(lqs, qs)


@torch.inference_mode()
def test_plain_quantization_without_norm():
    case = Case(1, 1, 20, 1024, 1024, seed=8, scale_dtype=torch.float32)
    y = torch.empty(20, 1024, device=DEV)
    q, qs = lowbit.row_epilogue(_slices(case, 1), case.dqs, case.dalpha, None, y, quantize_parts=3)
    torch.cuda.synchronize()
    rq, rqs = O.quantize(y.cpu().numpy(), 3, ldq=q.shape[2])
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(qs.cpu().numpy(), rqs)


class _Provider:
    def __init__(self):
        self.prequantized = {}


@torch.inference_mode()
def test_finish_residual_exact_caches_the_next_input():
    b, t, n, k = 2, 19, 1024, 4096
    case = Case(1, 3, b * t, n, k, seed=11, bias=True, scale_dtype=torch.float32)
    deferred = hybrid_exact.ExactDeferredProjection(_slices(case, 4), case.dalpha, case.dbias, 4, (b, t, n), case.dqs)
    residual = torch.randn(b, t, n, generator=torch.Generator().manual_seed(12)).to(DEV)
    ln = _layer_norm(n, 3).to(DEV)
    prov = _Provider()
    y = row_exact.finish_residual_exact(prov, deferred, residual, 0.5, ln)
    torch.cuda.synchronize()
    assert y.shape == (b, t, n) and y.data_ptr() != residual.data_ptr()
    key = (y.data_ptr(), b * t, n, id(ln))
    q, qs = prov.prequantized[key]
    want = (residual.cpu().numpy().reshape(-1, n) + case.oracle_y(case.oracle_acc()) * np.float32(0.5))
    assert np.array_equal(y.cpu().numpy().reshape(-1, n).view(np.uint32), want.astype(np.float32).view(np.uint32))
    lq, lqs, _ = lowbit.quantize(y, (y.stride(0), y.stride(1), 1, t), b * t, n, 3, norm=ln)
    assert torch.equal(lq, q) and torch.equal(lqs, qs)


@torch.inference_mode()
def test_contract_errors():
    case = Case(1, 1, 4, 1024, 1024, seed=9, scale_dtype=torch.float32)
    s = _slices(case, 1)
    y = torch.empty(4, 1024, device=DEV)
    with pytest.raises(ValueError):
        lowbit.row_epilogue(s[:, :, :, :1022].contiguous(), case.dqs, case.dalpha[:1022].contiguous(), None,
                            y[:, :1022])
    with pytest.raises(ValueError):
        lowbit.row_epilogue(s, case.dqs.half(), case.dalpha, None, y)
    with pytest.raises(ValueError):
        lowbit.row_epilogue(s, case.dqs, case.dalpha, None, y, norm=_layer_norm(1024, 1))
