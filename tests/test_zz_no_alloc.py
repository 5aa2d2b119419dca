"""kea_lowbit_gemm_noalloc, the allocation-free variant of kea_lowbit_gemm (include/kea_lowbit.h): called through the
C ABI, its outputs equal kea_lowbit_gemm's bit for bit (and the oracle's int32 accumulators) on calls in a row that
use its split-K scratch array, the later calls smaller than the first, so stale slices of a larger earlier call
cannot leak into a smaller one."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from kea_kernels import _hip
from kea_kernels.binary import kernels
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
vp, i64 = ctypes.c_void_p, ctypes.c_int64


def _inputs(wbits, m, n, k, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-127, 128, (1, m, k), generator=g, dtype=torch.int8)
    qs = (torch.rand(1, m, generator=g) * 0.02 + 1e-3).to(torch.float16)
    alpha = (torch.rand(n, generator=g) * 0.09 + 0.01).to(torch.float16)
    if wbits == 1:
        codes = O.pack_signs(torch.where(torch.rand(n, k, generator=g) < 0.5, -1, 1).to(torch.int8).numpy())
        acc = O.b1_gemm(q.numpy(), codes, k)
    else:
        codes = O.pack_ternary(torch.randint(-1, 2, (n, k), generator=g, dtype=torch.int8).numpy())
        acc = O.t2_gemm(q.numpy(), codes, k)
    words = kernels.relayout_codes(torch.from_numpy(codes), k, wbits).to(DEV)
    return q.to(DEV), qs.to(DEV), alpha.to(DEV), words, acc


def _call(fn, wbits, q, qs, words, n, k, alpha, y, acc, m, split, config, workspace=None):
    stream = vp(torch.cuda.current_stream().cuda_stream)
    args = [wbits, vp(q.data_ptr()), i64(m * k), i64(k), 1, vp(qs.data_ptr()), _hip.F16, i64(m),
            vp(words.data_ptr()), i64(n), i64(k), vp(alpha.data_ptr()), _hip.F16, i64(0), None, 0,
            vp(y.data_ptr()), _hip.F16, i64(n), vp(acc.data_ptr()), i64(n), i64(m), 0, split, config]
    if workspace is not None:
        args += [vp(workspace.data_ptr()) if workspace.numel() else None, i64(workspace.numel())]
    return fn(*args, stream)


@torch.inference_mode()
def test_noalloc_equals_the_workspace_entry_point_on_successive_calls():
    L = _hip.lib()
    # (wbits, m, n, k, config, split): ring tile 32x32 split 4, then smaller: a wave-split tile whose K range needs
    # two slices, a ring split of 2, and the two producer-wave tiles split 3 and 2; every call uses the scratch
    # array (workspace > 0)
    wsplit_16x32 = next(t for t in range(1, kernels.tile_count() + 1) if kernels.config_name(t) == "16x32 k/4")
    cases = [(2, 96, 1024, 8192, 4, 4), (1, 40, 512, 8192, wsplit_16x32, 0), (2, 24, 300, 4096, 4, 2),
             (1, 70, 512, 4096, 6, 3), (2, 50, 256, 2048, 7, 2)]
    for i, (wbits, m, n, k, config, split) in enumerate(cases):
        need = L.kea_lowbit_gemm_workspace(wbits, 1, m, n, k, 0, split, config)
        assert 0 < need <= 8 << 20, (i, need)
        q, qs, alpha, words, ref_acc = _inputs(wbits, m, n, k, seed=70 + i)
        y_ref = torch.full((m, n), float("nan"), device=DEV, dtype=torch.float16)
        a_ref = torch.full((1, m, n), -7, device=DEV, dtype=torch.int32)
        ws = torch.empty(need, dtype=torch.uint8, device=DEV)
        rc = _call(L.kea_lowbit_gemm, wbits, q, qs, words, n, k, alpha, y_ref, a_ref, m, split, config, ws)
        assert rc == 0, _hip.last_error()
        y = torch.full((m, n), float("nan"), device=DEV, dtype=torch.float16)
        a = torch.full((1, m, n), -7, device=DEV, dtype=torch.int32)
        rc = _call(L.kea_lowbit_gemm_noalloc, wbits, q, qs, words, n, k, alpha, y, a, m, split, config)
        assert rc == 0, _hip.last_error()
        torch.cuda.synchronize()
        assert np.array_equal(a.cpu().numpy(), ref_acc), f"call {i}: int32 accumulators differ from the oracle"
        assert torch.equal(a, a_ref), f"call {i}"
        assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16)), f"call {i}: outputs differ"


@torch.inference_mode()
def test_noalloc_refuses_more_than_its_scratch():
    L = _hip.lib()
    m, n, k = 1000, 4096, 8192
    assert L.kea_lowbit_gemm_workspace(1, 1, m, n, k, 0, 8, 4) > 8 << 20
    y = torch.empty(1, device=DEV)
    rc = L.kea_lowbit_gemm_noalloc(1, vp(y.data_ptr()), m * k, k, 1, vp(y.data_ptr()), 1, m, vp(y.data_ptr()), n, k,
                                   vp(y.data_ptr()), 1, 0, None, 0, vp(y.data_ptr()), 1, n, None, 0, m, 0, 8, 4, None)
    assert rc == -4 and b"scratch" in _hip.lib().kea_last_error()
