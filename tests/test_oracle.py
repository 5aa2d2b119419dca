"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each oracle function is checked against something that does not share its code: the reference's own known-answer
vectors (tests/golden/reference_kats.json), brute-force int64 matmuls in numpy, closed forms, numpy's IEEE float16
rounding and torch's bfloat16 rounding. Planted mistakes (a transposed or sign-flipped weight, a dropped part, a
swapped contraction) are applied to the oracle's inputs on the CPU and must be caught by the same checks.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def _rng(seed):
    return np.random.default_rng(seed)


def _signs(rng, n, k):
    return np.where(rng.random((n, k)) < 0.5, -1, 1).astype(np.int8)


# --- formats -------------------------------------------------------------------------------------------------------

def test_format_kats():
    kat = KATS["pack_signs_one_hot"]
    assert O.pack_signs(np.array(kat["signs"], np.int8)).tolist() == kat["codes"]
    with pytest.raises(ValueError, match="tail"):
        O.unpack_bits(np.array(KATS["tail_bits_rejected"]["codes"], np.uint8), KATS["tail_bits_rejected"]["k"])
    kat = KATS["dense_weight"]
    dense = O.dense_weight(O.pack_signs(np.array(kat["signs"], np.int8)), np.array(kat["scale"], np.float32), 3)
    assert dense.tolist() == kat["dense"]
    kat = KATS["pack_ternary"]
    assert O.pack_ternary(np.array(kat["values"], np.int8)).tolist() == kat["codes"]
    for bad in KATS["ternary_rejected"]:
        with pytest.raises(ValueError):
            O.unpack_ternary(np.array(bad["codes"], np.uint8), bad["k"])


@pytest.mark.parametrize("n,k", [(5, 21), (3, 8), (7, 1), (4, 300)])
def test_format_round_trips(n, k):
    rng = _rng(n * 1000 + k)
    s = _signs(rng, n, k)
    assert np.array_equal(O.unpack_signs(O.pack_signs(s), k), s)
    t = rng.integers(-1, 2, (n, k)).astype(np.int8)
    assert np.array_equal(O.unpack_ternary(O.pack_ternary(t), k), t)
    # bit-level closed form: code k at bit k % 8 of byte k // 8, LSB first
    codes = O.pack_signs(s)
    for row in range(n):
        for kk in range(k):
            assert ((codes[row, kk // 8] >> (kk % 8)) & 1) == (s[row, kk] == 1)


# --- the int32 GEMM ------------------------------------------------------------------------------------------------

def _brute(q, w):
    """Independent reference: int64 matmul of the int8 activations with the dense int8 weights."""
    return np.einsum("pmk,nk->pmn", q.astype(np.int64), w.astype(np.int64))


@pytest.mark.parametrize("p,m,n,k", [(1, 5, 7, 9), (3, 17, 33, 130), (2, 1, 16, 640), (1, 64, 40, 1024)])
def test_b1_gemm_matches_brute_force(p, m, n, k):
    rng = _rng(p + m + n + k)
    q = rng.integers(-127, 128, (p, m, k)).astype(np.int8)
    s = _signs(rng, n, k)
    acc = O.b1_gemm(q, O.pack_signs(s), k)
    assert acc.dtype == np.int32 and acc.shape == (p, m, n)
    assert np.array_equal(acc, _brute(q, s))
    assert np.abs(acc).max() <= 127 * k
    # planted mistakes must be caught by the same comparison
    assert not np.array_equal(O.b1_gemm(q, O.pack_signs(-s), k), _brute(q, s))
    if n == k:
        assert not np.array_equal(O.b1_gemm(q, O.pack_signs(np.ascontiguousarray(s.T)), k), _brute(q, s))


@pytest.mark.parametrize("p,m,n,k", [(1, 5, 7, 9), (3, 17, 33, 130), (2, 4, 30, 640)])
def test_t2_gemm_matches_brute_force(p, m, n, k):
    rng = _rng(7 * p + m + n + k)
    q = rng.integers(-127, 128, (p, m, k)).astype(np.int8)
    t = rng.integers(-1, 2, (n, k)).astype(np.int8)
    acc = O.t2_gemm(q, O.pack_ternary(t), k)
    assert np.array_equal(acc, _brute(q, t))
    assert not np.array_equal(O.t2_gemm(q, O.pack_ternary(-t), k), _brute(q, t))


def test_gemm_tiny_hand_computed():
    # q = [1, 2, 3], signs = [+1, -1, +1] -> 1 - 2 + 3 = 2; ternary [0, -1, +1] -> -2 + 3 = 1
    q = np.array([[[1, 2, 3]]], np.int8)
    assert O.b1_gemm(q, O.pack_signs(np.array([[1, -1, 1]], np.int8)), 3).item() == 2
    assert O.t2_gemm(q, O.pack_ternary(np.array([[0, -1, 1]], np.int8)), 3).item() == 1
    # extreme magnitudes: all -127 against all -1 over K = 4096 -> 127 * 4096
    qx = np.full((1, 1, 4096), -127, np.int8)
    assert O.b1_gemm(qx, O.pack_signs(np.full((1, 4096), -1, np.int8)), 4096).item() == 127 * 4096


def test_grouped_accumulators_sum_to_total():
    rng = _rng(11)
    q = rng.integers(-127, 128, (2, 6, 512)).astype(np.int8)
    t = rng.integers(-1, 2, (9, 512)).astype(np.int8)
    acc_g = O.t2_gemm(q, O.pack_ternary(t), 512, group=128)
    assert acc_g.shape == (4, 2, 6, 9)
    assert np.array_equal(acc_g.sum(0), O.t2_gemm(q, O.pack_ternary(t), 512))
    for g in range(4):
        assert np.array_equal(acc_g[g], _brute(q[:, :, 128 * g:128 * (g + 1)], t[:, 128 * g:128 * (g + 1)]))


# --- the FP32 epilogue ---------------------------------------------------------------------------------------------

def _epilogue_f64(acc, qs, alpha, bias):
    y = sum(acc[c].astype(np.float64) * qs[c].astype(np.float64)[:, None] for c in range(acc.shape[0]))
    y = y * alpha.astype(np.float64)[None, :]
    return y if bias is None else y + bias.astype(np.float64)[None, :]


@pytest.mark.parametrize("p", [1, 2, 3])
@pytest.mark.parametrize("with_bias", [False, True])
def test_epilogue_within_reference_tolerance_of_fp64(p, with_bias):
    rng = _rng(p * 10 + with_bias)
    m, n, k = 38, 64, 1024
    q = rng.integers(-127, 128, (p, m, k)).astype(np.int8)
    s = _signs(rng, n, k)
    acc = O.b1_gemm(q, O.pack_signs(s), k)
    qs = (rng.random((p, m)) * 0.02 + 1e-3).astype(np.float32) / np.array([1, 254, 254 ** 2][:p], np.float32)[:, None]
    alpha = (rng.random(n) * 0.02 + 0.001).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32) if with_bias else None
    y = O.epilogue(acc, qs, alpha, bias)
    ref = _epilogue_f64(acc, qs, alpha, bias)
    np.testing.assert_allclose(y, ref, rtol=2e-6, atol=1e-6)  # the reference's tolerance (tests/test_kernels_gpu.py:44)
    # a dropped part is caught
    if p > 1:
        y_drop = O.epilogue(acc[:p - 1], qs[:p - 1], alpha, bias)
        assert not np.allclose(y_drop, ref, rtol=2e-6, atol=1e-6)


def test_epilogue_exact_closed_forms():
    # power-of-two scales: every product and sum is exact, so the FP32 result equals the exact rational value
    acc = np.array([[[3, -5, 1000, -32768]]], np.int32)
    qs = np.array([[0.25]], np.float32)
    alpha = np.array([0.5, 2.0, 0.125, 1.0], np.float32)
    assert O.epilogue(acc, qs, alpha).tolist() == [[0.375, -2.5, 31.25, -8192.0]]
    bias = np.array([1.0, -1.0, 0.5, 0.0], np.float32)
    assert O.epilogue(acc, qs, alpha, bias).tolist() == [[1.375, -3.5, 31.75, -8192.0]]
    # P = 2: fma(a0, s0, a1 * s1) with exact operands
    acc2 = np.array([[[4]], [[-8]]], np.int32)
    assert O.epilogue(acc2, np.array([[0.5], [0.25]], np.float32), np.array([1.0], np.float32)).item() == 0.0


def test_epilogue_order_is_a_distinct_contraction():
    # find inputs where fma(a0, s0, a1*s1) and fma(a1, s1, a0*s0) round differently; the flag must follow
    rng = _rng(5)
    acc = rng.integers(-2 ** 20, 2 ** 20, (2, 1, 4096)).astype(np.int32)
    qs = np.array([[0.0123456], [0.0000987654]], np.float32)
    alpha = np.ones(4096, np.float32)
    y0 = O.epilogue(acc, qs, alpha, order=0)
    y1 = O.epilogue(acc, qs, alpha, order=1)
    a0, a1 = acc[0, 0].astype(np.float32), acc[1, 0].astype(np.float32)
    f0 = (a0.astype(np.float64) * qs[0, 0] + (a1 * qs[1, 0]).astype(np.float64)).astype(np.float32)
    f1 = (a1.astype(np.float64) * qs[1, 0] + (a0 * qs[0, 0]).astype(np.float64)).astype(np.float32)
    # a float64 fma of float32 operands rounded once to float32 is exact here (the products fit in 48 bits)
    assert np.array_equal(y0[0], f0) and np.array_equal(y1[0], f1)
    assert not np.array_equal(y0, y1)


def test_epilogue_silu_and_groups():
    rng = _rng(9)
    acc = rng.integers(-50000, 50000, (1, 8, 32)).astype(np.int32)
    qs = np.full((1, 8), 1e-3, np.float32)
    alpha = np.full(32, 0.01, np.float32)
    y = O.epilogue(acc, qs, alpha)
    ys = O.epilogue(acc, qs, alpha, silu=True)
    ref = y.astype(np.float64) / (1 + np.exp(-y.astype(np.float64)))
    np.testing.assert_allclose(ys, ref, rtol=1e-6, atol=1e-7)
    # per-group scales with all groups equal to the per-channel scale: fma chain = the same sum up to rounding
    acc_g = rng.integers(-3000, 3000, (4, 2, 3, 5)).astype(np.int32)
    qs2 = np.array([[0.5, 0.25, 1.0], [2 ** -9, 2 ** -8, 2 ** -7]], np.float32)
    al = np.array([[0.5] * 4, [0.25] * 4, [1.0] * 4, [2.0] * 4, [0.125] * 4], np.float32)
    yg = O.epilogue(acc_g, qs2, al)
    exact = (acc_g[:, 0].astype(np.float64) * qs2[0][None, :, None] + acc_g[:, 1].astype(np.float64)
             * qs2[1][None, :, None]).sum(0) * al[:, 0][None, :].astype(np.float64)
    assert np.array_equal(yg.astype(np.float64), exact)  # power-of-two scales, small integers: exact


# --- float16 / bfloat16 rounding -----------------------------------------------------------------------------------

def _special_floats():
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e9, -1e9, 6e-8, 2.9802322e-08,
            2.9802326e-08, 5.9604645e-08, 6.1035156e-05, 6.1e-05, 1.0009765625, 1.00048828125, 1.00146484375,
            float("inf"), float("-inf")]
    ties = [1 + (2 * i + 1) * 2.0 ** -11 for i in range(64)] + [2.0 ** -24 * (i + 0.5) for i in range(64)]
    return np.array(vals + ties, np.float32)


def test_f16_rounding_matches_numpy():
    rng = _rng(3)
    x = np.concatenate([_special_floats(), rng.standard_normal(200000).astype(np.float32) * 300,
                        (rng.standard_normal(100000) * 1e-5).astype(np.float32),
                        rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    x = x[~np.isnan(x)]
    assert np.array_equal(O.to_f16_bits(x), x.astype(np.float16).view(np.uint16))


def test_bf16_rounding_matches_torch():
    rng = _rng(4)
    x = np.concatenate([_special_floats(), rng.integers(0, 2 ** 32, 300000, dtype=np.uint64).astype(np.uint32)
                        .view(np.float32)])
    x = x[~np.isnan(x)]
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.to_bf16_bits(x), ref)


# --- the quantizer -------------------------------------------------------------------------------------------------

def _numpy_quantize(z, parts):
    """Independent restatement in numpy float32 (IEEE division, rint = round half to even)."""
    z = z.astype(np.float32).copy()
    qs, qv = [], []
    for _ in range(parts):
        s = np.maximum(np.abs(z).max(axis=1) / np.float32(127), np.float32(1e-30)).astype(np.float32)
        q = np.clip(np.rint(z / s[:, None]), -127, 127).astype(np.float32)
        qv.append(q.astype(np.int8))
        qs.append(s)
        z = (z - (q * s[:, None]).astype(np.float32)).astype(np.float32)
    return np.stack(qv), np.stack(qs)


@pytest.mark.parametrize("k", [16, 300, 1024])
def test_quantize_matches_numpy_and_invariants(k):
    rng = _rng(k)
    x = rng.standard_normal((37, k)).astype(np.float32) * np.float32(3)
    x[0] = 0.0  # an all-zero row: scale 1e-30, q = 0
    q, qs = O.quantize(x, 3, ldq=-(-k // 16) * 16)
    qn, qsn = _numpy_quantize(x, 3)
    assert np.array_equal(q[:, :, :k], qn) and np.array_equal(qs, qsn)
    assert not q[:, :, k:].any()
    assert np.abs(q).max() <= 127
    err = np.abs(x - q[0, :, :k].astype(np.float32) * qs[0][:, None])
    assert (err <= qs[0][:, None] * 0.5 * (1 + 1e-6)).all()
    for p in (1, 2):  # the first P parts of the 3-part quantizer are the P-part quantizer
        qp, qsp = O.quantize(x, p, ldq=q.shape[2])
        assert np.array_equal(qp, q[:p]) and np.array_equal(qsp, qs[:p])


def test_quantize_layernorm_close_to_fp64():
    rng = _rng(21)
    k = 1024
    x = rng.standard_normal((9, k)).astype(np.float32) * 2 + 0.5
    w = (rng.random(k) + 0.5).astype(np.float32)
    b = (rng.standard_normal(k) * 0.1).astype(np.float32)
    q, qs = O.quantize(x, 3, norm=(w, b), eps=1e-5)
    xd = x.astype(np.float64)
    ref = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-5) * w + b
    recon = sum(q[c].astype(np.float64) * qs[c][:, None] for c in range(3))
    np.testing.assert_allclose(recon, ref, rtol=0, atol=1e-5)


def test_quantize_fp16_scales_clamp():
    rng = _rng(22)
    x = rng.standard_normal((8, 256)).astype(np.float32)
    q, qs = O.quantize(x, 1, qs_f16=True)
    assert np.array_equal(qs.astype(np.float16).astype(np.float32), qs)  # representable in fp16
    assert np.abs(q).max() <= 127
    ref = np.clip(np.rint(x / qs[0][:, None]), -127, 127)
    assert np.array_equal(q[0].astype(np.float32), ref)


@pytest.mark.parametrize("parts", [1, 2, 3])
@pytest.mark.parametrize("qs_f16", [False, True])
def test_quantize_rounds_exact_ties_half_to_even(parts, qs_f16):
    """The oracle's quantizer on rows whose quotients are exact half-integers: 0.5 -> 0, 1.5 -> 2, -2.5 -> -2, ...
    (expected codes from integer arithmetic, tests/tie_rows.py); a round-half-away rule fails here."""
    from tie_rows import NAMED, tie_rows
    x, want = tie_rows(9, 300, seed=parts + 10 * qs_f16)
    q, qs = O.quantize(x, parts, qs_f16=qs_f16)
    assert np.array_equal(q[0], want)
    # the scale is the power of two the row was built on: amax / 127 exactly
    assert np.array_equal(qs[0], np.abs(x).max(axis=1) / 127)
    for h, c in NAMED.items():
        cols = np.nonzero(x[0] == np.float32(h * qs[0, 0]))[0]
        assert cols.size and (q[0, 0, cols] == c).all(), h
