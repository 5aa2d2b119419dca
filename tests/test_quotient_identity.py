"""The quantizers' rounding step without a division per element (kea_quantize.hip, round_quotient).

The kernels compute rint(z / s) as rint(fma(fma(-q, s, z), inv, q)) with q = RN(z * inv) and inv = RN(1 / s): one
correction step with the residual of the division. The oracle divides (IEEE, correctly rounded). This test emulates
the kernel's float32 operations exactly on the CPU (products of two float32 values are exact in float64; the sums are
carried as error-free float64 pairs and rounded once to float32) and checks the corrected quotient bitwise against
numpy's float32 division, on random rows and on values placed within a few ulps of every half-integer, for float32
scales and for scales rounded to float16 as the kernels store them. It also checks that the uncorrected product is
caught, so the emulation is strong enough to see a wrong rounding.
"""
from __future__ import annotations

import numpy as np
import pytest

F32, F64 = np.float32, np.float64


def _two_sum(a, b):
    s = a + b
    bb = s - a
    return s, (a - (s - bb)) + (b - bb)


def _round32(hi, lo):
    """Round-to-nearest-even float32 of the exact value hi + lo (|lo| at most half a float64 ulp of hi)."""
    c = hi.astype(F32)
    cf = c.astype(F64)
    other = np.where(hi > cf, np.nextafter(c, F32(np.inf)), np.nextafter(c, F32(-np.inf))).astype(F64)
    tie = hi == (cf + other) / 2
    return np.where(tie & (np.sign(lo) == np.sign(other - cf)), other.astype(F32), c)


def _fma32(a, b, c):
    hi, lo = _two_sum(a.astype(F64) * b.astype(F64), c.astype(F64))
    return _round32(hi, lo)


def _rows(seed, f16_scale):
    rng = np.random.default_rng(seed)
    amax = F32(10 ** rng.uniform(-20, 5))
    s = F32(max(amax / F32(127), F32(1e-30)))
    if f16_scale:
        s = F32(min(max(F32(np.float16(s)), F32(2.0 ** -24)), F32(65504)))
    z = (rng.uniform(-1, 1, 100_000) * amax).astype(F32)
    near = ((rng.integers(-127, 127, 100_000) + 0.5) * F64(s)).astype(F32)
    steps = rng.integers(-3, 4, near.size)
    for d in range(3):
        near = np.where(steps > d, np.nextafter(near, F32(np.inf)), near)
        near = np.where(steps < -d, np.nextafter(near, F32(-np.inf)), near)
    return np.concatenate([z, near.astype(F32)]), s


@pytest.mark.parametrize("seed", range(12))
def test_corrected_quotient_is_the_ieee_quotient(seed):
    z, s = _rows(seed, f16_scale=seed % 2 == 1)
    inv = np.full(z.shape, F32(1) / s, F32)
    sv = np.full(z.shape, s, F32)
    q = (z * inv).astype(F32)
    corrected = _fma32(_fma32(-q, sv, z), inv, q)
    ieee = (z / s).astype(F32)
    # below 1/4 the residual may underflow; the rounded integer is 0 either way
    big = np.abs(ieee) >= 0.25
    assert np.array_equal(corrected.view(np.uint32)[big], ieee.view(np.uint32)[big])
    clamp = lambda v: np.clip(np.rint(v), -127, 127)
    assert np.array_equal(clamp(corrected), clamp(ieee))


def test_uncorrected_product_is_caught():
    """Without the correction step the same check fails: z * inv rounds differently near half-integers."""
    clamp = lambda v: np.clip(np.rint(v), -127, 127)
    wrong = 0
    for seed in range(12):
        z, s = _rows(seed, f16_scale=seed % 2 == 1)
        wrong += int((clamp((z * (F32(1) / s)).astype(F32)) != clamp((z / s).astype(F32))).sum())
    assert wrong > 0
