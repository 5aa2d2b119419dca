"""Activation rows whose first-part quotients z / s are exact half-integers, for pinning the quantizer's rounding rule
(round half to even: kk/ternary/fused_kernels.py:47 `nearbyint`, the `cvt.rni` of kk/binary/kernels.py:585-614).

Row r holds amax = 127 * 2^e (so s = amax / 127 = 2^e exactly, also as an fp16 scale) and, everywhere else, values
(j + 1/2) * 2^e with integers j in [-127, 126]: z / s = j + 1/2 exactly, and z * (1 / s) is that same value with no
rounding. The expected code of each element is written from the integers alone (half to even: j when j is even,
else j + 1), not from any floating-point rounding routine, so a rule that rounds ties away from zero (roundf) or up
fails it at the first odd or even j."""
from __future__ import annotations

import numpy as np

# the tie cases the rounding rule is named by: +-0.5 -> 0, 1.5 -> 2, 2.5 -> 2, -1.5 -> -2, -2.5 -> -2, ...
NAMED = {0.5: 0, -0.5: 0, 1.5: 2, -1.5: -2, 2.5: 2, -2.5: -2, 3.5: 4, -3.5: -4, 126.5: 126, -126.5: -126,
         125.5: 126, -125.5: -126}


def tie_rows(m: int, k: int, seed: int, dtype=np.float32):
    """x [m, k] of `dtype` and the expected first-part codes int8 [m, k] (the amax element's code is +-127)."""
    rng = np.random.default_rng(seed)
    x = np.empty((m, k), np.float64)
    code = np.empty((m, k), np.int64)
    named = np.array(sorted(NAMED), np.float64)
    for r in range(m):
        e = int(rng.integers(-6, 3))                     # s = 2^e, within fp16's normal range
        j = rng.integers(-127, 127, size=k)              # (j + 1/2) in [-126.5, 126.5]
        h = j + 0.5
        h[: min(k, named.size)] = named[: min(k, named.size)]
        jj = np.floor(h).astype(np.int64)
        code[r] = np.where(jj % 2 == 0, jj, jj + 1)      # half to even, from the integers
        at = int(rng.integers(0, k))
        sign = 1 if rng.random() < 0.5 else -1
        h[at] = 127.0 * sign
        code[r, at] = 127 * sign
        x[r] = np.ldexp(h, e)
    return x.astype(dtype), code.astype(np.int8)
