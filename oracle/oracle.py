"""CPU oracle for the low-bit GEMM path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, and only as the checker
(or the timed CPU baseline); the product package never does. It restates the reference on its EXPORT layouts:

    numpy (formats)  pack_signs / unpack_bits / unpack_signs / dense_weight   kk/binary/bits.py:41-69
                     pack_ternary / unpack_ternary                             kk/formats.py:62-81
    C (kea_oracle.c) b1_gemm / t2_gemm / epilogue / quantize / f16 and bf16 rounding (see that file's header)

Pinning (tests/test_oracle.py): the reference's known-answer tests (tests/test_formats.py:14-59 of the reference,
restated as fixtures in tests/golden/), brute-force int64 matmuls written independently of the C loops, closed
forms (power-of-two scales, all-equal rows), numpy's own IEEE float16 rounding, torch's bfloat16 rounding, and a
planted-mistake check that a transposed or sign-flipped weight fails them.
"""
from __future__ import annotations

import ctypes
import math
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
_LIB = HERE / "lib" / "libkea_oracle.so"
_lib = None


def lib():
    """The oracle shared library (built by oracle/build.py)."""
    global _lib
    if _lib is None:
        if not _LIB.is_file():
            raise RuntimeError(f"{_LIB} is missing: run `python oracle/build.py` (or __graft_entry__.build())")
        L = ctypes.CDLL(str(_LIB))
        i64, i32, vp, f32 = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_float
        L.oracle_set_threads.argtypes, L.oracle_set_threads.restype = [i32], i32
        for name in ("oracle_b1_gemm", "oracle_t2_gemm"):
            fn = getattr(L, name)
            fn.argtypes = [vp, i64, i64, i32, vp, i64, i64, i64, i64, vp]
            fn.restype = i32
        L.oracle_epilogue.argtypes = [vp, i64, i32, i64, i64, vp, vp, i32, vp, i32, vp]
        L.oracle_epilogue.restype = i32
        L.oracle_f32_to_f16.argtypes = [vp, vp, i64]
        L.oracle_f32_to_bf16.argtypes = [vp, vp, i64]
        L.oracle_quantize.argtypes = [vp, i32, i64, i64, i64, i64, i64, i64, i32, vp, vp, f32, i32, vp, i64, vp, i32]
        L.oracle_quantize.restype = i32
        _lib = L
    return _lib


def set_threads(n: int) -> int:
    """OpenMP threads used by the oracle's loops; returns the effective count."""
    return lib().oracle_set_threads(int(n))


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# --- export formats (numpy restatements) --------------------------------------------------------------------------

def packed_row_bytes(k: int) -> int:
    return math.ceil(k / 8)


def pack_signs(signs: np.ndarray) -> np.ndarray:
    """int8 {-1, +1} [N, K] -> uint8 [N, ceil(K/8)]: code k is bit k % 8 of byte k // 8, 1 = +1 (kk/binary/bits.py:56-64)."""
    signs = np.asarray(signs)
    if signs.ndim != 2 or not np.isin(signs, (-1, 1)).all():
        raise ValueError("expected 2-D signs in {-1, +1}")
    n, k = signs.shape
    bits = np.zeros((n, 8 * packed_row_bytes(k)), np.uint8)
    bits[:, :k] = signs == 1
    return np.packbits(bits.reshape(n, -1, 8), axis=2, bitorder="little").reshape(n, -1)


def unpack_bits(codes: np.ndarray, k: int) -> np.ndarray:
    """uint8 [N, ceil(K/8)] -> {0, 1} [N, K]; nonzero tail bits raise (kk/binary/bits.py:41-48)."""
    codes = np.asarray(codes, np.uint8)
    if codes.ndim != 2 or codes.shape[1] != packed_row_bytes(k):
        raise ValueError("bad code shape")
    bits = np.unpackbits(codes, axis=1, bitorder="little")
    if bits[:, k:].any():
        raise ValueError("invalid packed codes: nonzero tail padding")
    return bits[:, :k]


def unpack_signs(codes: np.ndarray, k: int) -> np.ndarray:
    return (2 * unpack_bits(codes, k).astype(np.int8) - 1).astype(np.int8)


def dense_weight(codes: np.ndarray, scale: np.ndarray, k: int) -> np.ndarray:
    """signs * scale[:, None] in float64 (kk/binary/bits.py:67-69)."""
    return unpack_signs(codes, k).astype(np.float64) * np.asarray(scale, np.float64)[:, None]


def pack_ternary(values: np.ndarray) -> np.ndarray:
    """int8 {-1, 0, +1} [N, K] -> uint8 [N, ceil(K/4)]: 0 -> 00, +1 -> 01, -1 -> 10 at bits 2(k % 4) (kk/formats.py:62-70)."""
    values = np.asarray(values)
    if values.ndim != 2 or not np.isin(values, (-1, 0, 1)).all():
        raise ValueError("expected 2-D codes in {-1, 0, 1}")
    n, k = values.shape
    fields = np.zeros((n, 4 * math.ceil(k / 4)), np.uint8)
    fields[:, :k] = (values == 1).astype(np.uint8) | ((values == -1).astype(np.uint8) << 1)
    f = fields.reshape(n, -1, 4)
    return (f[..., 0] | (f[..., 1] << 2) | (f[..., 2] << 4) | (f[..., 3] << 6)).astype(np.uint8)


def unpack_ternary(packed: np.ndarray, k: int) -> np.ndarray:
    """Inverse of pack_ternary; the 11 pattern and nonzero tail codes raise (kk/formats.py:73-81)."""
    packed = np.asarray(packed, np.uint8)
    if packed.ndim != 2 or packed.shape[1] != math.ceil(k / 4):
        raise ValueError("bad code shape")
    fields = np.stack([(packed >> s) & 3 for s in (0, 2, 4, 6)], axis=2).reshape(packed.shape[0], -1)
    if (fields == 3).any() or fields[:, k:].any():
        raise ValueError("invalid packed codes")
    fields = fields[:, :k]
    return ((fields == 1).astype(np.int8) - (fields == 2).astype(np.int8)).astype(np.int8)


# --- the GEMM, epilogue, rounding and quantizer (C) ---------------------------------------------------------------

def _q3(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, np.int8)
    return q[None] if q.ndim == 2 else q


def b1_gemm(q: np.ndarray, codes: np.ndarray, k: int, group: int | None = None) -> np.ndarray:
    """Exact int32 accumulators. q int8 [P, M, ldq] (or [M, ldq]); codes uint8 [N, ceil(K/8)].
    Returns [P, M, N], or [G, P, M, N] with group = k-size of a group."""
    return _gemm("oracle_b1_gemm", q, codes, k, group)


def t2_gemm(q: np.ndarray, codes: np.ndarray, k: int, group: int | None = None) -> np.ndarray:
    """As b1_gemm for 2-bit ternary export codes uint8 [N, ceil(K/4)]."""
    return _gemm("oracle_t2_gemm", q, codes, k, group)


def _gemm(name, q, codes, k, group):
    q = _q3(q)
    codes = np.ascontiguousarray(codes, np.uint8)
    p, m, ldq = q.shape
    n = codes.shape[0]
    g = k if group is None else int(group)
    groups = math.ceil(k / g)
    acc = np.zeros((groups, p, m, n), np.int32)
    rc = getattr(lib(), name)(_ptr(q), m * ldq, ldq, p, _ptr(codes), n, k, m, g, _ptr(acc))
    if rc:
        raise ValueError(f"{name} rejected its arguments")
    return acc[0] if group is None else acc


def epilogue(acc: np.ndarray, qs: np.ndarray, alpha: np.ndarray, bias: np.ndarray | None = None, *,
             silu: bool = False, order: int = 0) -> np.ndarray:
    """FP32 epilogue. acc int32 [P, M, N] with alpha [N], or [G, P, M, N] with alpha [N, G]; qs [P, M]."""
    acc = np.ascontiguousarray(acc, np.int32)
    grouped = acc.ndim == 4
    if not grouped:
        acc = acc[None]
    groups, p, m, n = acc.shape
    qs = np.ascontiguousarray(np.asarray(qs, np.float32).reshape(p, m))
    alpha = np.ascontiguousarray(alpha, np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
    out = np.empty((m, n), np.float32)
    flags = int(silu) | 2 * int(order)
    rc = lib().oracle_epilogue(_ptr(acc), groups, p, m, n, _ptr(qs), _ptr(alpha), int(grouped), _ptr(bias), flags,
                               _ptr(out))
    if rc:
        raise ValueError("oracle_epilogue rejected its arguments")
    return out


def to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_f32_to_f16(_ptr(x), _ptr(out), x.size)
    return out


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_f32_to_bf16(_ptr(x), _ptr(out), x.size)
    return out


def quantize(x: np.ndarray, parts: int, *, ldq: int | None = None, norm: tuple | None = None, eps: float = 1e-5,
             input_silu: bool = False, qs_f16: bool = False, t: int | None = None):
    """Residual int8 quantizer on a contiguous [M, K] (float32 or float16) array.
    Returns q int8 [parts, M, ldq] and qs float32 [parts, M] (fp16-rounded values when qs_f16)."""
    x = np.ascontiguousarray(x)
    x_f16 = x.dtype == np.float16
    if not x_f16:
        x = np.ascontiguousarray(x, np.float32)
    m, k = x.shape
    ldq = k if ldq is None else ldq
    q = np.empty((parts, m, ldq), np.int8)
    qs = np.empty((parts, m), np.float32)
    nw = nb = None
    if norm is not None:
        nw = np.ascontiguousarray(norm[0], np.float32)
        nb = np.ascontiguousarray(norm[1], np.float32)
    tt = m if t is None else t
    xb, xt = tt * k, k
    rc = lib().oracle_quantize(_ptr(x.view(np.uint16) if x_f16 else x), int(x_f16), xb, xt, 1, max(tt, 1), m, k,
                               parts, _ptr(nw), _ptr(nb), float(eps), int(input_silu), _ptr(q), ldq, _ptr(qs),
                               int(qs_f16))
    if rc:
        raise ValueError("oracle_quantize rejected its arguments")
    return q, qs
