"""CPU tests of the C ABI library: it loads, exports every function include/*.h declares, its host-side
layout functions place every code where the header says, and its argument validation rejects bad calls before any
GPU work (no compute call is made without a GPU)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from kea_kernels import _hip
from oracle import oracle as O

INCLUDE = Path(__file__).resolve().parents[1] / "include"
# the product library's headers; include/kea_probe.h declares the benchmark's separate probe library
HEADERS = sorted(h for h in INCLUDE.glob("*.h") if h.name != "kea_probe.h")
PROBE_HEADER = INCLUDE / "kea_probe.h"


def declared_functions(headers=HEADERS) -> list[str]:
    names = set()
    for header in headers:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names.update(re.findall(r"\b(kea_\w+)\s*\(", text))
    return sorted(names)


def _exported(path: Path) -> set[str]:
    """Dynamic symbols a shared library defines (nm -D --defined-only)."""
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_library_exports_every_declared_function():
    names = declared_functions()
    assert len(HEADERS) >= 2 and len(names) >= 10
    assert {"kea_lowbit_gemm", "kea_quantize", "kea_relpos_attention", "kea_glu_dwconv"} <= set(names)
    L = _hip.lib()
    for name in names:
        assert hasattr(L, name), name
        assert name in _hip.SIGNATURES, f"{name} has no ctypes signature"
    assert L.kea_version() >= 100
    assert L.kea_config_count() >= 1 and L.kea_config_name(1)
    # the product library carries no measurement probes: they live in the benchmark's libkea_probe.so
    assert not {s for s in _exported(_hip.LIB_PATH) if s.startswith("kea_probe")}


def test_probe_library_exports_every_declared_function():
    import kea_probes
    names = declared_functions([PROBE_HEADER])
    assert "kea_probe_spin" in names and "kea_probe_last_error" in names
    L = kea_probes.lib()
    for name in names:
        assert hasattr(L, name), name
        assert name in kea_probes.SIGNATURES, f"{name} has no ctypes signature"
    assert set(names) == {s for s in _exported(kea_probes.LIB_PATH) if s.startswith("kea_")}


def _words(wbits, codes, n, k):
    L = _hip.lib()
    count = (L.kea_b1_native_words if wbits == 1 else L.kea_t2_native_words)(n, k)
    words = np.zeros(count, np.uint32)
    fn = L.kea_b1_relayout_host if wbits == 1 else L.kea_t2_relayout_host
    rc = fn(codes.ctypes.data_as(ctypes.c_void_p), n, k, words.ctypes.data_as(ctypes.c_void_p))
    return rc, words


def _index(t, j, lane, J):
    jq = j // 4
    wq = min(4, J - 4 * jq)
    return t * J * 64 + jq * 256 + lane * wq + (j - 4 * jq)


@pytest.mark.parametrize("n,k", [(1, 1), (16, 128), (20, 300), (33, 640), (5, 1100), (130, 200)])
def test_b1_native_layout_places_every_code(n, k):
    rng = np.random.default_rng(n * 7 + k)
    signs = np.where(rng.random((n, k)) < 0.5, -1, 1).astype(np.int8)
    codes = O.pack_signs(signs)
    rc, words = _words(1, codes, n, k)
    assert rc == 0
    J = -(-k // 128)
    P0 = -(-n // 16) * J * 64                      # the word part, then the bit-plane part
    KS = -(-k // 64)
    assert words.size == P0 + -(-n // 128) * KS * 64 * 4
    # the header's formula: word j of lane l of tile t, bit 8i + 4h + d = inverted sign of w[16t + l%16][128j + ...]
    for row in range(n):
        t, c = divmod(row, 16)
        for kk in range(k):
            j, r = divmod(kk, 128)
            h, r = divmod(r, 64)
            g, r = divmod(r, 16)
            d, i = divmod(r, 4)
            bit = (words[_index(t, j, c + 16 * g, J)] >> (8 * i + 4 * h + d)) & 1
            assert bit == (signs[row, kk] == -1)
    # the bit-plane part: unit (group, k-step, lane) word d, bit 8i + p = inverted sign of
    # w[128 group + 16p + lane%16][64 kstep + 16(lane/16) + 4d + i]; rows and k past the matrix are 0
    planes = words[P0:].reshape(-(-n // 128), KS, 64, 4)
    expect = np.zeros_like(planes)
    for row in range(n):
        grp, r = divmod(row, 128)
        pl, c = divmod(r, 16)
        for kk in range(k):
            s_, r2 = divmod(kk, 64)
            g2, r2 = divmod(r2, 16)
            d, i = divmod(r2, 4)
            if signs[row, kk] == -1:
                expect[grp, s_, c + 16 * g2, d] |= np.uint32(1 << (8 * i + pl))
    assert np.array_equal(planes, expect)
    back = np.zeros_like(codes)
    assert _hip.lib().kea_b1_unlayout_host(words.ctypes.data_as(ctypes.c_void_p), n, k,
                                           back.ctypes.data_as(ctypes.c_void_p)) == 0
    assert np.array_equal(back, codes)


@pytest.mark.parametrize("n,k", [(1, 1), (16, 64), (20, 300), (33, 640)])
def test_t2_native_layout_places_every_code(n, k):
    rng = np.random.default_rng(n * 11 + k)
    values = rng.integers(-1, 2, (n, k)).astype(np.int8)
    codes = O.pack_ternary(values)
    rc, words = _words(2, codes, n, k)
    assert rc == 0
    J = -(-k // 64)
    for row in range(n):
        t, c = divmod(row, 16)
        for kk in range(k):
            j, r = divmod(kk, 64)
            g, r = divmod(r, 16)
            d, i = divmod(r, 4)
            code = (words[_index(t, j, c + 16 * g, J)] >> (8 * i + 2 * d)) & 3
            assert code == {0: 0, 1: 1, -1: 2}[int(values[row, kk])]
    back = np.zeros_like(codes)
    assert _hip.lib().kea_t2_unlayout_host(words.ctypes.data_as(ctypes.c_void_p), n, k,
                                           back.ctypes.data_as(ctypes.c_void_p)) == 0
    assert np.array_equal(back, codes)


def test_relayout_rejects_invalid_codes():
    bad = np.array([[0, 0x80], [0, 0]], np.uint8)  # K = 12: bit 15 is tail padding
    rc, _ = _words(1, bad, 2, 12)
    assert rc == -3 and "tail" in _hip.last_error()
    rc, _ = _words(2, np.array([[0b11]], np.uint8), 1, 4)
    assert rc == -3
    rc, _ = _words(2, np.array([[0b01_00_00_00]], np.uint8), 1, 3)
    assert rc == -3


def test_gemm_argument_validation_happens_before_any_launch():
    L = _hip.lib()
    args = dict(wbits=1, q=None, part_stride=0, ldq=1024, parts=1, qs=None, qs_dtype=0, qs_stride=0, w=None, n=4096,
                k=1024, ws=None, ws_dtype=0, ws_group=0, bias=None, bias_dtype=0, y=None, y_dtype=0, ldy=4096,
                acc=None, acc_ld=0, m=128, flags=0, split=1, config=0, workspace=None, wsb=0, stream=None)

    def call(**over):
        a = dict(args, **over)
        return L.kea_lowbit_gemm(*a.values())

    assert call(wbits=3) == -1 and "wbits" in _hip.last_error()
    assert call(parts=4) == -1
    assert call() == -1  # missing q / w / scales
    fake = 4096  # never dereferenced: validation fails first
    base = dict(q=fake, qs=fake, w=fake, ws=fake, y=fake)
    assert call(**base, flags=8) == -1 and "flags" in _hip.last_error()
    assert call(**base, ldq=1000) == -1  # ldq < k
    assert call(**base, ldq=1032) == -2 and "aligned" in _hip.last_error()  # ldq % 16
    assert call(**dict(base, q=fake + 4)) == -2
    # scales and bias at less than their element alignment (f32: 4 bytes, f16: 2) are refused, not read misaligned
    for over in (dict(qs=fake + 2), dict(ws=fake + 2), dict(bias=fake + 2), dict(ws=fake + 1, ws_dtype=1)):
        assert call(**dict(base, **over)) == -2 and "element size" in _hip.last_error()
    assert call(**dict(base, ws=fake + 2, ws_dtype=1, split=4)) == -4  # f16 at a 2-byte offset passes this check
    assert call(**base, y_dtype=7) == -1
    assert call(**base, ldy=100) == -1
    assert call(**base, config=999) == -1
    assert call(**base, split=4) == -4 and "workspace" in _hip.last_error()
    assert call(**base, ws_group=100) == -1


def test_grids_past_one_dispatch_are_refused_before_any_launch():
    """A dispatch holds each grid dimension as a 32-bit work-item count; launches past it would be truncated and
    leave outputs unwritten, so the entry points refuse them (the checks run before any HIP call: the fake device
    pointers below are never dereferenced)."""
    L = _hip.lib()
    fake, big = 4096, 2**31 - 1
    # GEMM: N = 2^31 - 1 needs > 2^32 work-items along N for every tile
    rc = L.kea_lowbit_gemm(1, fake, 0, 1024, 1, fake, 0, 0, fake, big, 1024, fake, 0, 0, None, 0, fake, 1, big,
                           None, 0, 128, 0, 1, 0, None, 0, None)
    assert rc == -1 and "too large for one launch" in _hip.last_error()
    # N = 2^30: a grid that fits one dispatch, refused because the epilogues address per-column vectors with 32-bit
    # byte offsets (ldy = N; fake pointers, nothing launched)
    n30 = 2**30
    rc = L.kea_lowbit_gemm(1, fake, 0, 1024, 1, fake, 0, 0, fake, n30, 1024, fake, 0, 0, None, 0, fake, 1, n30,
                           None, 0, 128, 0, 1, 0, None, 0, None)
    assert rc == -1 and "too large for one launch" in _hip.last_error()
    # the same N with M = 0 is an empty call, not an error
    assert L.kea_lowbit_gemm(1, fake, 0, 1024, 1, fake, 0, 0, fake, big, 1024, fake, 0, 0, None, 0, fake, 1, big,
                             None, 0, 0, 0, 1, 0, None, 0, None) == 0
    # split-K finish over M x N / 4 lanes
    rc = L.kea_lowbit_slices_finish(fake, 2, 1, big, 4096, fake, 0, 0, fake, 0, None, 0, fake, 1, 4096, None, 0, 0,
                                    None)
    assert rc == -1 and "too large for one launch" in _hip.last_error()
    # per-token quantizer: one workgroup per row at K > 256
    rc = L.kea_quantize(fake, 0, 0, 1024, 1, big, big, 1024, 1, None, None, 1e-5, 0, fake, 1024, fake, 0, None)
    assert rc == -1 and "too large for one launch" in _hip.last_error()
    # the boundary: 2^24 rows of 256 work-items are one past the 32-bit count
    assert L.kea_quantize(fake, 0, 0, 1024, 1, 2**24, 2**24, 1024, 1, None, None, 1e-5, 0, fake, 1024, fake, 0,
                          None) == -1


def test_tile_and_split_tables_are_pure_functions():
    L = _hip.lib()
    for (m, n, k) in [(128, 4096, 1024), (1000, 3072, 1024), (1, 2560, 640), (16, 1024, 4096)]:
        t1, t2 = L.kea_lowbit_gemm_tile(1, 1, m, n, k), L.kea_lowbit_gemm_tile(1, 1, m, n, k)
        assert t1 == t2 and 1 <= t1 <= L.kea_config_count()
        s = L.kea_lowbit_gemm_split(1, 1, m, n, k, 0, 0)
        assert s >= 1
        ws = L.kea_lowbit_gemm_workspace(1, 1, m, n, k, 0, 0, 0)
        assert ws == (s * m * n * 4 if s > 1 else 0)


def test_every_tile_table_entry_is_the_chooser_pick_and_resolves():
    """Each entry of the measured tile table (csrc/kea_gemm_table.h) is what the chooser returns at that swept shape,
    and the library resolves it there (registers, LDS and K range fit; no silent fall-back to another tile)."""
    L = _hip.lib()
    text = (Path(__file__).resolve().parents[1] / "kea-kernels_amd" / "csrc" / "kea_gemm_table.h").read_text()
    entries = [tuple(int(v) for v in e) for e in re.findall(r"\{(\d+), (\d+), (\d+), (\d+), (\d+), (\d+)\},", text)]
    assert len(entries) >= 300
    for wbits, parts, n, k, m, tile in entries:
        assert 1 <= tile <= L.kea_config_count()
        assert L.kea_lowbit_gemm_tile(wbits, parts, m, n, k) == tile, (wbits, parts, n, k, m, tile)
        assert L.kea_lowbit_gemm_workspace(wbits, parts, m, n, k, 0, 0, tile) >= 0, _hip.last_error()


def test_plan_refuses_what_the_direct_call_refuses():
    """kea_lowbit_gemm_plan returns NULL (with the same message) on arguments kea_lowbit_gemm refuses; nothing is
    launched and no device is touched."""
    L = _hip.lib()
    h = L.kea_lowbit_gemm_plan(3, None, 0, 16, 1, None, 0, 1, None, 64, 64, None, 0, 0, None, 0, None, 0, 64, None,
                               0, 1, 0, 0, 0, None, 0, None, 0, 1.0)
    assert not h and b"wbits" in L.kea_last_error()
    h = L.kea_lowbit_gemm_plan(1, ctypes.c_void_p(8), 0, 64, 1, ctypes.c_void_p(16), 0, 1, ctypes.c_void_p(16), 64,
                               64, ctypes.c_void_p(16), 0, 0, None, 0, ctypes.c_void_p(16), 0, 64, None, 0, 1, 0, 0,
                               0, None, 0, None, 0, 1.0)
    assert not h and b"aligned" in L.kea_last_error()
    assert L.kea_lowbit_gemm_plan_launch(None, None) == -1
    L.kea_lowbit_gemm_plan_free(None)


def test_plan_launch_with_refuses_mismatched_buffers_before_any_launch():
    """kea_lowbit_gemm_plan_launch_with binds new buffers to a plan: NULL plan, an unaligned or missing q, a missing
    qs, buffers present where the plan has none (or absent where it has one) and a short split-K workspace are all
    refused on the host; no device is touched (fake addresses)."""
    L = _hip.lib()
    P = ctypes.c_void_p

    def plan(acc=None, split=1):
        return L.kea_lowbit_gemm_plan(1, P(0x1000), 64 * 1024, 1024, 1, P(0x2000), 0, 64, P(0x3000), 256, 1024,
                                      P(0x4000), 0, 0, None, 0, P(0x10000), 0, 256, acc, 256 if acc else 0, 64, 0,
                                      split, 0, P(0x100000) if split > 1 else None, 1 << 20 if split > 1 else 0,
                                      None, 0, 1.0)

    h = plan()
    assert h, L.kea_last_error()
    try:
        assert L.kea_lowbit_gemm_plan_workspace(h) == 0
        call = L.kea_lowbit_gemm_plan_launch_with
        assert call(None, P(0x1000), P(0x2000), P(0x10000), None, None, None, 0, None) == -1
        assert call(h, P(0x1008), P(0x2000), P(0x10000), None, None, None, 0, None) == -2
        assert call(h, P(0x1000), P(0x2002), P(0x10000), None, None, None, 0, None) == -2  # f32 qs off its alignment
        assert call(h, None, P(0x2000), P(0x10000), None, None, None, 0, None) == -2
        assert call(h, P(0x1000), None, P(0x10000), None, None, None, 0, None) == -1
        assert call(h, P(0x1000), P(0x2000), None, None, None, None, 0, None) == -1
        assert b"exactly where the plan has them" in L.kea_last_error()
        assert call(h, P(0x1000), P(0x2000), P(0x10000), P(0x20000), None, None, 0, None) == -1
        assert call(h, P(0x1000), P(0x2000), P(0x10000), None, P(0x30000), None, 0, None) == -1
    finally:
        L.kea_lowbit_gemm_plan_free(h)
    hs = plan(split=4)  # a split K needs a workspace per launch: slices [S][P][M][N] int32
    assert hs, L.kea_last_error()
    if hs:
        try:
            need = L.kea_lowbit_gemm_plan_workspace(hs)
            assert need > 0 and need % (1 * 64 * 256 * 4) == 0
            assert L.kea_lowbit_gemm_plan_launch_with(hs, P(0x1000), P(0x2000), P(0x10000), None, None, None, 0,
                                                      None) == -4
            assert L.kea_lowbit_gemm_plan_launch_with(hs, P(0x1000), P(0x2000), P(0x10000), None, None, P(0x100008),
                                                      need, None) == -2
        finally:
            L.kea_lowbit_gemm_plan_free(hs)


def test_project_plan_refuses_what_the_two_calls_refuse_and_sizes_its_workspace():
    """kea_lowbit_project_plan takes a GEMM plan made on the quantizer's layout (y only; part_stride = m * ldq,
    qs_stride = m) plus kea_quantize's arguments, and refuses what either would; its workspace holds the int8 parts,
    then their scales, then any split-K slices, each 16-byte aligned. kea_lowbit_project_launch refuses a NULL plan,
    missing x or y and a missing, short or unaligned workspace on the host (fake addresses: no device is touched)."""
    L = _hip.lib()
    P = ctypes.c_void_p

    def plan(acc=None, split=1, part_stride=64 * 1024, qs_stride=64):
        return L.kea_lowbit_gemm_plan(1, P(0x1000), part_stride, 1024, 1, P(0x2000), 0, qs_stride, P(0x3000), 256,
                                      1024, P(0x4000), 0, 0, None, 0, P(0x10000), 0, 256, acc, 256 if acc else 0, 64,
                                      0, split, 0, P(0x100000) if split > 1 else None, 1 << 20 if split > 1 else 0,
                                      None, 0, 1.0)

    def project(h, x_dtype=0, t=64, nw=None, nb=None):
        return L.kea_lowbit_project_plan(h, x_dtype, 0, 1024, 1, t, nw, nb, 1e-5, 0)

    assert not project(None) and b"plan is NULL" in L.kea_last_error()
    for kwargs, message in (({"acc": P(0x20000)}, b"writes y only"), ({"part_stride": 65 * 1024}, b"part_stride"),
                            ({"qs_stride": 128}, b"qs_stride")):
        h = plan(**kwargs)
        assert h, L.kea_last_error()
        try:
            assert not project(h) and message in L.kea_last_error()
        finally:
            L.kea_lowbit_gemm_plan_free(h)
    h = plan()
    try:
        assert not project(h, x_dtype=2) and b"x dtype" in L.kea_last_error()
        assert not project(h, t=0) and b"t must be" in L.kea_last_error()
        assert not project(h, nw=P(0x5000)) and b"go together" in L.kea_last_error()
        pp = project(h)
        assert pp, L.kea_last_error()
    finally:
        L.kea_lowbit_gemm_plan_free(h)  # the projection plan holds its own copy
    try:
        need = L.kea_lowbit_project_workspace(pp)
        assert need == 64 * 1024 + 64 * 4
        call = L.kea_lowbit_project_launch
        assert call(None, P(0x8000), P(0x10000), P(0x100000), need, None) == -1
        assert call(pp, None, P(0x10000), P(0x100000), need, None) == -1
        assert call(pp, P(0x8000), None, P(0x100000), need, None) == -1
        assert call(pp, P(0x8000), P(0x10000), None, need, None) == -4
        assert call(pp, P(0x8000), P(0x10000), P(0x100000), need - 1, None) == -4
        assert call(pp, P(0x8000), P(0x10000), P(0x100008), need, None) == -2
    finally:
        L.kea_lowbit_project_plan_free(pp)
    hs = plan(split=4)
    assert hs, L.kea_last_error()
    try:
        pp = project(hs)
        assert pp, L.kea_last_error()
        assert L.kea_lowbit_project_workspace(pp) == 64 * 1024 + 64 * 4 + L.kea_lowbit_gemm_plan_workspace(hs)
        L.kea_lowbit_project_plan_free(pp)
    finally:
        L.kea_lowbit_gemm_plan_free(hs)
    L.kea_lowbit_project_plan_free(None)
