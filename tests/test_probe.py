"""The benchmark's probe library (libkea_probe.so, include/kea_probe.h): argument checks on the CPU; on the GPU its checksum against a numpy
emulation of v_mfma_i32_16x16x64_i8, which also pins the operand layout the GEMM relies on (source A lane l: row
l % 16, k = 16 * (l // 16) + byte; source B lane l: column l % 16, same k; result lane l: rows 4 * (l // 16) + r of
column l % 16)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import kea_probes


def test_probe_arguments():
    L = kea_probes.lib()
    assert L.kea_probe_mfma_i8_ops(2048, 2000) == 2048 * 4 * 2000 * 8 * 16 * 16 * 64 * 2
    assert L.kea_probe_mfma_i8_ops(0, 10) == 0 and L.kea_probe_mfma_i8_ops(1, 0) == 0
    assert L.kea_probe_mfma_i8(0, 10, None, None) == -1
    assert b"blocks" in L.kea_probe_last_error()
    assert L.kea_probe_mfma_i8(1, 1, None, None) == -1


def test_floor_and_spin_probe_arguments():
    """The launch-floor and spin probes refuse bad arguments before any launch (no GPU is touched)."""
    L = kea_probes.lib()
    vp = ctypes.c_void_p
    assert L.kea_probe_floor(4, 128, 4096, 1024, 32, 32, None, None, None, 4096, None) == -1
    assert b"kind" in L.kea_probe_last_error()
    assert L.kea_probe_floor(0, 128, 4096, 1024, 24, 32, None, None, None, 4096, None) == -1   # bm % 16
    assert L.kea_probe_floor(0, 100, 4096, 1024, 32, 32, None, None, None, 4096, None) == -1   # m % bm
    assert L.kea_probe_floor(0, 128, 4096, 1000, 32, 32, None, None, None, 4096, None) == -1   # k % 128
    assert L.kea_probe_floor(1, 128, 4096, 1024, 32, 32, None, None, None, 4096, None) == -1   # loads need a, w
    assert L.kea_probe_floor(2, 128, 4096, 1024, 32, 32, None, None, None, 4096, None) == -1   # stores need y
    assert L.kea_probe_floor(2, 128, 4096, 1024, 32, 32, None, None, vp(16), 4000, None) == -1  # ldy < n
    assert L.kea_probe_floor(1, 256, 256, 65536, 256, 256, vp(16), vp(16), None, 256, None) == -1  # LDS
    assert b"LDS" in L.kea_probe_last_error()
    assert L.kea_probe_spin(-1, None) == -1 and L.kea_probe_spin(100000001, None) == -1
    assert L.kea_probe_floor_waves(0, 128, 4096, 1024, 32, 32, 0, None, None, None, 4096, None) == -1  # waves
    assert L.kea_probe_floor_waves(0, 128, 4096, 1024, 32, 32, 17, None, None, None, 4096, None) == -1
    assert b"waves" in L.kea_probe_last_error()


def test_operand_and_exchange_probe_arguments():
    """The operand-fed MFMA loop and the exchange probe refuse bad arguments before any launch."""
    L = kea_probes.lib()
    vp = ctypes.c_void_p
    assert L.kea_probe_mfma_i8_operands(1, 1, vp(8), vp(16), None) == -2       # operands not 16-byte aligned
    assert b"operands" in L.kea_probe_last_error()
    assert L.kea_probe_mfma_i8_operands(0, 1, None, vp(16), None) == -1        # blocks
    assert L.kea_probe_exchange(3, 64, 64, 4, vp(16), vp(16), vp(16), None) == -1  # kind
    assert b"kind" in L.kea_probe_last_error()
    assert L.kea_probe_exchange(0, 0, 64, 1, vp(16), None, None, None) == -1      # workgroups
    assert L.kea_probe_exchange(0, 64, 64, 65, vp(16), None, None, None) == -1    # group > workgroups
    assert L.kea_probe_exchange(0, 64, 64, 4, vp(8), None, None, None) == -2      # slots alignment
    assert L.kea_probe_exchange(1, 64, 64, 4, vp(16), None, None, None) == -1     # counting needs counters
    assert L.kea_probe_exchange(2, 64, 64, 4, vp(16), vp(16), None, None) == -1   # fenced needs a result


def _operand_bytes(words):
    """[64 lanes, 4 int32] -> [64, 16] bytes, little-endian."""
    return np.asarray(words, dtype=np.int64).astype(np.uint32).view(np.uint8).reshape(64, 16)


def _pattern_words():
    lane = np.arange(64, dtype=np.int64)
    a = np.stack([0x01020304 + lane, 0x05060708 - lane, 0x090A0B0C ^ lane, 0x0D0E0F10 + 3 * lane], 1)
    b = np.stack([0x11121314 - lane, 0x15161718 + lane, 0x191A1B1C ^ (lane << 8), 0x1D1E1F20 + 5 * lane], 1)
    return a, b


def expected_checksums(iters: int, words=None) -> np.ndarray:
    """Per-lane checksums of the probe: words = (a, b), each [64][4] int32 operand words (default: the pattern)."""
    aw, bw = words if words is not None else _pattern_words()
    a, b = _operand_bytes(aw), _operand_bytes(bw)
    A = np.zeros((16, 64), np.int64)
    B = np.zeros((64, 16), np.int64)
    for l in range(64):
        A[l % 16, 16 * (l // 16):16 * (l // 16) + 16] = a[l].view(np.int8)
        B[16 * (l // 16):16 * (l // 16) + 16, l % 16] = b[l].view(np.int8)
    D = A @ B
    sums = np.zeros(64, np.int64)
    for l in range(64):
        rows = D[4 * (l // 16):4 * (l // 16) + 4, l % 16]
        for c in range(8):  # chain c starts at {c, 0, 0, 0}; each MFMA adds D (int32 wrap)
            acc = (np.array([c, 0, 0, 0], np.int64) + iters * rows) % (1 << 32)
            sums[l] += acc.sum()
    return (sums % (1 << 32)).astype(np.uint32).view(np.int32)


@pytest.mark.gpu
def test_probe_checksum_matches_the_mfma_emulation():
    L = kea_probes.lib()
    dev = torch.device("cuda", 0)
    blocks, iters = 3, 5
    out = torch.full((blocks * 256,), -1, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    rc = L.kea_probe_mfma_i8(blocks, iters, ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(stream.cuda_stream))
    assert rc == 0, L.kea_probe_last_error()
    torch.cuda.synchronize()
    want = np.tile(expected_checksums(iters), blocks * 4)
    assert np.array_equal(out.cpu().numpy(), want)


@pytest.mark.gpu
def test_operand_fed_probe_checksum_on_random_operands():
    L = kea_probes.lib()
    dev = torch.device("cuda", 0)
    g = np.random.default_rng(7)
    words = g.integers(-2 ** 31, 2 ** 31, size=(128, 4), dtype=np.int64).astype(np.int32)
    ops = torch.from_numpy(words).to(dev)
    blocks, iters = 2, 7
    out = torch.full((blocks * 256,), -1, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    rc = L.kea_probe_mfma_i8_operands(blocks, iters, ctypes.c_void_p(ops.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                                      ctypes.c_void_p(stream.cuda_stream))
    assert rc == 0, L.kea_probe_last_error()
    torch.cuda.synchronize()
    want = np.tile(expected_checksums(iters, (words[:64], words[64:])), blocks * 4)
    assert np.array_equal(out.cpu().numpy(), want)


@pytest.mark.gpu
@pytest.mark.parametrize("workgroups,words,group", [(64, 64, 4), (300, 1024, 300), (257, 16, 5)])
def test_exchange_probe_fenced_sum_and_counters(workgroups, words, group):
    """The fenced exchange's last arrivers read every member's slot: after two launches the sum is twice
    0 + 1 + ... + (workgroups - 1), and every group counter is back at zero."""
    L = kea_probes.lib()
    dev = torch.device("cuda", 0)
    slots = torch.zeros(workgroups * words * 4, dtype=torch.int32, device=dev)
    counters = torch.zeros(-(-workgroups // group), dtype=torch.int32, device=dev)
    result = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    vp = ctypes.c_void_p
    for kind in (1, 2, 2):
        rc = L.kea_probe_exchange(kind, workgroups, words, group, vp(slots.data_ptr()), vp(counters.data_ptr()),
                                  vp(result.data_ptr()), vp(stream.cuda_stream))
        assert rc == 0, L.kea_probe_last_error()
    torch.cuda.synchronize()
    assert int(result.item()) & 0xFFFFFFFF == (workgroups * (workgroups - 1)) & 0xFFFFFFFF
    assert not counters.any()
    last = slots.view(workgroups, words, 4)[:, -1].cpu().numpy()
    assert np.array_equal(last[:, 0], np.arange(workgroups)) and np.array_equal(last[:, 1], np.full(workgroups, words - 1))
