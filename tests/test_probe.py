"""The measured-peak probe (include/kea_probe.h): argument checks on the CPU; on the GPU its checksum against a numpy
emulation of v_mfma_i32_16x16x64_i8, which also pins the operand layout the GEMM relies on (source A lane l: row
l % 16, k = 16 * (l // 16) + byte; source B lane l: column l % 16, same k; result lane l: rows 4 * (l // 16) + r of
column l % 16)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from kea_kernels import _hip


def test_probe_arguments():
    L = _hip.lib()
    assert L.kea_probe_mfma_i8_ops(2048, 2000) == 2048 * 4 * 2000 * 8 * 16 * 16 * 64 * 2
    assert L.kea_probe_mfma_i8_ops(0, 10) == 0 and L.kea_probe_mfma_i8_ops(1, 0) == 0
    assert L.kea_probe_mfma_i8(0, 10, None, None) == -1
    assert b"blocks" in L.kea_last_error()
    assert L.kea_probe_mfma_i8(1, 1, None, None) == -1


def test_floor_and_spin_probe_arguments():
    """The launch-floor and spin probes refuse bad arguments before any launch (no GPU is touched)."""
    L = _hip.lib()
    vp = ctypes.c_void_p
    assert L.kea_probe_floor(4, 128, 4096, 1024, 32, 32, None, None, None, 4096, None) == -1
    assert b"kind" in L.kea_last_error()
    assert L.kea_probe_floor(0, 128, 4096, 1024, 24, 32, None, None, None, 4096, None) == -1   # bm % 16
    assert L.kea_probe_floor(0, 100, 4096, 1024, 32, 32, None, None, None, 4096, None) == -1   # m % bm
    assert L.kea_probe_floor(0, 128, 4096, 1000, 32, 32, None, None, None, 4096, None) == -1   # k % 128
    assert L.kea_probe_floor(1, 128, 4096, 1024, 32, 32, None, None, None, 4096, None) == -1   # loads need a, w
    assert L.kea_probe_floor(2, 128, 4096, 1024, 32, 32, None, None, None, 4096, None) == -1   # stores need y
    assert L.kea_probe_floor(2, 128, 4096, 1024, 32, 32, None, None, vp(16), 4000, None) == -1  # ldy < n
    assert L.kea_probe_floor(1, 256, 256, 65536, 256, 256, vp(16), vp(16), None, 256, None) == -1  # LDS
    assert b"LDS" in L.kea_last_error()
    assert L.kea_probe_spin(-1, None) == -1 and L.kea_probe_spin(100000001, None) == -1


def _operand_bytes(words):
    """[64 lanes, 4 int32] -> [64, 16] bytes, little-endian."""
    return np.asarray(words, dtype=np.int64).astype(np.uint32).view(np.uint8).reshape(64, 16)


def expected_checksums(iters: int) -> np.ndarray:
    lane = np.arange(64, dtype=np.int64)
    a = _operand_bytes(np.stack([0x01020304 + lane, 0x05060708 - lane, 0x090A0B0C ^ lane, 0x0D0E0F10 + 3 * lane], 1))
    b = _operand_bytes(np.stack([0x11121314 - lane, 0x15161718 + lane, 0x191A1B1C ^ (lane << 8),
                                 0x1D1E1F20 + 5 * lane], 1))
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
    L = _hip.lib()
    dev = torch.device("cuda", 0)
    blocks, iters = 3, 5
    out = torch.full((blocks * 256,), -1, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    rc = L.kea_probe_mfma_i8(blocks, iters, ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(stream.cuda_stream))
    assert rc == 0, L.kea_last_error()
    torch.cuda.synchronize()
    want = np.tile(expected_checksums(iters), blocks * 4)
    assert np.array_equal(out.cpu().numpy(), want)
