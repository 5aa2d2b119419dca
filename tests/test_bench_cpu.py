"""The bench.py contract pieces that run without a GPU: the single-GPU refusal, argument checks, the roofline
accounting constants of config 1 and the traffic figure read from the committed profile."""
from __future__ import annotations

import json
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def _run(*args, env=None):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=300, env=env)


def test_more_than_one_gpu_is_refused():
    p = _run("--gpus", "2", "--no-cpu", "--no-encoder", "--no-peaks")
    assert p.returncode == 2 and "one GPU only" in p.stderr and p.stdout == ""
    env = dict(os.environ, WORLD_SIZE="4")
    p = _run("--no-cpu", "--no-encoder", "--no-peaks", env=env)
    assert p.returncode == 2 and "one GPU only" in p.stderr


def test_steps_must_be_positive():
    p = _run("--steps", "0", "--no-cpu", "--no-encoder", "--no-peaks")
    assert p.returncode == 2 and "--steps" in p.stderr


def test_config1_accounting():
    """2*M*N*K int8 ops and the algorithmic bytes of config 1 (A + 1-bit W + fp16 alpha + fp16 row scales + fp16 Y),
    which put it on the MFMA / HBM ridge (0.215 vs 0.214 us)."""
    assert (bench.M, bench.N, bench.K) == (128, 4096, 1024)
    assert bench.OPS == 1_073_741_824
    assert bench.BYTES == 128 * 1024 + 4096 * 1024 // 8 + 2 * 4096 + 2 * 128 + 2 * 128 * 4096 == 1_712_384
    t_mfma = bench.OPS / (bench.PEAK_INT8_TOPS * 1e12)
    t_hbm = bench.BYTES / (bench.PEAK_HBM_GBS * 1e9)
    assert abs(t_mfma - 0.2147e-6) < 1e-9 and abs(t_hbm - 0.2140e-6) < 1e-9 and t_mfma >= t_hbm


def test_traffic_comes_from_the_committed_profile():
    data = json.loads((ROOT / "profiles" / "b1_gemm_config1_traffic.json").read_text())
    assert bench.traffic_from_profiles() == (data["hbm_bytes_per_launch"], data.get("kernel_sources_sha"))
    assert data["hbm_bytes_per_launch"] == data["fetch_bytes_per_launch"] + data["write_bytes_per_launch"]
    assert data["algorithmic_bytes_per_launch"] == bench.BYTES


def test_kernel_source_hash_names_the_build():
    """The hash a traffic profile is labeled with covers every kernel source and nothing else."""
    h = bench.kernel_sources_sha()
    assert len(h) == 16 and h == bench.kernel_sources_sha()
    int(h, 16)
