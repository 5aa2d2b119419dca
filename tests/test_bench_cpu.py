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


def test_suite_covers_configs_2_to_4():
    """The headline line's `suite`: config 2 per-channel and group-128, config 3's six encoder linears at M = 1000,
    config 4's 640 -> 2560 / 640 -> 1030 at M in {1, 4, 16} and 4096 -> 1024 at M = 16, both weight widths, hot and
    cold, all at BASELINE.json's sizes."""
    names = {bench._case_name(name, cold) for name, *_, cold in bench.BASELINE_CASES}
    assert len(names) == len(bench.BASELINE_CASES) == 2 + 6 + 2 * (2 * 3 * 2 + 2)
    shapes = {(w, m, n, k, g) for _, w, m, n, k, g, _ in bench.BASELINE_CASES}
    assert {(2, 128, 1024, 4096, 0), (2, 128, 1024, 4096, 128)} <= shapes
    assert {(1, 1000, n, k, 0) for n, k in [(3072, 1024), (1024, 1024), (4096, 1024), (1024, 4096),
                                            (2048, 1024)]} <= shapes
    for w in (1, 2):
        assert {(w, m, n, 640, 0) for m in (1, 4, 16) for n in (2560, 1030)} <= shapes
        assert (w, 16, 1024, 4096, 0) in shapes
    assert sum(1 for *_, cold in bench.BASELINE_CASES if cold) == 2 * (3 * 2 + 1)


def test_trace_summary_reads_queued_regions(tmp_path):
    """Each run of one kernel behind a spin kernel gives (last end - first start) / dispatches beside the mean
    traced duration: overlapping traced durations (longer than the cadence) do not inflate the per-dispatch time."""
    header = '"Kind","Dispatch_Id","Kernel_Name","Start_Timestamp","End_Timestamp"\n'
    rows = [("(anonymous namespace)::spin_kernel(unsigned long long)", 0, 1000)]
    rows += [("gemm(int)", 1000 + 100 * i, 1000 + 100 * i + 150) for i in range(10)]   # 150 ns each, 100 ns apart
    rows += [("other(int)", 5000, 5010), ("spin_kernel(unsigned long long)", 6000, 7000)]
    rows += [("gemm(int)", 7000 + 200 * i, 7000 + 200 * i + 200) for i in range(4)]
    body = "".join(f'"KERNEL_DISPATCH",{i},"{n}",{a},{b}\n' for i, (n, a, b) in enumerate(rows))
    path = tmp_path / "t_kernel_trace.csv"
    path.write_text(header + body)
    out = bench.trace_summary(str(path))
    first, second = out["regions"]
    assert first["kernel"] == "gemm" and first["dispatches"] == 10
    assert first["span_us_per_dispatch"] == round((900 + 150) / 10 / 1e3, 4)
    assert first["mean_duration_us"] == 0.15 and first["median_gap_us"] == -0.05
    assert second["dispatches"] == 4 and second["span_us_per_dispatch"] == 0.2
