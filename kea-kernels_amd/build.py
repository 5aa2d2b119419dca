"""Build libkea_hip.so (the gfx950 kernels and the C ABI of include/kea_lowbit.h and include/kea_encoder.h) and the
benchmark's probe library libkea_probe.so (include/kea_probe.h) in-tree with hipcc.

    python kea-kernels_amd/build.py [-j JOBS] [--max-stages N]

Objects go to kea-kernels_amd/_build/, the product library to kea-kernels_amd/kea_kernels/lib/libkea_hip.so and the
probe library, which nothing in the package loads, to kea-kernels_amd/kea_probes/lib/libkea_probe.so.
--max-stages N rebuilds every translation unit with another LDS-ring depth cap for the ring kernel (default 2; a
measurement knob: the host's LDS sizing and the kernels must agree, so it is never set per file).
Every source is compiled for gfx950 only; device FP contraction is off (the epilogue's FP32 op order is part
of the contract) and packed-FP32 instruction selection is disabled.
"""
from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "kea_kernels" / "lib" / "libkea_hip.so"
PROBE_DIR = HERE / "kea_probes"
PROBE_LIB = PROBE_DIR / "lib" / "libkea_probe.so"
PROBE_SOURCES = ["kea_probe.hip"]
SOURCES = ["kea_gemm_ring_w1.hip", "kea_gemm_ring_w2.hip", "kea_gemm_wsplit_p1.hip", "kea_gemm_wsplit_p2.hip",
           "kea_gemm_wsplit_p3.hip", "kea_gemm_wsplit_g1.hip", "kea_gemm_wsplit_g2.hip", "kea_gemm_wsplit_g3.hip",
           "kea_gemm.hip", "kea_gemm_wsplit.hip", "kea_quantize.hip", "kea_encoder.hip",
           "kea_layout.cpp"]
ARCH = "gfx950"
# Per-source flags. The probe's loop keeps eight MFMA accumulators live across iterations; in the accumulator
# (AGPR) form the register allocator shuffles them with accvgpr moves every iteration, which would be measured as
# matrix-core time, so it selects the VGPR form of the MFMAs.
SOURCE_FLAGS = {"kea_probe.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}
# The wave-split kernels take their load operands as ten leading scalar arguments (4 pointers, 6 ints: 14 SGPRs) that
# the dispatch preloads into SGPRs, so the first loads issue without a kernel-argument round trip.
for _p in (1, 2, 3):
    SOURCE_FLAGS[f"kea_gemm_wsplit_p{_p}.hip"] = ["-mllvm", "-amdgpu-kernarg-preload-count=10"]
    SOURCE_FLAGS[f"kea_gemm_wsplit_g{_p}.hip"] = ["-mllvm", "-amdgpu-kernarg-preload-count=10"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libkea_hip.so)")


EXTRA_DEFINES: list[str] = []


def flags() -> list[str]:
    return [*EXTRA_DEFINES, "-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall", "-Wno-unused-function",
            f"-I{HERE.parent / 'include'}"]


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *flags(), *SOURCE_FLAGS.get(src.name, [])]
    if src.suffix == ".cpp":
        cmd += ["-x", "c++"]  # host-only translation unit
    cmd += ["-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in res.stderr.splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def _link(objs: list[Path], lib: Path) -> None:
    lib.parent.mkdir(parents=True, exist_ok=True)
    tmp = lib.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stderr}")
    os.replace(tmp, lib)


def build(jobs: int | None = None) -> Path:
    """Compiles every translation unit of both libraries (in parallel) and links them; returns the product library."""
    BUILD.mkdir(exist_ok=True)
    units = [(CSRC / s, BUILD / (Path(s).stem + ".o")) for s in SOURCES]
    probe_units = [(PROBE_DIR / s, BUILD / (Path(s).stem + ".o")) for s in PROBE_SOURCES]
    jobs = jobs or min(len(units) + len(probe_units), os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        futures = [pool.submit(_compile, src, obj) for src, obj in units + probe_units]
        for f in futures:
            f.result()
    _link([obj for _, obj in units], LIB)
    _link([obj for _, obj in probe_units], PROBE_LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("-j", "--jobs", type=int, default=None)
    ap.add_argument("--max-stages", type=int, default=None, help="ring depth cap (2..8)")
    args = ap.parse_args()
    if args.max_stages is not None:
        if not 2 <= args.max_stages <= 8:
            ap.error("--max-stages must be 2..8")
        EXTRA_DEFINES.append(f"-DKEA_MAX_STAGES={args.max_stages}")
    print(build(args.jobs))
