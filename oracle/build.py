"""Build the CPU oracle (oracle/kea_oracle.c -> oracle/lib/libkea_oracle.so) with gcc. TEST INFRASTRUCTURE ONLY.

The reference keeps its kernels as CUDA C++ strings compiled by NVRTC for SM120 plus Triton JIT code
(kk/binary/kernels.py, kk/ternary/*.py); none of it can be built in this image, so there is no oracle/_ref build.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB = HERE / "lib" / "libkea_oracle.so"


def build() -> Path:
    cc = os.environ.get("CC") or shutil.which("gcc") or "cc"
    LIB.parent.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, "-O3", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-fopenmp",
           "-fvisibility=hidden", "-Wall", "-o", str(tmp), str(HERE / "kea_oracle.c"), "-lm"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed: {' '.join(cmd)}\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
