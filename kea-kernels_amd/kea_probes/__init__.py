"""ctypes binding of libkea_probe.so, the benchmark's measurement library (include/kea_probe.h).

The probes are kept out of the product library libkea_hip.so: bench.py and the tests load them from here. They measure
what the MI355X sustains (the int8 MFMA loop), what a GEMM-shaped grid costs before it computes anything (launch
floors), what a cross-workgroup exchange costs, and keep host submission out of timed regions (a bounded spin). Status
codes as the product library's: negative = a contract violation (ValueError), positive = a hipError_t (RuntimeError).
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libkea_probe.so"

_i32, _i64, _vp, _cp = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_char_p

SIGNATURES = {
    "kea_probe_mfma_i8": (_i32, [_i64, _i64, _vp, _vp]),
    "kea_probe_mfma_i8_ops": (_i64, [_i64, _i64]),
    "kea_probe_mfma_i8_operands": (_i32, [_i64, _i64, _vp, _vp, _vp]),
    "kea_probe_mfma_i8_32": (_i32, [_i64, _i64, _vp, _vp, _vp]),
    "kea_probe_mfma_i8_32_ops": (_i64, [_i64, _i64]),
    "kea_probe_exchange": (_i32, [_i32, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "kea_probe_floor": (_i32, [_i32, _i64, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _i64, _vp]),
    "kea_probe_floor_waves": (_i32, [_i32, _i64, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _i64, _vp]),
    "kea_probe_spin": (_i32, [_i64, _vp]),
    "kea_probe_last_error": (_cp, []),
}

_lock = threading.Lock()
_lib = None


def lib() -> ctypes.CDLL:
    """The loaded probe library (RuntimeError if it was not built)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.is_file():
                    raise RuntimeError(f"{LIB_PATH} is missing: build it with `python kea-kernels_amd/build.py`")
                handle = ctypes.CDLL(str(LIB_PATH))
                for name, (restype, argtypes) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype, fn.argtypes = restype, argtypes
                _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc == 0:
        return
    message = f"{what}: {lib().kea_probe_last_error().decode(errors='replace')}"
    if rc < 0:
        raise ValueError(message)
    raise RuntimeError(f"{message} (hipError {rc})")
