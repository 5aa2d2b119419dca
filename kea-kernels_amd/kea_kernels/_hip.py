"""ctypes binding of libkea_hip.so (the C ABI of include/kea_lowbit.h).

This replaces the reference's NVRTC loader and launcher (kk/_nvrtc.py): every kernel is compiled ahead of time
for gfx950 by kea-kernels_amd/build.py, so there is no runtime compilation, no kernel cache and nothing to refuse
during graph capture. Calls are enqueued on torch's current stream (`torch.cuda.current_stream().cuda_stream` is
the hipStream_t on ROCm), never synchronize, and allocate nothing.

Error mapping (as the reference's): a negative status (contract violation, nothing launched) raises ValueError, a
positive one (the HIP runtime refused a launch) raises RuntimeError (kk/_nvrtc.py:123-124). The library missing is
a RuntimeError: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libkea_hip.so"

F32, F16, BF16 = 0, 1, 2
FLAG_SILU, FLAG_ORDER = 1, 2
DTYPES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

# (name, restype, argtypes) of every exported function
_i32, _i64, _vp, _f32, _cp = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_float, ctypes.c_char_p

SIGNATURES = {
    "kea_b1_native_words": (_i64, [_i64, _i64]),
    "kea_t2_native_words": (_i64, [_i64, _i64]),
    "kea_b1_relayout_host": (_i32, [_vp, _i64, _i64, _vp]),
    "kea_t2_relayout_host": (_i32, [_vp, _i64, _i64, _vp]),
    "kea_b1_unlayout_host": (_i32, [_vp, _i64, _i64, _vp]),
    "kea_t2_unlayout_host": (_i32, [_vp, _i64, _i64, _vp]),
    "kea_lowbit_gemm": (_i32, [_i32, _vp, _i64, _i64, _i32, _vp, _i32, _i64, _vp, _i64, _i64, _vp, _i32, _i64,
                               _vp, _i32, _vp, _i32, _i64, _vp, _i64, _i64, _i32, _i32, _i32, _vp, _i64, _vp]),
    "kea_lowbit_gemm_plan": (_vp, [_i32, _vp, _i64, _i64, _i32, _vp, _i32, _i64, _vp, _i64, _i64, _vp, _i32, _i64,
                                    _vp, _i32, _vp, _i32, _i64, _vp, _i64, _i64, _i32, _i32, _i32, _vp, _i64, _vp,
                                    _i64, _f32]),
    "kea_lowbit_gemm_plan_launch": (_i32, [_vp, _vp]),
    "kea_lowbit_gemm_plan_launch_with": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp]),
    "kea_lowbit_gemm_plan_workspace": (_i64, [_vp]),
    "kea_lowbit_gemm_plan_free": (None, [_vp]),
    "kea_lowbit_project_plan": (_vp, [_vp, _i32, _i64, _i64, _i64, _i64, _vp, _vp, _f32, _i32]),
    "kea_lowbit_project_workspace": (_i64, [_vp]),
    "kea_lowbit_project_launch": (_i32, [_vp, _vp, _vp, _vp, _i64, _vp]),
    "kea_lowbit_project_plan_free": (None, [_vp]),
    "kea_lowbit_gemm_noalloc": (_i32, [_i32, _vp, _i64, _i64, _i32, _vp, _i32, _i64, _vp, _i64, _i64, _vp, _i32,
                                       _i64, _vp, _i32, _vp, _i32, _i64, _vp, _i64, _i64, _i32, _i32, _i32, _vp]),
    "kea_lowbit_gemm_residual": (_i32, [_i32, _vp, _i64, _i64, _i32, _vp, _i32, _i64, _vp, _i64, _i64, _vp, _i32,
                                        _i64, _vp, _i32, _vp, _i32, _i64, _vp, _i64, _i64, _i32, _i32, _i32, _vp,
                                        _i64, _vp, _i64, _f32, _vp]),
    "kea_lowbit_gemm_slices": (_i32, [_i32, _vp, _i64, _i64, _i32, _vp, _i64, _i64, _i64, _i32, _i32, _vp, _vp]),
    "kea_lowbit_slices_finish": (_i32, [_vp, _i32, _i32, _i64, _i64, _vp, _i32, _i64, _vp, _i32, _vp, _i32, _vp,
                                        _i32, _i64, _vp, _i64, _i32, _vp]),
    "kea_row_epilogue": (_i32, [_vp, _i32, _i32, _i64, _i64, _vp, _i64, _vp, _i32, _vp, _i32, _i32, _vp, _i64, _f32,
                                _vp, _vp, _f32, _vp, _i64, _vp, _vp, _f32, _i32, _vp, _i64, _vp, _vp]),
    "kea_lowbit_gemm_workspace": (_i64, [_i32, _i32, _i64, _i64, _i64, _i64, _i32, _i32]),
    "kea_lowbit_gemm_tile": (_i32, [_i32, _i32, _i64, _i64, _i64]),
    "kea_lowbit_gemm_split": (_i32, [_i32, _i32, _i64, _i64, _i64, _i64, _i32]),
    "kea_config_count": (_i32, []),
    "kea_config_name": (_cp, [_i32]),
    "kea_quantize": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _f32, _i32, _vp, _i64,
                            _vp, _i32, _vp]),
    "kea_relpos_attention": (_i32, [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _f32, _vp]),
    "kea_relpos_attention_workspace": (_i64, [_i64, _i64, _i32]),
    "kea_relpos_attention_ws": (_i32, [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _f32, _vp,
                                       _i64, _vp]),
    "kea_attention_merge_quantize": (_i32, [_vp, _i64, _i64, _i64, _i32, _i32, _vp, _i64, _vp, _vp]),
    "kea_glu_dwconv": (_i32, [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp]),
    "kea_norm_quantize": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _f32, _vp, _i64, _vp, _vp, _f32, _i32, _vp, _i64,
                                 _vp, _vp]),
    "kea_glu_dwconv_quantize": (_i32, [_vp, _i64, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _vp, _i64, _vp, _vp]),
    "kea_logmel_normalize": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _f32, _f32, _vp, _vp]),
    "kea_logmel_normalize_frames": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _f32, _f32, _vp, _vp]),
    "kea_stft_frames": (_i32, [_vp, _i64, _i64, _f32, _vp, _i64, _i64, _vp, _vp]),
    "kea_subsample_front": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _vp, _vp]),
    "kea_dwconv2d_s2": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "kea_bias_relu_flatten": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "kea_dwconv_quantize": (_i32, [_vp, _i64, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _vp, _i64, _vp, _vp]),
    "kea_last_error": (_cp, []),
    "kea_version": (_i32, []),
}

_lock = threading.Lock()
_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library (RuntimeError if it was not built)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.is_file():
                    raise RuntimeError(f"{LIB_PATH} is missing: build it with `python kea-kernels_amd/build.py` "
                                       "(the kernels have no CPU or eager fallback)")
                handle = ctypes.CDLL(str(LIB_PATH))
                for name, (restype, argtypes) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype, fn.argtypes = restype, argtypes
                _lib = handle
    return _lib


def last_error() -> str:
    return lib().kea_last_error().decode(errors="replace")


def check(rc: int, what: str) -> None:
    if rc == 0:
        return
    message = f"{what}: {last_error()}"
    if rc < 0:
        raise ValueError(message)
    raise RuntimeError(f"{message} (hipError {rc})")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """torch's current stream on `device`; ValueError for a device that is not a GPU (the kernels would read host
    pointers as device addresses). Read through torch's raw-stream accessor where it has one (a fraction of a
    microsecond; torch.cuda.current_stream(device) builds a Stream object and costs about 2 us per call)."""
    if device.type != "cuda":
        raise ValueError(f"the kernels run on the GPU: tensors on {device} cannot be launched on")
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def require_gfx950(device: torch.device) -> None:
    """ValueError unless `device` is a ROCm gfx950 GPU (the only target the kernels are built for)."""
    if device.type != "cuda":
        raise ValueError("the low-bit kernels run on ROCm GPUs only (device must be 'cuda' or 'cuda:N')")
    if not torch.cuda.is_available():
        raise ValueError("no GPU is available to PyTorch")
    if torch.version.hip is None:
        raise ValueError("this build targets AMD MI355X (gfx950) under ROCm; PyTorch is not a ROCm build")
    arch = torch.cuda.get_device_properties(device).gcnArchName.split(":")[0]
    if arch != "gfx950":
        raise ValueError(f"the kernels are built for gfx950 (MI355X); {device} is {arch}")
