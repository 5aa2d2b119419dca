"""Tensor-level launchers of the C ABI: the low-bit GEMM and the residual int8 quantizer.

`gemm` is the single launch path of every operator in this package (binary.layer, binary.layer_parts,
ternary.fused_kernels): it checks tensors, resolves the split-K workspace from torch's caching allocator (as the
reference does for its L2 workspace, kk/binary/layer.py:194-195) and enqueues kea_lowbit_gemm on the current stream.
`quantize` enqueues kea_quantize. None of them synchronizes the host.
"""
from __future__ import annotations

import ctypes
import functools

import torch
from torch import Tensor

from kea_kernels import _hip

_SCALE_DTYPES = (torch.float32, torch.float16)


def _on(device: torch.device, *tensors: Tensor | None) -> None:
    for t in tensors:
        if t is not None and t.device != device:
            raise ValueError(f"tensor on {t.device}, expected {device}")


@functools.lru_cache(maxsize=256)
def _native_words(wbits: int, n: int, k: int) -> int:
    L = _hip.lib()
    return (L.kea_b1_native_words if wbits == 1 else L.kea_t2_native_words)(n, k)


def _check_words(words: Tensor, n: int, k: int, wbits: int) -> None:
    """The kernels read the whole native layout of an n x k matrix: refuse a buffer that does not hold it."""
    if wbits not in (1, 2):
        raise ValueError(f"wbits must be 1 or 2, got {wbits}")
    need = _native_words(wbits, n, k)
    if need <= 0:
        raise ValueError(f"bad weight shape {n} x {k}")
    if not words.is_contiguous() or words.numel() * words.element_size() < 4 * need:
        raise ValueError(f"words must be a contiguous buffer of the {need} native words of a {n} x {k} "
                         f"{wbits}-bit matrix")


@functools.lru_cache(maxsize=1024)
def _workspace_bytes(wbits: int, parts: int, m: int, n: int, k: int, ws_group: int, split: int, tile: int) -> int:
    need = _hip.lib().kea_lowbit_gemm_workspace(wbits, parts, m, n, k, ws_group, split, tile)
    if need < 0:
        _hip.check(-1, "kea_lowbit_gemm_workspace")
    return need


def _gemm_args(wbits, q, qs, words, n, k, wscale, bias, y, acc_out, m, silu, order, config, ws_group, residual, glu):
    """Checks the arguments of a GEMM call and returns (C arguments up to the workspace, device, workspace)."""
    if q.dtype != torch.int8 or q.dim() != 3:
        raise ValueError(f"q must be int8 [P, M, ldq], got {q.dtype} {tuple(q.shape)}")
    parts, rows, ldq = q.shape
    m = rows if m is None else m
    if m > rows:
        raise ValueError(f"m = {m} exceeds the {rows} rows of q")
    if q.stride(2) != 1 or q.stride(1) != ldq:
        raise ValueError("q rows must be contiguous with row stride ldq")
    if qs.dim() != 2 or qs.shape[0] != parts or qs.shape[1] < m or qs.stride(1) != 1 or qs.dtype not in _SCALE_DTYPES:
        raise ValueError(f"qs must be f32/f16 [{parts}, >= {m}] with unit column stride")
    groups = -(-k // ws_group) if ws_group > 0 else 1
    if wscale.dtype not in _SCALE_DTYPES or not wscale.is_contiguous() or wscale.numel() < n * groups:
        raise ValueError(f"weight scales must be contiguous f32 or f16 [{n}]" +
                         (f" x {groups} groups" if ws_group > 0 else ""))
    if bias is not None and (bias.dtype not in _SCALE_DTYPES or not bias.is_contiguous() or bias.numel() != n):
        raise ValueError("bias must be contiguous f32 or f16 [N]")
    _check_words(words, n, k, wbits)
    if y is None and acc_out is None:
        raise ValueError("nothing to compute: y and acc_out are both None")
    ny = n // 2 if glu else n
    if y is not None and (y.dim() != 2 or y.shape[0] < m or y.shape[1] < ny or y.stride(1) != 1):
        raise ValueError(f"y must be a row-major [>= {m}, >= {ny}] view")
    if acc_out is not None and (acc_out.dtype != torch.int32 or acc_out.dim() != 3 or acc_out.shape[0] != parts
                                or acc_out.shape[1] != m or acc_out.shape[2] < n or acc_out.stride(2) != 1
                                or acc_out.stride(0) != m * acc_out.stride(1)):
        raise ValueError(f"acc_out must be int32 [{parts}, {m}, >= {n}] with dense part planes")
    if residual is not None and (y is None or residual.dtype != torch.float32 or residual.dim() != 2
                                 or residual.shape[0] < m or residual.shape[1] < n or residual.stride(1) != 1):
        raise ValueError(f"residual must be a row-major FP32 [>= {m}, >= {n}] view and needs y")
    if torch.is_grad_enabled() and (q.requires_grad or qs.requires_grad):
        raise RuntimeError("the low-bit GEMM is inference only: an input requires grad")
    device = q.device
    _on(device, qs, words, wscale, bias, y, acc_out, residual)
    if config is not None and not hasattr(config, "tile"):
        config = None  # a reference tile tuple (its RTX 5090 tiling): accepted, results never depend on tiles
    tile = 0 if config is None else int(config.tile)
    split = 0 if config is None else int(config.split)
    need = _workspace_bytes(wbits, parts, max(m, 1), n, k, ws_group, split, tile)
    workspace = torch.empty(need, dtype=torch.uint8, device=device) if need else None
    args = (wbits, q.data_ptr(), q.stride(0), ldq, parts,
            qs.data_ptr(), _hip.dtype_code(qs.dtype), qs.stride(0),
            words.data_ptr(), n, k,
            wscale.data_ptr(), _hip.dtype_code(wscale.dtype), ws_group,
            _hip.ptr(bias), _hip.dtype_code(bias.dtype) if bias is not None else 0,
            _hip.ptr(y), _hip.dtype_code(y.dtype) if y is not None else 0, y.stride(0) if y is not None else 0,
            _hip.ptr(acc_out), acc_out.stride(1) if acc_out is not None else 0,
            m, int(silu) | (2 * int(order)) | (4 * int(glu)), split, tile,
            _hip.ptr(workspace), need)
    return args, device, workspace


def gemm(wbits: int, q: Tensor, qs: Tensor, words: Tensor, n: int, k: int, wscale: Tensor, bias: Tensor | None,
         y: Tensor | None = None, acc_out: Tensor | None = None, *, m: int | None = None, silu: bool = False,
         order: int = 0, config=None, ws_group: int = 0, residual: Tensor | None = None,
         residual_factor: float = 1.0, glu: bool = False) -> None:
    """y[:m] (rows of stride y.stride(0)) and/or acc_out [P, m, N] from q int8 [P, M, ldq] (16-byte aligned rows) and
    qs [P, M] (f32 or f16). words: native layout of `wbits`-bit weights; wscale [N] (or [N, G] with ws_group).
    residual (FP32 [>= m, >= N] rows, may be y itself): y = residual + value * residual_factor.
    glu: y [m, N/2] = value[2j] * sigmoid(value[2j + 1]) (weight rows interleaved value, gate)."""
    args, device, _ = _gemm_args(wbits, q, qs, words, n, k, wscale, bias, y, acc_out, m, silu, order, config,
                                 ws_group, residual, glu)
    L = _hip.lib()
    if residual is None:
        _hip.check(L.kea_lowbit_gemm(*args, _hip.stream_handle(device)), "kea_lowbit_gemm")
    else:
        _hip.check(L.kea_lowbit_gemm_residual(*args, residual.data_ptr(), residual.stride(0), float(residual_factor),
                                              _hip.stream_handle(device)), "kea_lowbit_gemm_residual")


class GemmPlan:
    """A GEMM call validated once: the checks of gemm() and the library's tile / split / kernel resolution run here
    (kea_lowbit_gemm_plan), and each call only enqueues the launch (kea_lowbit_gemm_plan_launch) on the given stream
    or torch's current stream. Same arguments as gemm(). The plan keeps references to every tensor it was built on
    (they must keep their storage: the plan launches on those buffers) and its own split-K workspace."""

    def __init__(self, wbits: int, q: Tensor, qs: Tensor, words: Tensor, n: int, k: int, wscale: Tensor,
                 bias: Tensor | None, y: Tensor | None = None, acc_out: Tensor | None = None, *, m: int | None = None,
                 silu: bool = False, order: int = 0, config=None, ws_group: int = 0, residual: Tensor | None = None,
                 residual_factor: float = 1.0, glu: bool = False):
        args, self.device, workspace = _gemm_args(wbits, q, qs, words, n, k, wscale, bias, y, acc_out, m, silu,
                                                  order, config, ws_group, residual, glu)
        self._keep = (q, qs, words, wscale, bias, y, acc_out, residual, workspace)
        L = _hip.lib()
        self._free = L.kea_lowbit_gemm_plan_free
        self._launch = L.kea_lowbit_gemm_plan_launch
        self._handle = L.kea_lowbit_gemm_plan(*args, _hip.ptr(residual), residual.stride(0) if residual is not None
                                              else 0, float(residual_factor))
        if not self._handle:
            _hip.check(-1, "kea_lowbit_gemm_plan")

    def __call__(self, stream: int | None = None) -> None:
        """Enqueue the GEMM on `stream` (a hipStream_t handle, e.g. torch.cuda.Stream.cuda_stream) or on torch's
        current stream."""
        rc = self._launch(self._handle, _hip.stream_handle(self.device) if stream is None else stream)
        if rc:
            _hip.check(rc, "kea_lowbit_gemm_plan_launch")

    def __del__(self):
        handle, self._handle = getattr(self, "_handle", None), None
        if handle:
            self._free(handle)


def gemm_slices(wbits: int, q: Tensor, words: Tensor, n: int, k: int, slices: Tensor, *, m: int | None = None,
                config=None) -> None:
    """Exact deferred split-K: slices int32 [S, P, m, N] <- the int32 K-slice sums (S = slices.shape[0])."""
    if q.dtype != torch.int8 or q.dim() != 3 or q.stride(2) != 1 or q.stride(1) != q.shape[2]:
        raise ValueError("q must be int8 [P, M, ldq] with contiguous rows")
    parts, rows, ldq = q.shape
    m = rows if m is None else m
    if m > rows:
        raise ValueError(f"m = {m} exceeds the {rows} rows of q")
    if (slices.dtype != torch.int32 or slices.dim() != 4 or tuple(slices.shape[1:]) != (parts, m, n)
            or not slices.is_contiguous()):
        raise ValueError(f"slices must be contiguous int32 [S, {parts}, {m}, {n}]")
    _check_words(words, n, k, wbits)
    _on(q.device, words, slices)
    tile = 0 if config is None or not hasattr(config, "tile") else int(config.tile)
    rc = _hip.lib().kea_lowbit_gemm_slices(wbits, q.data_ptr(), q.stride(0), ldq, parts, words.data_ptr(), n, k, m,
                                           slices.shape[0], tile, slices.data_ptr(), _hip.stream_handle(q.device))
    _hip.check(rc, "kea_lowbit_gemm_slices")


def slices_finish(slices: Tensor, qs: Tensor, wscale: Tensor, bias: Tensor | None, y: Tensor | None = None,
                  acc_out: Tensor | None = None, *, silu: bool = False, order: int = 0) -> None:
    """y[:m] and/or acc_out from exact int32 slices [S, P, m, N]: slice sums in slice order, then the GEMM epilogue
    (bitwise the unsplit GEMM's result)."""
    if slices.dtype != torch.int32 or slices.dim() != 4 or not slices.is_contiguous():
        raise ValueError("slices must be contiguous int32 [S, P, M, N]")
    split, parts, m, n = slices.shape
    if qs.dim() != 2 or qs.shape[0] != parts or qs.shape[1] < m or qs.stride(1) != 1 or qs.dtype not in _SCALE_DTYPES:
        raise ValueError(f"qs must be f32/f16 [{parts}, >= {m}] with unit column stride")
    if wscale.dtype not in _SCALE_DTYPES or not wscale.is_contiguous() or wscale.numel() != n:
        raise ValueError("weight scales must be contiguous f32 or f16 [N]")
    if bias is not None and (bias.dtype not in _SCALE_DTYPES or not bias.is_contiguous() or bias.numel() != n):
        raise ValueError("bias must be contiguous f32 or f16 [N]")
    if y is None and acc_out is None:
        raise ValueError("nothing to compute: y and acc_out are both None")
    if y is not None and (y.dim() != 2 or y.shape[0] < m or y.shape[1] < n or y.stride(1) != 1):
        raise ValueError(f"y must be a row-major [>= {m}, >= {n}] view")
    if acc_out is not None and (acc_out.dtype != torch.int32 or tuple(acc_out.shape[:2]) != (parts, m)
                                or acc_out.shape[2] < n or acc_out.stride(2) != 1
                                or acc_out.stride(0) != m * acc_out.stride(1)):
        raise ValueError(f"acc_out must be int32 [{parts}, {m}, >= {n}] with dense part planes")
    _on(slices.device, qs, wscale, bias, y, acc_out)
    rc = _hip.lib().kea_lowbit_slices_finish(
        slices.data_ptr(), split, parts, m, n, qs.data_ptr(), _hip.dtype_code(qs.dtype), qs.stride(0),
        wscale.data_ptr(), _hip.dtype_code(wscale.dtype), _hip.ptr(bias),
        _hip.dtype_code(bias.dtype) if bias is not None else 0,
        _hip.ptr(y), _hip.dtype_code(y.dtype) if y is not None else 0, y.stride(0) if y is not None else 0,
        _hip.ptr(acc_out), acc_out.stride(1) if acc_out is not None else 0,
        int(silu) | (2 * int(order)), _hip.stream_handle(slices.device))
    _hip.check(rc, "kea_lowbit_slices_finish")


def _norm_params(norm, n: int, device) -> tuple[Tensor | None, Tensor | None, float]:
    if norm is None:
        return None, None, 0.0
    w = norm.weight.detach()
    b = norm.bias.detach()
    if w.numel() != n or b.numel() != n:
        raise ValueError("LayerNorm shape does not match the row length")
    if w.dtype != torch.float32 or w.device != device or not w.is_contiguous():
        w = w.to(device=device, dtype=torch.float32).contiguous()
    if b.dtype != torch.float32 or b.device != device or not b.is_contiguous():
        b = b.to(device=device, dtype=torch.float32).contiguous()
    return w, b, float(norm.eps)


def row_epilogue(slices: Tensor, qs: Tensor, wscale: Tensor, bias: Tensor | None, y: Tensor, *,
                 residual: Tensor | None = None, factor: float = 1.0, out_norm=None, norm=None,
                 quantize_parts: int = 0, silu: bool = False, order: int = 0) -> tuple[Tensor, Tensor] | None:
    """The exact row epilogue (kea_row_epilogue): y [M, N] FP32 rows <- [out_norm](residual + factor * value), value
    the unsplit GEMM epilogue of the int32 slices [S, P, M, N]; with quantize_parts > 0 also returns (q, q_scales),
    the quantize_parts-part quantization of norm(y) (of y when norm is None), as kea_quantize would."""
    if slices.dtype != torch.int32 or slices.dim() != 4 or not slices.is_contiguous():
        raise ValueError("slices must be contiguous int32 [S, P, M, N]")
    split, parts, m, n = slices.shape
    if qs.dim() != 2 or qs.shape[0] != parts or qs.shape[1] < m or qs.stride(1) != 1 or qs.dtype != torch.float32:
        raise ValueError(f"qs must be FP32 [{parts}, >= {m}] with unit column stride")
    if wscale.dtype not in _SCALE_DTYPES or not wscale.is_contiguous() or wscale.numel() != n:
        raise ValueError("weight scales must be contiguous f32 or f16 [N]")
    if bias is not None and (bias.dtype not in _SCALE_DTYPES or not bias.is_contiguous() or bias.numel() != n):
        raise ValueError("bias must be contiguous f32 or f16 [N]")
    if y.dtype != torch.float32 or y.dim() != 2 or y.shape[0] < m or y.shape[1] < n or y.stride(1) != 1:
        raise ValueError(f"y must be a row-major FP32 [>= {m}, >= {n}] view")
    if residual is not None and (residual.dtype != torch.float32 or residual.dim() != 2 or residual.shape[0] < m
                                 or residual.shape[1] < n or residual.stride(1) != 1):
        raise ValueError(f"residual must be a row-major FP32 [>= {m}, >= {n}] view")
    if not 0 <= quantize_parts <= 3 or (norm is not None and quantize_parts == 0):
        raise ValueError("quantize_parts must be 1..3 when a next LayerNorm is given (0: no quantization)")
    device = slices.device
    _on(device, qs, wscale, bias, y, residual)
    ow, ob, oeps = _norm_params(out_norm, n, device)
    nw, nb, eps = _norm_params(norm, n, device)
    q = qsc = None
    ldq = round_up(n, 16)
    if quantize_parts:
        q = torch.empty(quantize_parts, m, ldq, device=device, dtype=torch.int8)
        qsc = torch.empty(quantize_parts, m, device=device, dtype=torch.float32)
    rc = _hip.lib().kea_row_epilogue(
        slices.data_ptr(), split, parts, m, n, qs.data_ptr(), qs.stride(0), wscale.data_ptr(),
        _hip.dtype_code(wscale.dtype), _hip.ptr(bias), _hip.dtype_code(bias.dtype) if bias is not None else 0,
        int(silu) | (2 * int(order)), _hip.ptr(residual), residual.stride(0) if residual is not None else 0,
        float(factor), _hip.ptr(ow), _hip.ptr(ob), oeps, y.data_ptr(), y.stride(0), _hip.ptr(nw), _hip.ptr(nb), eps,
        quantize_parts, _hip.ptr(q), ldq, _hip.ptr(qsc), _hip.stream_handle(device))
    _hip.check(rc, "kea_row_epilogue")
    return (q, qsc) if quantize_parts else None


def round_up(v: int, multiple: int) -> int:
    return -(-v // multiple) * multiple


def quantize(x: Tensor, rows: tuple, m: int, k: int, parts: int, *, norm=None, input_activation: str = "",
             qs_dtype: torch.dtype = torch.float32, ldq: int | None = None) -> tuple[Tensor, Tensor, int]:
    """Residual int8 parts of x: row r at x + (r // T) * XB + (r % T) * XT + kk * XK with rows = (XB, XT, XK, T).

    Returns q int8 [parts, m, ldq] (zero padded from k to ldq = round_up(k, 16)), qs [parts, m] and ldq."""
    if x.dtype not in (torch.float32, torch.float16):
        raise ValueError(f"expected FP32 or FP16 input, got {x.dtype}")
    if input_activation not in ("", "silu"):
        raise ValueError(f"unsupported input activation {input_activation!r}")
    xb, xt, xk, t = rows
    if m > 0:
        if min(xb, xt, xk) < 0 or t < 1 or k < 1:
            raise ValueError(f"row addressing {rows} needs non-negative strides, T >= 1 and k >= 1")
        # the furthest element any row reads: the last row, or the last row of the last full batch before it
        b_last, r_last = divmod(m - 1, t)
        far = b_last * xb + r_last * xt
        if b_last >= 1:
            far = max(far, (b_last - 1) * xb + (t - 1) * xt)
        far += (k - 1) * xk
        if x.storage_offset() + far >= x.untyped_storage().nbytes() // x.element_size():
            raise ValueError(f"rows {rows} x {m} rows x {k} features reach past the end of x's storage")
    ldq = round_up(k, 16) if ldq is None else ldq
    q = torch.empty(parts, m, ldq, device=x.device, dtype=torch.int8)
    qs = torch.empty(parts, m, device=x.device, dtype=qs_dtype)
    if m == 0:
        return q, qs, ldq
    nw = nb = None
    eps = 0.0
    if norm is not None:
        nw = norm.weight.detach().to(device=x.device, dtype=torch.float32).contiguous()
        nb = norm.bias.detach().to(device=x.device, dtype=torch.float32).contiguous()
        eps = float(norm.eps)
        if nw.numel() != k or nb.numel() != k:
            raise ValueError("LayerNorm shape does not match the input features")
    rc = _hip.lib().kea_quantize(x.data_ptr(), _hip.dtype_code(x.dtype), xb, xt, xk, max(t, 1), m, k, parts,
                                 _hip.ptr(nw), _hip.ptr(nb), eps, int(input_activation == "silu"), q.data_ptr(), ldq,
                                 qs.data_ptr(), _hip.dtype_code(qs_dtype), _hip.stream_handle(x.device))
    _hip.check(rc, "kea_quantize")
    return q, qs, ldq


class _Entry:
    """One resolved call layout of a Launches cache: a plan (a projection plan, or a GEMM plan for dot()), the C
    function that frees it and the device workspace bytes one launch of it needs."""
    __slots__ = ("plan", "free", "need")

    def __del__(self):
        plan, self.plan = getattr(self, "plan", None), None
        if plan:
            self.free(plan)


class Launches:
    """The launches of one weight matrix (an operator's layer), resolved once per call layout.

    An operator call is the residual quantizer of its input plus the low-bit GEMM. gemm() and quantize() check every
    argument and resolve the tile, split and kernel on each call, about 11 us of host time each. Here the first call
    of a layout (input dtype, shape and strides, part count, output dtype and row stride, epilogue flags, LayerNorm)
    does those checks once and keeps a projection plan (kea_lowbit_project_plan: the quantizer's arguments and a GEMM
    plan); later calls of that layout allocate one workspace for the int8 parts, their scales and any split-K slices
    and make one C call, kea_lowbit_project_launch, which enqueues the quantizer and the GEMM on the new x, y and
    workspace. The reference validates and launches on every call (kk/binary/layer.py:154-165 and :182-209,
    kk/ternary/fused_kernels.py:139-160); the results are the same bits either way. Layouts are kept up to
    `max_entries` (the oldest is dropped first)."""

    def __init__(self, wbits: int, words: Tensor, n: int, k: int, wscale: Tensor, bias: Tensor | None, *,
                 max_entries: int = 64):
        self.wbits, self.words, self.n, self.k, self.wscale, self.bias = wbits, words, n, k, wscale, bias
        self.max_entries = max_entries
        self._entries: dict = {}
        self._calls: dict = {}

    def __len__(self) -> int:
        return len(self._entries)

    @staticmethod
    def _norm_key(norm, device):
        """(weight pointer, bias pointer, eps) of a LayerNorm whose parameters the kernel can read in place (f32,
        contiguous, on the device), None without one, False where they would need a copy (the uncached path)."""
        if norm is None:
            return None
        w, b = getattr(norm, "weight", None), getattr(norm, "bias", None)
        for t in (w, b):
            if t is None or t.dtype != torch.float32 or t.device != device or not t.is_contiguous():
                return False
        return (w.data_ptr(), b.data_ptr(), float(norm.eps))

    def project(self, x: Tensor, rows: tuple, m: int, parts: int, y: Tensor, *, silu: bool = False,
                order: int = 0, norm=None, input_activation: str = "", config=None) -> bool:
        """y[:m] (row-major [>= m, N] view) = the GEMM of the parts-part quantization of x's rows (x's own rows:
        `rows` = (XB, XT, XK, T) derived from x's shape and strides by the caller, so every row lies inside x).
        Returns the layout's entry (for remember()), or False, having done nothing, where the call needs the uncached
        path (a LayerNorm whose parameters are not f32 device-contiguous)."""
        nkey = self._norm_key(norm, x.device)
        if nkey is False:
            return False
        tile = 0 if config is None or not hasattr(config, "tile") else (int(config.tile), int(config.split))
        key = (x.dtype, x.device, tuple(x.shape), x.stride(), rows, m, parts, y.dtype, y.stride(0), tuple(y.shape),
               bool(silu), order, nkey, input_activation, tile)
        e = self._entries.get(key)
        if e is None:
            e = self._resolve(key, x, rows, m, parts, y, silu, order, norm, input_activation, config)
        self.launch(e, x, y)
        return e

    @staticmethod
    def launch(e: _Entry, x: Tensor, y: Tensor) -> None:
        """One launch of a projection entry on x and y of its layout: a workspace from torch's allocator (stream
        ordered, so it may be reused as soon as the launches are enqueued) and kea_lowbit_project_launch."""
        ws = torch.empty(e.need, dtype=torch.uint8, device=x.device)
        rc = _hip.lib().kea_lowbit_project_launch(e.plan, x.data_ptr(), y.data_ptr(), ws.data_ptr(), e.need,
                                                  _hip.stream_handle(x.device))
        if rc:
            _hip.check(rc, "kea_lowbit_project_launch")

    def recall(self, key):
        """What an operator kept with remember() for `key`: (entry, output shape), or None."""
        try:
            return self._calls.get(key)
        except TypeError:  # an unhashable argument, which the operator's checks refuse
            return None

    def remember(self, key, e: _Entry, out_shape: tuple) -> None:
        """Keeps a projection entry under an operator's own key: a tuple of the call's inputs (tensor shapes,
        strides, dtypes, device) from which the operator derives every argument it checks and passes, so that a call
        with the same key may skip to launch(). Up to `max_entries` keys (the oldest is dropped first)."""
        if len(self._calls) >= self.max_entries:
            self._calls.pop(next(iter(self._calls)), None)
        self._calls[key] = (e, out_shape)

    def _resolve(self, key, x, rows, m, parts, y, silu, order, norm, input_activation, config) -> _Entry:
        """The first call of a layout: the full checks of quantize() and gemm() on real buffers, then the plan."""
        if m < 1:
            raise ValueError("a cached launch needs at least one row")
        q, qs, _ = quantize(x, rows, m, self.k, parts, norm=norm, input_activation=input_activation)
        args, _, workspace = _gemm_args(self.wbits, q, qs, self.words, self.n, self.k, self.wscale, self.bias, y,
                                        None, m, silu, order, config, 0, None, False)
        L = _hip.lib()
        plan = L.kea_lowbit_gemm_plan(*args, None, 0, 1.0)
        if not plan:
            _hip.check(-1, "kea_lowbit_gemm_plan")
        nw, nb, eps = (None, None, 0.0) if norm is None else (norm.weight.data_ptr(), norm.bias.data_ptr(),
                                                              float(norm.eps))
        xb, xt, xk, t = rows
        try:  # the projection plan copies the GEMM plan
            pp = L.kea_lowbit_project_plan(plan, _hip.dtype_code(x.dtype), xb, xt, xk, max(t, 1), nw, nb, eps,
                                           int(input_activation == "silu"))
        finally:
            L.kea_lowbit_gemm_plan_free(plan)
        if not pp:
            _hip.check(-1, "kea_lowbit_project_plan")
        e = _Entry()
        e.free = L.kea_lowbit_project_plan_free
        e.plan = pp
        e.need = int(L.kea_lowbit_project_workspace(pp))
        if len(self._entries) >= self.max_entries:
            self._entries.pop(next(iter(self._entries)), None)
        self._entries[key] = e
        return e

    def dot(self, q: Tensor, qs: Tensor, m: int, y: Tensor | None, acc_out: Tensor | None = None, *,
            silu: bool = False, order: int = 0, config=None) -> None:
        """gemm() of caller-made parts q int8 [P, >= m, ldq] / qs [P, >= m] with this matrix, resolved once per
        layout of (q, qs, y, acc_out, flags)."""
        tile = 0 if config is None or not hasattr(config, "tile") else (int(config.tile), int(config.split))
        key = ("dot", q.dtype, q.device, tuple(q.shape), q.stride(), qs.dtype, tuple(qs.shape), qs.stride(), m,
               None if y is None else (y.dtype, tuple(y.shape), y.stride()),
               None if acc_out is None else (acc_out.dtype, tuple(acc_out.shape), acc_out.stride()),
               bool(silu), order, tile)
        e = self._entries.get(key)
        if e is None or m < 1:
            if m < 1:  # nothing to launch (the library's m = 0 path)
                gemm(self.wbits, q, qs, self.words, self.n, self.k, self.wscale, self.bias, y, acc_out, m=m, silu=silu,
                     order=order, config=config)
                return
            args, _, _ = _gemm_args(self.wbits, q, qs, self.words, self.n, self.k, self.wscale, self.bias, y, acc_out,
                                    m, silu, order, config, 0, None, False)
            L = _hip.lib()
            e = _Entry()
            e.free = L.kea_lowbit_gemm_plan_free
            e.plan = L.kea_lowbit_gemm_plan(*args, None, 0, 1.0)
            if not e.plan:
                _hip.check(-1, "kea_lowbit_gemm_plan")
            e.need = int(L.kea_lowbit_gemm_plan_workspace(e.plan))
            if len(self._entries) >= self.max_entries:
                self._entries.pop(next(iter(self._entries)), None)
            self._entries[key] = e
        if torch.is_grad_enabled() and (q.requires_grad or qs.requires_grad):
            raise RuntimeError("the low-bit GEMM is inference only: an input requires grad")
        ws = torch.empty(e.need, dtype=torch.uint8, device=q.device) if e.need else None
        rc = _hip.lib().kea_lowbit_gemm_plan_launch_with(
            e.plan, q.data_ptr(), qs.data_ptr(), _hip.ptr(y), _hip.ptr(acc_out), None,
            ws.data_ptr() if ws is not None else None, e.need, _hip.stream_handle(q.device))
        if rc:
            _hip.check(rc, "kea_lowbit_gemm_plan_launch_with")
