"""Packed ternary modules (drop-in for kk/ternary/runtime.py).

PackedLinear keeps the reference's resident form, `packed_t` = the export bytes padded to whole 32-bit words and
transposed to int32 [ceil(K/16), N] (code k of row n at bits 2 * (k % 16) of packed_t[k // 16, n];
kk/ternary/runtime.py:33-35), and adds `native`, the same codes in the gfx950 wavefront layout the int8 GEMM reads
(include/kea_lowbit.h). Both stay 2 bits per weight on the GPU.

forward runs the int8 path: x is split into `parts` residual int8 parts (3 unless the mode says otherwise) and
multiplied on int8 MFMA. The reference's FP-activation modes (tf32x3 / bf16x3 / fp16 Triton kernels) are not part of
this build; their mode names are accepted and map to three int8 parts, whose error against FP64 (~1e-6 relative) is
within the reference's own bound for those modes (1e-5, tests/test_kernels_gpu.py:93-105 of the reference).
"""
from __future__ import annotations

from pathlib import Path

import torch
from torch import nn

from kea_kernels.binary import kernels as layout

MODES = {"tf32x3": 3, "bf16x3": 3, "fp16": 3, "x1": 1, "x2": 2, "x3": 3}


def packed_t_from_codes(packed: torch.Tensor) -> torch.Tensor:
    """Export codes uint8 [N, ceil(K/4)] -> int32 [ceil(K/16), N] (the reference's resident word layout)."""
    padded = torch.nn.functional.pad(packed, (0, (-packed.shape[1]) % 4))
    return padded.contiguous().view(torch.int32).t().contiguous()


def codes_from_packed_t(packed_t: torch.Tensor, in_features: int) -> torch.Tensor:
    """Inverse of packed_t_from_codes (on the CPU)."""
    words = packed_t.detach().cpu().t().contiguous()
    return words.view(torch.uint8)[:, :-(-in_features // 4)].contiguous()


def native_words(mod) -> torch.Tensor:
    """The gfx950 native words of a module with `packed_t` (cached on the module, on packed_t's device)."""
    native = getattr(mod, "native", None)
    if native is not None and native.device == mod.packed_t.device:
        return native
    codes = codes_from_packed_t(mod.packed_t, mod.in_features)
    native = layout.relayout_codes(codes, mod.in_features, 2).to(mod.packed_t.device)
    if isinstance(mod, nn.Module) and "native" in mod._buffers:
        mod._buffers["native"] = native
    else:
        object.__setattr__(mod, "native", native)
    return native


def _finite_f32_vector(t, n: int) -> bool:
    return t.shape == (n,) and t.dtype == torch.float32 and bool(torch.isfinite(t).all())


def _validate(packed: torch.Tensor, scale: torch.Tensor, in_features: int, bias: torch.Tensor | None,
              mode: str) -> None:
    """The module's argument checks, in the reference's order and with its messages (kk/ternary/runtime.py:12-31):
    dimensions, one device, valid 2-bit codes (the 11 pattern and tail codes raise), finite FP32 scale and bias of
    length N, a known mode."""
    from kea_kernels.formats import unpack_ternary
    if in_features < 1 or packed.ndim != 2 or packed.shape[0] < 1:
        raise ValueError("weight dimensions must be positive")
    if any(t is not None and t.device != packed.device for t in (scale, bias)):
        raise ValueError("codes, scales, and bias must be on the same device")
    unpack_ternary(packed, in_features)
    n = packed.shape[0]
    if not _finite_f32_vector(scale, n):
        raise ValueError("scale must be finite FP32 [N]")
    if bias is not None and not _finite_f32_vector(bias, n):
        raise ValueError("bias must be finite FP32 [N]")
    if mode not in MODES:
        raise ValueError(f"unknown mode {mode!r}")


class PackedLinear(nn.Module):
    """A ternary linear layer kept 2 bits per weight on the GPU: `packed_t` (the reference's resident words) and
    `native` (the gfx950 layout the int8 GEMM reads); forward quantizes x to `parts` int8 parts and runs the GEMM."""

    def __init__(self, packed: torch.Tensor, scale: torch.Tensor, in_features: int, bias: torch.Tensor | None = None,
                 *, mode: str = "bf16x3"):
        super().__init__()
        _validate(packed, scale, in_features, bias, mode)
        self.in_features, self.out_features, self.mode = in_features, packed.shape[0], mode
        self.register_buffer("packed_t", packed_t_from_codes(packed))
        self.register_buffer("scale", scale.contiguous())
        self.register_buffer("bias", None if bias is None else bias.contiguous())
        self.register_buffer("native", layout.relayout_codes(packed.cpu(), in_features, 2).to(packed.device),
                             persistent=False)
        self.eval()

    @property
    def parts(self) -> int:
        return MODES[self.mode]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        from kea_kernels.ternary.fused_kernels import int8_matmul
        return int8_matmul(x, self, components=self.parts)

    def extra_repr(self):
        return f"in_features={self.in_features}, out_features={self.out_features}, mode={self.mode!r}"


class PackedPointwiseConv1d(PackedLinear):
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        from kea_kernels.ternary.fused_kernels import int8_matmul
        return int8_matmul(x, self, conv=True, components=self.parts)


_PACKED_KINDS = {"linear": PackedLinear, "pointwise_conv1d": PackedPointwiseConv1d}
LOADER_MODES = ("tf32x3", "bf16x3")


def load_packed(directory: str | Path, manifest: dict, device: str | torch.device = "cuda", *, mode: str = "bf16x3"):
    """A NeMo model from a validated parakeet-ternary-v1 export with its 264 quantized modules replaced by packed
    modules built from the export's codes (no dense ternary weight is formed) and every other tensor loaded as FP32.
    Needs nemo_toolkit (RuntimeError from formats.build_nemo without it)."""
    from safetensors.torch import load_file

    from kea_kernels import formats
    if mode not in LOADER_MODES:
        raise ValueError("the model loader requires a high-accuracy mode (tf32x3 or bf16x3)")
    directory = Path(directory)
    model = formats.build_nemo(manifest, directory)
    tensors = load_file(directory / manifest["file"])
    state = {}
    for name, info in manifest["quantized_layers"].items():
        n, k = info["shape"]
        if tuple(model.get_submodule(name).weight.shape[:2]) != (n, k):
            raise ValueError(f"invalid shape for {name}")
        bias = tensors.pop(f"{name}.bias") if info["bias"] else None
        module = _PACKED_KINDS[info["kind"]](tensors.pop(f"{name}.codes"), tensors.pop(f"{name}.scale"), k, bias,
                                             mode=mode)
        model.set_submodule(name, module)
        state.update({f"{name}.{key}": value for key, value in module.state_dict().items()})
    state.update({key: value.float() if value.is_floating_point() else value for key, value in tensors.items()})
    model.load_state_dict(state, strict=True)
    return model.to(device=torch.device(device)).eval()
