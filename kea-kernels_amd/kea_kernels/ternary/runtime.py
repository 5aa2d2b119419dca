"""Packed ternary modules (drop-in for kk/ternary/runtime.py).

PackedLinear keeps the reference's resident form, `packed_t` = the export bytes padded to whole 32-bit words and
transposed to int32 [ceil(K/16), N] (code k of row n at bits 2 * (k % 16) of packed_t[k // 16, n];
kk/ternary/runtime.py:182-184), and adds `native`, the same codes in the gfx950 wavefront layout the int8 GEMM reads
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


class PackedLinear(nn.Module):
    def __init__(self, packed: torch.Tensor, scale: torch.Tensor, in_features: int, bias: torch.Tensor | None = None,
                 *, mode: str = "bf16x3"):
        super().__init__()
        from kea_kernels.formats import unpack_ternary
        if in_features < 1 or packed.ndim != 2 or packed.shape[0] < 1:
            raise ValueError("weight dimensions must be positive")
        if packed.device != scale.device or (bias is not None and bias.device != packed.device):
            raise ValueError("codes, scales, and bias must be on the same device")
        unpack_ternary(packed, in_features)  # validates: the 11 pattern and tail codes raise
        n = packed.shape[0]
        if scale.shape != (n,) or scale.dtype != torch.float32 or not bool(torch.isfinite(scale).all()):
            raise ValueError("scale must be finite FP32 [N]")
        if bias is not None and (bias.shape != (n,) or bias.dtype != torch.float32
                                 or not bool(torch.isfinite(bias).all())):
            raise ValueError("bias must be finite FP32 [N]")
        if mode not in MODES:
            raise ValueError(f"unknown mode {mode!r}")
        self.in_features, self.out_features, self.mode = in_features, n, mode
        self.register_buffer("packed_t", packed_t_from_codes(packed))
        self.register_buffer("scale", scale.contiguous())
        self.register_buffer("bias", bias.contiguous() if bias is not None else None)
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


def load_packed(directory: str | Path, manifest: dict, device: str | torch.device = "cuda", *, mode: str = "bf16x3"):
    """A NeMo model from a validated export with the 264 ternary layers packed (kk/ternary/runtime.py:52-82).

    Needs nemo_toolkit (not installed in this build's image): RuntimeError from formats.build_nemo otherwise."""
    from safetensors.torch import load_file

    from kea_kernels import formats
    if mode not in ("tf32x3", "bf16x3"):
        raise ValueError("the model loader requires a high-accuracy mode (tf32x3 or bf16x3)")
    device = torch.device(device)
    directory = Path(directory)
    layers = manifest["quantized_layers"]
    model = formats.build_nemo(manifest, directory)
    tensors = load_file(directory / manifest["file"])
    packed_state = {}
    for name, layer in layers.items():
        original = model.get_submodule(name)
        n, k = layer["shape"]
        if tuple(original.weight.shape[:2]) != (n, k):
            raise ValueError(f"invalid shape for {name}")
        cls = {"linear": PackedLinear, "pointwise_conv1d": PackedPointwiseConv1d}[layer["kind"]]
        module = cls(tensors.pop(f"{name}.codes"), tensors.pop(f"{name}.scale"), k,
                     tensors.pop(f"{name}.bias") if layer["bias"] else None, mode=mode)
        model.set_submodule(name, module)
        packed_state.update((f"{name}.{key}", value) for key, value in module.state_dict().items())
    state = {key: value.float() if value.is_floating_point() else value for key, value in tensors.items()}
    state.update(packed_state)
    model.load_state_dict(state, strict=True)
    return model.to(device=device).eval()
