"""The 1-bit layers at the projection-provider seam (drop-in for kk/binary/provider.py).

Every quantized-layer call of the encoder goes through one `provider` object (kk/binary/provider.py:3-15):

    provider(x, mod, conv=False, components=3, activation="", norm=None, config=None, input_activation="")

    xx = x.transpose(1, 2) if conv else x           # conv: [B, K, T] -> [B, T, K] view
    z  = LayerNorm(norm)(xx) if norm else xx        # fused input normalization
    z  = z * sigmoid(z) if input_activation == "silu" else z
    y  = alpha * (W z) + bias                       # the quantized layer, [B, T, N]
    y  = y * sigmoid(y) if activation == "silu" else y
    return y.transpose(1, 2) if conv else y          # conv returns a [B, N, T] view

`components` is the number of residual int8 activation parts. Modules carry no GPU weights: a module's `packed_t` is
a CPU int64 row HANDLE [1, N] (global row ids), and torch.cat of the Q/K/V handles yields the handle of the fused
[3072, 1024] QKV layer, which the provider resolves to that layer (kk/binary/provider.py:17-23, :78-79). The 1-bit
layer objects (Int8MmaLayer / Int8MmaPartsLayer) hold the only GPU copy of the weights.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path

import torch
import torch.nn.functional as F
from torch import Tensor, nn

QKV = ("linear_q", "linear_k", "linear_v")


@dataclass
class Entry:
    """One prepared 1-bit layer and the global row-handle range of its outputs."""
    name: str
    layer: object
    kind: str            # "linear" or "conv"
    out_features: int
    in_features: int
    start: int           # first global row id
    members: tuple = ()  # a fused QKV entry: the three module names


@dataclass
class Table:
    entries: list = field(default_factory=list)
    next_row: int = 0

    def add(self, name, layer, kind, n, k, members=()) -> Entry:
        entry = Entry(name, layer, kind, n, k, self.next_row, tuple(members))
        self.entries.append(entry)
        self.next_row += n
        return entry

    def resolve(self, start: int, count: int) -> tuple[Entry, int]:
        """(entry, offset) of the layer whose rows [start, start + count) are; ValueError across layers."""
        for entry in self.entries:
            if entry.start <= start < entry.start + entry.out_features:
                if start + count > entry.start + entry.out_features:
                    raise ValueError("handle range crosses layers")
                return entry, start - entry.start
        raise KeyError(f"no layer owns row handle {start}")

    def weight_bytes(self) -> int:
        return sum(entry.layer.weight_bytes() for entry in self.entries)


def _handle(start: int, n: int) -> Tensor:
    return torch.arange(start, start + n, dtype=torch.int64).view(1, n)


class _BinaryMixin:
    """The attributes encoder transforms read: in_features, out_features, mode, packed_t (a row handle), scale, bias."""

    def _setup(self, entry: Entry, offset: int, n: int, k: int, scale_cpu: Tensor, bias_cpu: Tensor | None):
        nn.Module.__init__(self)
        self.in_features, self.out_features, self.mode = k, n, "binary"
        self._entry, self._offset = entry, offset
        # plain attributes, not buffers: never moved to the GPU, absent from state_dict
        object.__setattr__(self, "packed_t", _handle(entry.start + offset, n))
        object.__setattr__(self, "scale", scale_cpu.detach().clone().contiguous())
        object.__setattr__(self, "bias", None if bias_cpu is None else bias_cpu.detach().clone().contiguous())
        self.eval()

    def _run(self, x: Tensor, conv: bool) -> Tensor:
        entry = self._entry
        y = entry.layer.conv(x) if conv else entry.layer.linear(x)
        if self.out_features == entry.out_features:
            return y
        lo, hi = self._offset, self._offset + self.out_features  # a member of a fused layer called alone
        return y[:, lo:hi] if conv else y[..., lo:hi]

    def extra_repr(self):
        return f"in_features={self.in_features}, out_features={self.out_features}, layer={self._entry.name!r}"


def _packed_classes():
    """BinaryLinear / BinaryPointwiseConv1d: subclasses of the ternary packed modules, as encoder transforms that
    dispatch on module type expect (kk/binary/provider.py:107-124)."""
    from kea_kernels.ternary.runtime import PackedLinear, PackedPointwiseConv1d

    class BinaryLinear(_BinaryMixin, PackedLinear):
        def __init__(self, *a):
            self._setup(*a)

        def forward(self, x):
            return self._run(x, False)

    class BinaryPointwiseConv1d(_BinaryMixin, PackedPointwiseConv1d):
        def __init__(self, *a):
            self._setup(*a)

        def forward(self, x):
            return self._run(x, True)

    return BinaryLinear, BinaryPointwiseConv1d


class BinaryProjection:
    """The provider object: resolves a module's row handle to its layer and runs the fused op."""

    def __init__(self, table: Table, names: dict | None = None):
        self.table = table
        self._resolved: dict = {}
        self.names = names or {}

    @property
    def bytes(self) -> int:
        return self.table.weight_bytes()

    def _lookup(self, mod) -> tuple[Entry, int, int]:
        handle = mod.packed_t
        key = (handle.data_ptr(), tuple(handle.shape))
        hit = self._resolved.get(key)
        if hit is None:
            if handle.is_cuda or handle.dtype != torch.int64 or handle.dim() != 2 or handle.shape[0] != 1:
                raise TypeError("BinaryProjection serves BinaryLinear / BinaryPointwiseConv1d handles only")
            start, count = int(handle[0, 0]), handle.shape[1]
            if not torch.equal(handle[0], torch.arange(start, start + count)):
                raise ValueError("non-contiguous row handle")
            entry, offset = self.table.resolve(start, count)
            hit = (entry, offset, count)
            self._resolved[key] = hit
        return hit

    def __call__(self, x, mod, conv=False, components=3, activation="", norm=None, config=None, input_activation=""):
        if config is not None:
            raise ValueError("BinaryProjection takes no tile config")
        if activation not in ("", "silu") or input_activation not in ("", "silu"):
            raise ValueError(f"unsupported activation {activation!r} / {input_activation!r}")
        entry, offset, count = self._lookup(mod)
        layer = entry.layer
        if hasattr(layer, "project"):
            y = layer.project(x, conv=conv, components=components, activation=activation, norm=norm,
                              input_activation=input_activation)
        else:  # a layer object with linear / conv only: unfused LayerNorm / SiLU around it
            z = x.transpose(1, 2) if conv else x
            if norm is not None:
                z = F.layer_norm(z, norm.normalized_shape, norm.weight, norm.bias, norm.eps)
            if input_activation == "silu":
                z = F.silu(z)
            y = layer.linear(z)
            if activation == "silu":
                y = F.silu(y)
            if conv:
                y = y.transpose(1, 2)
        if count != entry.out_features:
            y = y[:, offset:offset + count] if conv else y[..., offset:offset + count]
        return y


class PartCount:
    """Wraps a provider and sets `components` (the int8 activation part count) to n on every call, including callers
    that hard-code components=3. Attribute writes other than (provider, n) reach the wrapped provider
    (kk/binary/provider.py:185-209)."""

    OWN = ("provider", "n")

    def __init__(self, provider, n: int):
        if n not in (1, 2, 3):
            raise ValueError("n must be 1, 2 or 3")
        object.__setattr__(self, "provider", provider)
        object.__setattr__(self, "n", n)

    def __setattr__(self, name, value):
        if name in PartCount.OWN:
            object.__setattr__(self, name, value)
        else:
            setattr(self.provider, name, value)

    def __call__(self, x, mod, conv=False, components=3, activation="", norm=None, config=None, input_activation=""):
        return self.provider(x, mod, conv, self.n, activation, norm, config, input_activation)

    def __getattr__(self, name):
        return getattr(self.provider, name)


def prepare_table(layers: dict, layer_cls, device="cuda", *, fuse_qkv: bool = True):
    """Table and modules from {name: (codes, scale, bias, kind)} without NeMo: Q/K/V of one attention block are
    prepared as one fused layer (the handles of the three modules are row slices of it). Returns (table, modules)."""
    BinaryLinear, BinaryPointwiseConv1d = _packed_classes()
    table = Table()
    modules = {}
    pending = dict(layers)
    if fuse_qkv:
        blocks = sorted({name.rsplit(".", 1)[0] for name in layers if name.endswith("." + QKV[0])})
        for block in blocks:
            names = [f"{block}.{q}" for q in QKV]
            if not all(name in layers for name in names):
                continue
            shapes = {tuple(layers[name][0].shape) for name in names}
            if len(shapes) != 1 or any(layers[name][2] is not None or layers[name][3] != "linear" for name in names):
                raise ValueError(f"{block}: Q/K/V must be equal-shape bias-free linear layers")
            k = layers[names[0]][4] if len(layers[names[0]]) > 4 else 8 * layers[names[0]][0].shape[1]
            n = layers[names[0]][0].shape[0]
            codes = torch.cat([layers[name][0] for name in names])
            scales = torch.cat([layers[name][1] for name in names])
            layer = layer_cls.prepare(codes, scales, None, k, device)
            entry = table.add(f"{block}.qkv", layer, "linear", 3 * n, k, names)
            for i, name in enumerate(names):
                modules[name] = BinaryLinear(entry, i * n, n, k, scales[i * n:(i + 1) * n], None)
                del pending[name]
    for name, item in pending.items():
        codes, scale, bias, kind = item[:4]
        k = item[4] if len(item) > 4 else 8 * codes.shape[1]
        layer = layer_cls.prepare(codes, scale, bias, k, device)
        entry = table.add(name, layer, kind, codes.shape[0], k)
        cls = BinaryPointwiseConv1d if kind == "conv" else BinaryLinear
        modules[name] = cls(entry, 0, codes.shape[0], k, scale, bias)
    return table, modules


def load_binary_model(directory, manifest: dict, layer_cls, device="cuda", *, fuse_qkv: bool = True):
    """(NeMo model on `device`, Table) from a validated parakeet-binary-v1 export (kk/binary/provider.py:212-262).

    Needs nemo_toolkit (not installed in this build's image): RuntimeError from formats.build_nemo otherwise."""
    from safetensors.torch import load_file

    from kea_kernels import formats
    directory = Path(directory)
    device = torch.device(device)
    model = formats.build_nemo(manifest, directory)
    tensors = load_file(directory / manifest["file"])
    layers = {}
    for name, info in manifest["quantized_layers"].items():
        n, k = info["shape"]
        bias = tensors.pop(f"{name}.bias") if info["bias"] else None
        kind = "conv" if info["kind"] == "pointwise_conv1d" else "linear"
        layers[name] = (tensors.pop(f"{name}.codes"), tensors.pop(f"{name}.scale"), bias, kind, k)
    table, modules = prepare_table(layers, layer_cls, device, fuse_qkv=fuse_qkv)
    for name, module in modules.items():
        original = model.get_submodule(name)
        if tuple(original.weight.shape[:2]) != (module.out_features, module.in_features):
            raise ValueError(f"invalid shape for {name}")
        model.set_submodule(name, module)
    state = {key: value.float() if value.is_floating_point() else value for key, value in tensors.items()}
    model.load_state_dict(state, strict=True)
    return model.to(device=device).eval(), table


def module_names(model) -> dict:
    return {id(m): n for n, m in model.named_modules()}
