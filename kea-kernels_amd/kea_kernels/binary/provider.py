"""The 1-bit layers at the projection-provider seam (drop-in for kk/binary/provider.py).

The contract kept from the reference (kk/binary/provider.py:3-23):

    provider(x, mod, conv=False, components=3, activation="", norm=None, config=None, input_activation="")

    xx = x.transpose(1, 2) if conv else x           # conv: [B, K, T] -> [B, T, K] view
    z  = LayerNorm(norm)(xx) if norm else xx        # fused input normalization
    z  = z * sigmoid(z) if input_activation == "silu" else z
    y  = alpha * (W z) + bias                       # the quantized layer, [B, T, N]
    y  = y * sigmoid(y) if activation == "silu" else y
    return y.transpose(1, 2) if conv else y          # conv returns a [B, N, T] view

`components` is the number of residual int8 activation parts. A module's `packed_t` is a CPU int64 row HANDLE [1, N]
of global row ids, and torch.cat of the Q/K/V handles of one block is the handle of their fused [3072, 1024] layer.

How this module keeps it: every prepared layer owns a contiguous range of a global row space (RowSpace, searched by
bisection); modules are views of row ranges (BinaryLinear / BinaryPointwiseConv1d, subclasses of the ternary packed
modules because encoder transforms dispatch on those types); BinaryProjection resolves a handle once per handle
tensor and runs the layer's fused op, slicing the rows a member handle names. The layer objects (Int8MmaLayer /
Int8MmaPartsLayer) hold the only GPU copy of the weights.
"""
from __future__ import annotations

import bisect
from dataclasses import dataclass
from pathlib import Path

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from kea_kernels.ternary.runtime import PackedLinear, PackedPointwiseConv1d

QKV = ("linear_q", "linear_k", "linear_v")


@dataclass(frozen=True)
class Segment:
    """A prepared layer's rows [first, first + out_features) of the global row space."""
    name: str
    layer: object
    kind: str            # "linear" or "conv"
    first: int
    out_features: int
    in_features: int
    members: tuple = ()  # a fused QKV layer: the names of the modules that are its row slices

    @property
    def stop(self) -> int:
        return self.first + self.out_features


class RowSpace:
    """Global row ids of the prepared layers: each layer is allocated the next contiguous range."""

    def __init__(self):
        self.segments: list[Segment] = []
        self._firsts: list[int] = []

    @property
    def rows(self) -> int:
        return self.segments[-1].stop if self.segments else 0

    def allocate(self, name: str, layer, kind: str, out_features: int, in_features: int, members=()) -> Segment:
        segment = Segment(name, layer, kind, self.rows, out_features, in_features, tuple(members))
        self.segments.append(segment)
        self._firsts.append(segment.first)
        return segment

    def locate(self, first: int, count: int) -> tuple[Segment, int]:
        """(segment, offset) of the layer owning rows [first, first + count): KeyError when no layer owns `first`,
        ValueError when the range runs past the end of that layer."""
        i = bisect.bisect_right(self._firsts, first) - 1
        if i < 0 or first >= self.segments[i].stop:
            raise KeyError(f"no layer owns row handle {first}")
        segment = self.segments[i]
        if first + count > segment.stop:
            raise ValueError(f"row handle [{first}, {first + count}) crosses layers")
        return segment, first - segment.first

    def weight_bytes(self) -> int:
        return sum(segment.layer.weight_bytes() for segment in self.segments)


def row_handle(first: int, count: int) -> Tensor:
    """The CPU int64 [1, count] handle of rows first .. first + count - 1."""
    return torch.arange(first, first + count, dtype=torch.int64).unsqueeze(0)


def _bind_rows(module: nn.Module, segment: Segment, offset: int, out_features: int, scale: Tensor,
               bias: Tensor | None) -> None:
    """Makes `module` the view of rows [offset, offset + out_features) of `segment`'s layer. The attributes the encoder
    transforms read (packed_t = the row handle, scale, bias) are plain host attributes: never moved to the GPU and
    absent from state_dict."""
    nn.Module.__init__(module)
    module.in_features, module.out_features, module.mode = segment.in_features, out_features, "binary"
    module._segment, module._offset = segment, offset
    for name, value in (("packed_t", row_handle(segment.first + offset, out_features)),
                        ("scale", scale.detach().clone().contiguous()),
                        ("bias", None if bias is None else bias.detach().clone().contiguous())):
        object.__setattr__(module, name, value)
    module.eval()


def _rows_forward(module, x: Tensor, conv: bool) -> Tensor:
    segment = module._segment
    y = segment.layer.conv(x) if conv else segment.layer.linear(x)
    if module.out_features == segment.out_features:
        return y
    rows = slice(module._offset, module._offset + module.out_features)  # a member of a fused layer, called alone
    return y[:, rows] if conv else y[..., rows]


class BinaryLinear(PackedLinear):
    """A linear module standing for rows of a prepared 1-bit layer."""

    def __init__(self, segment: Segment, offset: int, out_features: int, scale: Tensor, bias: Tensor | None = None):
        _bind_rows(self, segment, offset, out_features, scale, bias)

    def forward(self, x: Tensor) -> Tensor:
        return _rows_forward(self, x, conv=False)

    def extra_repr(self):
        return f"in_features={self.in_features}, out_features={self.out_features}, layer={self._segment.name!r}"


class BinaryPointwiseConv1d(PackedPointwiseConv1d):
    """A pointwise Conv1d ([B, K, T] -> [B, N, T]) standing for rows of a prepared 1-bit layer."""

    def __init__(self, segment: Segment, offset: int, out_features: int, scale: Tensor, bias: Tensor | None = None):
        _bind_rows(self, segment, offset, out_features, scale, bias)

    def forward(self, x: Tensor) -> Tensor:
        return _rows_forward(self, x, conv=True)

    def extra_repr(self):
        return f"in_features={self.in_features}, out_features={self.out_features}, layer={self._segment.name!r}"


_ACTIVATIONS = ("", "silu")


class BinaryProjection:
    """The provider object: resolves a module's row handle to its prepared layer and runs the fused op."""

    def __init__(self, table: RowSpace, names: dict | None = None):
        self.table = table
        self.names = names or {}
        self._handles: dict = {}  # id(handle tensor) -> (handle, segment, offset, count)

    @property
    def bytes(self) -> int:
        return self.table.weight_bytes()

    def resolve(self, mod) -> tuple[Segment, int, int]:
        """(segment, offset, count) of the rows `mod.packed_t` names (cached per handle tensor)."""
        handle = mod.packed_t
        hit = self._handles.get(id(handle))
        if hit is not None and hit[0] is handle:
            return hit[1:]
        if not isinstance(handle, Tensor) or handle.device.type != "cpu" or handle.dtype != torch.int64 \
                or handle.dim() != 2 or handle.shape[0] != 1:
            raise TypeError("BinaryProjection serves the CPU int64 [1, N] row handles of BinaryLinear / "
                            "BinaryPointwiseConv1d")
        first, count = int(handle[0, 0]), handle.shape[1]
        if not torch.equal(handle, row_handle(first, count)):
            raise ValueError("non-contiguous row handle")
        segment, offset = self.table.locate(first, count)
        self._handles[id(handle)] = (handle, segment, offset, count)
        return segment, offset, count

    def __call__(self, x, mod, conv=False, components=3, activation="", norm=None, config=None, input_activation=""):
        if config is not None:
            raise ValueError("BinaryProjection takes no tile config")
        if activation not in _ACTIVATIONS or input_activation not in _ACTIVATIONS:
            raise ValueError(f"unsupported activation {activation!r} / {input_activation!r}")
        segment, offset, count = self.resolve(mod)
        layer = segment.layer
        if hasattr(layer, "project"):
            y = layer.project(x, conv=conv, components=components, activation=activation, norm=norm,
                              input_activation=input_activation)
        else:
            y = _unfused(layer, x, conv, activation, norm, input_activation)
        if count == segment.out_features:
            return y
        rows = slice(offset, offset + count)
        return y[:, rows] if conv else y[..., rows]


def _unfused(layer, x: Tensor, conv: bool, activation: str, norm, input_activation: str) -> Tensor:
    """The provider semantics around a layer object that has linear() only."""
    z = x.transpose(1, 2) if conv else x
    if norm is not None:
        z = F.layer_norm(z, norm.normalized_shape, norm.weight, norm.bias, norm.eps)
    if input_activation == "silu":
        z = F.silu(z)
    y = layer.linear(z)
    if activation == "silu":
        y = F.silu(y)
    return y.transpose(1, 2) if conv else y


class PartCount:
    """A provider wrapper that runs every call at `n` activation parts (whatever `components` the caller passes).
    Reads of other attributes and writes other than `provider` / `n` go to the wrapped provider
    (kk/binary/provider.py:185-209)."""

    _OWN = frozenset(("provider", "n"))

    def __init__(self, provider, n: int):
        if n not in (1, 2, 3):
            raise ValueError("n must be 1, 2 or 3")
        self.__dict__.update(provider=provider, n=n)

    def __call__(self, x, mod, conv=False, components=3, activation="", norm=None, config=None, input_activation=""):
        return self.provider(x, mod, conv, self.n, activation, norm, config, input_activation)

    def __getattr__(self, name):
        return getattr(self.__dict__["provider"], name)

    def __setattr__(self, name, value):
        if name in PartCount._OWN:
            self.__dict__[name] = value
        else:
            setattr(self.provider, name, value)


def _unpack_item(item) -> tuple:
    """(codes, scale, bias, kind, in_features) from a layer item (codes, scale, bias, kind[, in_features])."""
    codes, scale, bias, kind = item[:4]
    return codes, scale, bias, kind, (item[4] if len(item) > 4 else 8 * codes.shape[1])


def prepare_table(layers: dict, layer_cls, device="cuda", *, fuse_qkv: bool = True):
    """(RowSpace, {name: module}) from {name: (codes, scale, bias, kind[, in_features])} without NeMo. With fuse_qkv,
    the Q, K and V linears of one attention block (equal shapes, no bias) are prepared as one layer and their three
    modules are row slices of it."""
    space, modules = RowSpace(), {}
    fused = set()
    if fuse_qkv:
        blocks = sorted({name[: -len(QKV[0]) - 1] for name in layers if name.endswith("." + QKV[0])})
        for block in blocks:
            names = [f"{block}.{member}" for member in QKV]
            if not all(name in layers for name in names):
                continue
            items = [_unpack_item(layers[name]) for name in names]
            if len({tuple(codes.shape) for codes, *_ in items}) != 1 or \
                    any(bias is not None or kind != "linear" for _, _, bias, kind, _ in items):
                raise ValueError(f"{block}: Q/K/V must be equal-shape bias-free linear layers")
            n, k = items[0][0].shape[0], items[0][4]
            codes = torch.cat([item[0] for item in items])
            scales = torch.cat([item[1] for item in items])
            segment = space.allocate(f"{block}.qkv", layer_cls.prepare(codes, scales, None, k, device), "linear",
                                     3 * n, k, names)
            for i, name in enumerate(names):
                modules[name] = BinaryLinear(segment, i * n, n, scales[i * n:(i + 1) * n])
            fused.update(names)
    for name, item in layers.items():
        if name in fused:
            continue
        codes, scale, bias, kind, k = _unpack_item(item)
        segment = space.allocate(name, layer_cls.prepare(codes, scale, bias, k, device), kind, codes.shape[0], k)
        cls = BinaryPointwiseConv1d if kind == "conv" else BinaryLinear
        modules[name] = cls(segment, 0, codes.shape[0], scale, bias)
    return space, modules


def load_binary_model(directory, manifest: dict, layer_cls, device="cuda", *, fuse_qkv: bool = True):
    """(NeMo model on `device`, RowSpace) from a validated parakeet-binary-v1 export: the 264 quantized modules
    replaced by row views of prepared 1-bit layers, every other tensor loaded as FP32. Needs nemo_toolkit
    (RuntimeError from formats.build_nemo without it)."""
    from safetensors.torch import load_file

    from kea_kernels import formats
    directory = Path(directory)
    model = formats.build_nemo(manifest, directory)
    tensors = load_file(directory / manifest["file"])
    layers = {}
    for name, info in manifest["quantized_layers"].items():
        kind = "conv" if info["kind"] == "pointwise_conv1d" else "linear"
        bias = tensors.pop(f"{name}.bias") if info["bias"] else None
        layers[name] = (tensors.pop(f"{name}.codes"), tensors.pop(f"{name}.scale"), bias, kind, info["shape"][1])
    space, modules = prepare_table(layers, layer_cls, torch.device(device), fuse_qkv=fuse_qkv)
    for name, module in modules.items():
        if tuple(model.get_submodule(name).weight.shape[:2]) != (module.out_features, module.in_features):
            raise ValueError(f"invalid shape for {name}")
        model.set_submodule(name, module)
    model.load_state_dict({key: value.float() if value.is_floating_point() else value
                           for key, value in tensors.items()}, strict=True)
    return model.to(device=torch.device(device)).eval(), space


def module_names(model) -> dict:
    """{id(module): qualified name} of every module of `model`."""
    return {id(module): name for name, module in model.named_modules()}
