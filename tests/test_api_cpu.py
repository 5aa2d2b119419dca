"""CPU contract tests of the host API: export formats and checks, the provider seam (Table, row handles, fused QKV,
BinaryProjection, PartCount), the ternary packed_t form and the native relayout. Restates the reference's CPU tests
(tests/test_formats.py:14-130, tests/test_kernels_cpu.py:12-17, :53-71) against this build's modules."""
from __future__ import annotations

import json
import math
from pathlib import Path

import pytest
import torch

from kea_kernels import formats
from kea_kernels.binary import bits, kernels, provider
from kea_kernels.ternary import runtime


def write_fake_export(directory: Path, kind: str, *, n: int = 8, k: int = 16, extra: dict | None = None) -> Path:
    """A structurally valid parakeet-*-v1 export: the 264 layer names at a tiny shape, one tokenizer file."""
    from safetensors.torch import save_file
    directory.mkdir(parents=True, exist_ok=True)
    per_byte = 8 if kind == "binary" else 4
    layers, tensors = {}, {}
    for layer in range(formats.LAYERS):
        for suffix in formats.PER_LAYER:
            name = f"encoder.layers.{layer}.{suffix}"
            layers[name] = {"kind": "pointwise_conv1d" if "pointwise" in suffix else "linear", "shape": [n, k],
                            "bias": False}
            tensors[f"{name}.codes"] = torch.zeros(n, math.ceil(k / per_byte), dtype=torch.uint8)
            tensors[f"{name}.scale"] = torch.ones(n, dtype=torch.float32)
    fmt = formats.BINARY_FORMAT if kind == "binary" else formats.TERNARY_FORMAT
    save_file(tensors, str(directory / formats.FILE), metadata={"format": fmt})
    (directory / "tokenizer").mkdir(exist_ok=True)
    (directory / "tokenizer" / "vocab.txt").write_text("a\n")
    files = {rel: formats.sha256_file(directory / rel) for rel in (formats.FILE, "tokenizer/vocab.txt")}
    manifest = {"format": fmt, "file": formats.FILE, "sha256": files[formats.FILE], "files": files,
                "config": {"target": formats.MODEL_TARGET}, "quantized_layers": layers, "extra": extra or {}}
    (directory / formats.MANIFEST).write_text(json.dumps(manifest))
    return directory


# --- export formats and checks -------------------------------------------------------------------------------------
def test_binary_codes_round_trip_and_layout():
    g = torch.Generator().manual_seed(5)
    signs = torch.where(torch.rand(5, 21, generator=g) < 0.5, -1, 1).to(torch.int8)
    packed = bits.pack_signs(signs)
    assert packed.dtype == torch.uint8 and packed.shape == (5, 3)
    assert torch.equal(bits.unpack_signs(packed, 21), signs)
    one = torch.full((1, 8), -1, dtype=torch.int8)
    one[0, 3] = 1
    assert bits.pack_signs(one).tolist() == [[1 << 3]]


def test_binary_codes_reject_tail_bits_and_bad_scales():
    codes = torch.zeros(2, 2, dtype=torch.uint8)
    codes[0, 1] = 0x80
    with pytest.raises(ValueError, match="tail"):
        bits.unpack_bits(codes, 12)
    with pytest.raises(ValueError, match="tail"):
        bits.validate_weights(codes, torch.ones(2), None, 12)
    good = torch.zeros(2, 2, dtype=torch.uint8)
    assert bits.validate_weights(good, torch.ones(2), None, 12) == (2, 12)
    with pytest.raises(ValueError, match="finite"):
        bits.validate_weights(good, torch.tensor([1.0, float("nan")]), None, 12)
    with pytest.raises(ValueError, match="codes must be"):
        bits.validate_weights(good, torch.ones(2), None, 20)


def test_ternary_codes_round_trip_and_reject_the_unused_pattern():
    g = torch.Generator().manual_seed(6)
    codes = torch.randint(-1, 2, (4, 13), dtype=torch.int8, generator=g)
    packed = formats.pack_ternary(codes)
    assert packed.shape == (4, 4)
    assert torch.equal(formats.unpack_ternary(packed, 13), codes)
    assert formats.pack_ternary(torch.tensor([[0, 1, -1, 1]], dtype=torch.int8)).tolist() == [[0b01_10_01_00]]
    with pytest.raises(ValueError):
        formats.unpack_ternary(torch.tensor([[0b11]], dtype=torch.uint8), 4)
    with pytest.raises(ValueError):
        formats.unpack_ternary(torch.tensor([[0b01_00_00_00]], dtype=torch.uint8), 3)


def test_sha256_file_matches_hashlib(tmp_path):
    import hashlib
    data = bytes(range(256)) * 9000  # spans several read chunks
    (tmp_path / "f").write_bytes(data)
    assert formats.sha256_file(tmp_path / "f", chunk=4096) == hashlib.sha256(data).hexdigest()


@pytest.mark.parametrize("kind", ["binary", "ternary"])
def test_check_export_accepts_an_intact_export(tmp_path, kind):
    d = write_fake_export(tmp_path / "m", kind)
    manifest = formats.check_export(d, kind)
    assert len(manifest["quantized_layers"]) == formats.EXPECTED_MODULES == 264


def test_check_export_refuses_the_other_format(tmp_path):
    d = write_fake_export(tmp_path / "m", "ternary")
    with pytest.raises(ValueError, match="expected 'parakeet-binary-v1'"):
        formats.check_export(d, "binary")


def test_check_export_refuses_a_modified_file(tmp_path):
    d = write_fake_export(tmp_path / "m", "binary")
    (d / "tokenizer" / "vocab.txt").write_text("b\n")
    with pytest.raises(ValueError, match="SHA-256"):
        formats.check_export(d, "binary")
    formats.check_export(d, "binary", verify_hashes=False)


def test_check_export_refuses_a_truncated_or_malformed_tensor_file(tmp_path):
    """The safetensors structure is checked without the SHA-256 too: a truncated data buffer, one with trailing
    bytes, overlapping or mis-sized data_offsets and a header that is not a JSON object are all ValueErrors."""
    import struct
    d = write_fake_export(tmp_path / "t", "binary")
    path = d / formats.FILE
    intact = path.read_bytes()
    (length,) = struct.unpack("<Q", intact[:8])
    header = json.loads(intact[8:8 + length])
    data = intact[8 + length:]

    def write(hdr, payload):
        text = json.dumps(hdr).encode()
        path.write_bytes(struct.pack("<Q", len(text)) + text + payload)

    for payload, match in ((data[:-1], "truncated or corrupt"), (data + b"\0", "truncated or corrupt")):
        path.write_bytes(intact[:8 + length] + payload)
        with pytest.raises(ValueError, match=match):
            formats.check_export(d, "binary", verify_hashes=False)
    name = next(k for k in header if k != "__metadata__")
    bad = json.loads(json.dumps(header))
    bad[name]["data_offsets"][1] += 1  # one byte more than its shape holds
    write(bad, data)
    with pytest.raises(ValueError, match="do not hold"):
        formats.check_export(d, "binary", verify_hashes=False)
    ranges = sorted((v["data_offsets"][0], k) for k, v in header.items() if k != "__metadata__")
    bad = json.loads(json.dumps(header))
    second = ranges[1][1]
    size = bad[second]["data_offsets"][1] - bad[second]["data_offsets"][0]
    bad[second]["data_offsets"] = [0, size]  # overlaps the first tensor
    write(bad, data)
    with pytest.raises(ValueError, match="starts at byte"):
        formats.check_export(d, "binary", verify_hashes=False)
    write([1, 2, 3], b"")
    with pytest.raises(ValueError, match="not a JSON object"):
        formats.check_export(d, "binary", verify_hashes=False)
    path.write_bytes(intact)
    formats.check_export(d, "binary", verify_hashes=False)


def test_check_export_refuses_missing_layers(tmp_path):
    d = write_fake_export(tmp_path / "m", "binary")
    manifest = json.loads((d / "manifest.json").read_text())
    manifest["quantized_layers"].pop(next(iter(manifest["quantized_layers"])))
    (d / "manifest.json").write_text(json.dumps(manifest))
    with pytest.raises(ValueError, match="264"):
        formats.check_export(d, "binary")


def test_check_export_refuses_wrong_code_shapes(tmp_path):
    d = write_fake_export(tmp_path / "m", "binary", n=8, k=16)
    manifest = json.loads((d / "manifest.json").read_text())
    for info in manifest["quantized_layers"].values():
        info["shape"] = [8, 32]
    (d / "manifest.json").write_text(json.dumps(manifest))
    with pytest.raises(ValueError, match="codes must be uint8"):
        formats.check_export(d, "binary", verify_hashes=False)


def test_describe_recognises_the_three_downloads(tmp_path):
    keab = write_fake_export(tmp_path / "kea-b", "binary")
    keat = write_fake_export(tmp_path / "kea-t", "ternary")
    root = tmp_path / "kea-b-0.1"
    write_fake_export(root / "compat", "binary", extra={"keab": {"bundle_sha256": "abc"}})
    (root / "manifest.json").write_text(json.dumps({"format": formats.BUNDLE_FORMAT, "sha256": "abc"}))
    assert (formats.describe(keab).name, formats.describe(keab).default_mode) == ("kea-b", "x2")
    assert (formats.describe(keat).name, formats.describe(keat).default_mode) == ("kea-t", "x2")
    info = formats.describe(root)
    assert (info.name, info.kind, info.default_mode, info.export) == ("kea-b-0.1", "binary", "x1",
                                                                       (root / "compat").resolve())
    assert formats.describe(root / "compat").default_mode == "x1"


def test_describe_refuses_a_bundle_without_its_export_or_mismatched(tmp_path):
    root = tmp_path / "kea-b-0.1"
    root.mkdir()
    (root / "manifest.json").write_text(json.dumps({"format": formats.BUNDLE_FORMAT, "sha256": "abc"}))
    with pytest.raises(ValueError, match="compat"):
        formats.describe(root)
    write_fake_export(root / "compat", "binary", extra={"keab": {"bundle_sha256": "other"}})
    with pytest.raises(ValueError, match="bundle"):
        formats.describe(root)


def test_describe_refuses_unknown_directories(tmp_path):
    with pytest.raises(ValueError, match="manifest.json"):
        formats.describe(tmp_path)
    (tmp_path / "manifest.json").write_text(json.dumps({"format": "something-else"}))
    with pytest.raises(ValueError, match="unsupported format"):
        formats.describe(tmp_path)


def test_nemo_loader_fails_loudly_without_nemo(tmp_path):
    d = write_fake_export(tmp_path / "m", "binary")
    manifest = formats.check_export(d, "binary")
    try:
        import nemo  # noqa: F401
    except ImportError:
        with pytest.raises(RuntimeError, match="NeMo"):
            formats.build_nemo(manifest, d)


# --- relayouts -----------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("n,k", [(8, 128), (24, 1024), (5, 300), (17, 33)])
def test_native_relayout_round_trips(n, k):
    g = torch.Generator().manual_seed(n * k)
    b = torch.randint(0, 2, (n, k), dtype=torch.uint8, generator=g)
    words = kernels.relayout(b)
    assert words.dtype == torch.int32 and words.numel() == kernels.native_words(n, k, 1)
    assert torch.equal(kernels.unlayout(words, n, k), b)


@pytest.mark.parametrize("n,k", [(4, 13), (16, 64), (33, 200)])
def test_ternary_packed_t_and_native_round_trip(n, k):
    g = torch.Generator().manual_seed(n + k)
    codes = formats.pack_ternary(torch.randint(-1, 2, (n, k), dtype=torch.int8, generator=g))
    packed_t = runtime.packed_t_from_codes(codes)
    assert packed_t.dtype == torch.int32 and packed_t.shape == (-(-k // 16), n)
    # closed form: code j of row r at bits 2 * (j % 16) of packed_t[j // 16, r]
    dense = formats.unpack_ternary(codes, k)
    for r, j in [(0, 0), (n - 1, k - 1), (n // 2, k // 2)]:
        field = (int(packed_t[j // 16, r]) >> (2 * (j % 16))) & 3
        assert {0: 0, 1: 1, 2: -1}[field] == int(dense[r, j])
    assert torch.equal(runtime.codes_from_packed_t(packed_t, k), codes)
    words = kernels.relayout_codes(codes, k, 2)
    assert torch.equal(kernels.unlayout_codes(words, n, k, 2), codes)


# --- provider seam -------------------------------------------------------------------------------------------------
class DenseLayer:
    """A CPU stand-in with the layer interface the provider needs: y = x @ (signs * scale)^T + bias (FP64)."""

    PARTS = 3
    prepared = []

    def __init__(self, codes, scale, bias, k):
        self.w = bits.dense_weight(codes, scale, k)
        self.bias = None if bias is None else bias.double()
        self.out_features, self.in_features = codes.shape[0], k

    @classmethod
    def prepare(cls, codes, scale, bias, k, device):
        layer = cls(codes, scale, bias, k)
        cls.prepared.append(layer)
        return layer

    def weight_bytes(self):
        return self.w.numel() // 8

    def linear(self, x):
        y = x.double() @ self.w.T
        return (y if self.bias is None else y + self.bias).float()

    def conv(self, x):
        return self.linear(x.transpose(1, 2)).transpose(1, 2)


def _layers(n=16, k=32, seed=0):
    g = torch.Generator().manual_seed(seed)
    out = {}
    for i, name in enumerate(["enc.0.self_attn.linear_q", "enc.0.self_attn.linear_k", "enc.0.self_attn.linear_v",
                              "enc.0.self_attn.linear_out", "enc.0.conv.pointwise_conv1"]):
        codes = bits.pack_signs(torch.where(torch.rand(n + 8 * ("conv" in name), k, generator=g) < .5, -1, 1).to(torch.int8))
        scale = torch.rand(codes.shape[0], generator=g) + 0.5
        bias = torch.randn(codes.shape[0], generator=g) if "out" in name else None
        out[name] = (codes, scale, bias, "conv" if "conv" in name else "linear", k)
    return out


def test_table_fuses_qkv_and_hands_out_row_handles():
    layers = _layers()
    table, modules = provider.prepare_table(layers, DenseLayer, "cpu")
    names = [s.name for s in table.segments]
    assert names[0] == "enc.0.self_attn.qkv" and table.segments[0].out_features == 48
    q, k, v = (modules[f"enc.0.self_attn.{x}"] for x in provider.QKV)
    assert torch.equal(torch.cat([q.packed_t, k.packed_t, v.packed_t], 1), torch.arange(48).view(1, 48))
    assert table.locate(16, 16) == (table.segments[0], 16)
    assert table.locate(0, 48) == (table.segments[0], 0)
    assert table.locate(48, 16) == (table.segments[1], 0)
    with pytest.raises(ValueError, match="crosses"):
        table.locate(40, 16)
    with pytest.raises(KeyError):
        table.locate(10_000, 1)
    assert all(not isinstance(getattr(m, "packed_t"), torch.nn.Parameter) for m in modules.values())
    assert "packed_t" not in q.state_dict()


def test_binary_projection_resolves_members_and_fused_handles():
    layers = _layers(seed=1)
    table, modules = provider.prepare_table(layers, DenseLayer, "cpu")
    proj = provider.BinaryProjection(table)
    x = torch.randn(2, 5, 32)
    q, k, v = (modules[f"enc.0.self_attn.{x}"] for x in provider.QKV)
    fused = type("Fused", (), {"packed_t": torch.cat([q.packed_t, k.packed_t, v.packed_t], 1)})()
    y = proj(x, fused)
    assert y.shape == (2, 5, 48)
    for i, mod in enumerate((q, k, v)):
        part = proj(x, mod)
        assert torch.equal(part, y[..., 16 * i:16 * (i + 1)])
        assert torch.equal(mod(x), part)  # module forward: the layer's linear, sliced
    dense = layers["enc.0.self_attn.linear_q"]
    ref = x.double() @ bits.dense_weight(dense[0], dense[1], 32).T
    assert torch.allclose(proj(x, q).double(), ref, rtol=1e-6, atol=1e-5)
    conv = modules["enc.0.conv.pointwise_conv1"]
    xc = torch.randn(2, 32, 7)
    yc = proj(xc, conv, conv=True)
    assert yc.shape == (2, 24, 7)
    assert torch.equal(yc, conv(xc))
    with pytest.raises(ValueError):
        proj(x, q, activation="gelu")
    with pytest.raises(TypeError):
        proj(x, type("M", (), {"packed_t": torch.zeros(1, 3, dtype=torch.int32)})())


def test_binary_projection_unfused_norm_and_silu():
    layers = _layers(seed=2)
    table, modules = provider.prepare_table(layers, DenseLayer, "cpu")
    proj = provider.BinaryProjection(table)
    out = modules["enc.0.self_attn.linear_out"]
    norm = torch.nn.LayerNorm(32)
    x = torch.randn(1, 3, 32)
    y = proj(x, out, norm=norm, input_activation="silu", activation="silu")
    with torch.no_grad():
        ref = torch.nn.functional.silu(out(torch.nn.functional.silu(norm(x))))
    assert torch.allclose(y, ref, rtol=1e-5, atol=1e-5)


def test_part_count_overrides_components_and_forwards_writes():
    calls = []

    class Provider:
        defer_epilogue = False

        def __call__(self, x, mod, conv=False, components=3, activation="", norm=None, config=None,
                     input_activation=""):
            calls.append(components)
            return x

    inner = Provider()
    wrapped = provider.PartCount(inner, 2)
    wrapped(torch.zeros(1), None, components=3)
    assert calls == [2]
    wrapped.defer_epilogue = True
    assert inner.defer_epilogue is True and wrapped.n == 2
    assert wrapped.defer_epilogue is True
    with pytest.raises(ValueError):
        provider.PartCount(inner, 4)


def test_packed_linear_validates_like_the_reference():
    codes = formats.pack_ternary(torch.zeros(4, 8, dtype=torch.int8))
    with pytest.raises(ValueError, match="finite"):
        runtime.PackedLinear(codes, torch.tensor([1.0, 2.0, float("inf"), 1.0]), 8)
    with pytest.raises(ValueError, match="mode"):
        runtime.PackedLinear(codes, torch.ones(4), 8, mode="tf64")
    bad = codes.clone()
    bad[0, 0] = 0b11
    with pytest.raises(ValueError):
        runtime.PackedLinear(bad, torch.ones(4), 8)
    mod = runtime.PackedLinear(codes, torch.ones(4), 8, mode="x2")
    assert mod.parts == 2 and set(mod.state_dict()) == {"packed_t", "scale"}


def test_product_path_has_no_cpu_fallback():
    """The GEMM launchers refuse CPU tensors instead of computing on the host."""
    from kea_kernels import lowbit
    q = torch.zeros(1, 4, 16, dtype=torch.int8)
    qs = torch.ones(1, 4)
    words = torch.zeros(kernels.native_words(16, 16, 1), dtype=torch.int32)
    y = torch.empty(4, 16)
    with pytest.raises((RuntimeError, ValueError, OSError)):
        lowbit.gemm(1, q, qs, words, 16, 16, torch.ones(16), None, y)


def test_gemm_refuses_short_weight_and_scale_buffers():
    """The launcher checks, before any C call, that the weight words hold the whole native layout of an n x k
    matrix and that the weight scales cover every output column (and group): a short buffer would be read past its
    end by the kernel."""
    from kea_kernels import lowbit
    m, n, k = 4, 64, 256
    q = torch.zeros(1, m, k, dtype=torch.int8)
    qs = torch.ones(1, m, dtype=torch.float16)
    y = torch.empty(m, n, dtype=torch.float16)
    for wbits in (1, 2):
        words = torch.zeros(kernels.native_words(n, k, wbits), dtype=torch.int32)
        alpha = torch.ones(n, dtype=torch.float16)
        with pytest.raises(ValueError, match="native words"):
            lowbit.gemm(wbits, q, qs, words[:-1], n, k, alpha, None, y)
        with pytest.raises(ValueError, match="native words"):
            lowbit.gemm(wbits, q, qs, words.view(-1, 4).t(), n, k, alpha, None, y)  # not contiguous
        with pytest.raises(ValueError, match="weight scales"):
            lowbit.gemm(wbits, q, qs, words, n, k, alpha[:-1], None, y)
        with pytest.raises(ValueError, match="groups"):
            lowbit.gemm(wbits, q, qs, words, n, k, alpha, None, y, ws_group=128)  # needs [n, 2]
        slices = torch.empty(2, 1, m, n, dtype=torch.int32)
        with pytest.raises(ValueError, match="native words"):
            lowbit.gemm_slices(wbits, q, words[:-4], n, k, slices)
    with pytest.raises(ValueError, match="wbits"):
        lowbit.gemm(3, q, qs, words, n, k, alpha, None, y)


def test_quantize_refuses_rows_past_the_input_storage():
    """kea_quantize reads row r at x + (r // T) * XB + (r % T) * XT + kk * XK: the launcher refuses an addressing
    whose furthest element lies past x's storage (or negative strides) before any C call."""
    from kea_kernels import lowbit
    x = torch.zeros(2, 5, 64)  # B = 2, T = 5, K = 64
    rows = (x.stride(0), x.stride(1), x.stride(2), 5)
    with pytest.raises(ValueError, match="past the end"):
        lowbit.quantize(x, rows, 11, 64, 1)  # an 11th row
    with pytest.raises(ValueError, match="past the end"):
        lowbit.quantize(x, rows, 10, 65, 1)  # a 65th feature
    with pytest.raises(ValueError, match="past the end"):
        lowbit.quantize(x[1:], (320, 64, 1, 5), 6, 64, 1)  # the second batch's rows 0-4, then a missing batch
    with pytest.raises(ValueError, match="non-negative"):
        lowbit.quantize(x, (x.stride(0), -64, 1, 5), 10, 64, 1)
    # a view's storage offset counts: the second batch alone has room for 5 rows, not 6
    with pytest.raises(ValueError, match="past the end"):
        lowbit.quantize(x[1], (0, 64, 1, 6), 6, 64, 1)
