"""Export formats the kernels read, their checks, and which model a directory holds (drop-in for kk/formats.py).

Two export formats, one directory each (`export.safetensors`, `manifest.json`, `tokenizer/`), as the reference
defines them (kk/formats.py:1-15):
  * "parakeet-binary-v1": every quantized layer as `<name>.codes` uint8 [N, ceil(K/8)] (1 bit per weight, see
    binary.bits) and `<name>.scale` FP32 [N];
  * "parakeet-ternary-v1": `<name>.codes` uint8 [N, ceil(K/4)] (2 bits per weight: 00 = 0, 01 = +1, 10 = -1, code k
    at bits 2 * (k % 4) of byte k // 4) and `<name>.scale` FP32 [N].
The Kea-B 0.1 download is an 8-bit bundle ("keab-8bit-v1") whose `compat/` directory is a binary export.
"""
from __future__ import annotations

import copy
import hashlib
import json
import math
import re
import struct
from dataclasses import dataclass
from pathlib import Path

import torch
from torch import Tensor

BINARY_FORMAT = "parakeet-binary-v1"
TERNARY_FORMAT = "parakeet-ternary-v1"
BUNDLE_FORMAT = "keab-8bit-v1"
FILE = "export.safetensors"
MANIFEST = "manifest.json"
COMPAT_DIR = "compat"
TOKENIZER_DIR = "tokenizer"
TOKENIZER_FILES = {"model_path": "tokenizer.model", "vocab_path": "vocab.txt", "spe_tokenizer_vocab": "tokenizer.vocab"}
MODEL_TARGET = "nemo.collections.asr.models.rnnt_bpe_models.EncDecRNNTBPEModel"

LAYERS = 24
PER_LAYER = ("feed_forward1.linear1", "feed_forward1.linear2", "feed_forward2.linear1", "feed_forward2.linear2",
             "self_attn.linear_q", "self_attn.linear_k", "self_attn.linear_v", "self_attn.linear_out",
             "self_attn.linear_pos", "conv.pointwise_conv1", "conv.pointwise_conv2")
EXPECTED_MODULES = LAYERS * len(PER_LAYER)  # 264 quantized linears
QUANTIZED_PATTERN = re.compile(
    r"encoder\.layers\.\d+\.(feed_forward[12]\.linear[12]|self_attn\.linear_(q|k|v|out|pos)|conv\.pointwise_conv[12])")

# Modes per export kind; the first is the kind's default.
BINARY_MODES = ("x2", "x3", "x1")
TERNARY_MODES = ("x2", "x3", "compact")

_FIELD_SHIFT = torch.tensor([0, 2, 4, 6], dtype=torch.int32)


def sha256_file(path: Path, chunk: int = 1 << 20) -> str:
    digest = hashlib.sha256()
    with open(path, "rb") as handle:
        while True:
            block = handle.read(chunk)
            if not block:
                break
            digest.update(block)
    return digest.hexdigest()


# --- 2-bit ternary codes ------------------------------------------------------------------------------------------

def pack_ternary(codes: Tensor) -> Tensor:
    """int8 [out, in] in {-1, 0, 1} -> uint8 [out, ceil(in/4)]; 0 -> 00, +1 -> 01, -1 -> 10, code k at bits 2(k % 4)."""
    if codes.dtype != torch.int8 or codes.dim() != 2 or bool(((codes < -1) | (codes > 1)).any()):
        raise ValueError("expected 2-D int8 codes in {-1, 0, 1}")
    rows, k = codes.shape
    width = math.ceil(k / 4)
    field = torch.zeros(rows, 4 * width, dtype=torch.int32, device=codes.device)
    field[:, :k] = codes.eq(1).to(torch.int32) + 2 * codes.eq(-1).to(torch.int32)
    shifted = field.view(rows, width, 4) << _FIELD_SHIFT.to(codes.device)
    return shifted.sum(dim=2).to(torch.uint8)  # disjoint bit fields: the sum is their OR


def unpack_ternary(packed: Tensor, in_features: int) -> Tensor:
    """Inverse of pack_ternary; the unused 11 pattern and nonzero tail codes raise ValueError."""
    width = math.ceil(in_features / 4)
    if packed.dtype != torch.uint8 or packed.dim() != 2 or packed.shape[1] != width:
        raise ValueError(f"expected uint8 [out, {width}], got {packed.dtype} {tuple(packed.shape)}")
    fields = ((packed.to(torch.int32).unsqueeze(-1) >> _FIELD_SHIFT.to(packed.device)) & 3).reshape(packed.shape[0], -1)
    if bool(fields.eq(3).any()) or bool(fields[:, in_features:].ne(0).any()):
        raise ValueError("invalid packed codes")
    fields = fields[:, :in_features]
    return (fields.eq(1).to(torch.int8) - fields.eq(2).to(torch.int8)).contiguous()


# --- exports ------------------------------------------------------------------------------------------------------
# What the checks keep from the reference (kk/formats.py:84-189): the format strings, the order in which an export
# is rejected (format, listed file, hashes, model target, layer names, per-layer tensors) and the message fragments
# callers match on. How they run is this module's own: a table of format handlers for describe(), a list of checks
# for check_export(), and the safetensors header parsed directly (no tensor is read).

@dataclass(frozen=True)
class ModelDir:
    """What a directory holds: the export the kernels read and its kind."""
    name: str            # "kea-b-0.1", "kea-b" or "kea-t"
    kind: str            # "binary" or "ternary"
    export: Path         # the parakeet-*-v1 export directory
    default_mode: str


@dataclass(frozen=True)
class _Layout:
    """One export format: its manifest / metadata string and how many weight codes a byte holds."""
    format: str
    codes_per_byte: int


_LAYOUTS = {"binary": _Layout(BINARY_FORMAT, 8), "ternary": _Layout(TERNARY_FORMAT, 4)}
_LAYER_KINDS = ("linear", "pointwise_conv1d")


def read_manifest(directory: Path) -> dict:
    path = Path(directory) / MANIFEST
    if not path.is_file():
        raise ValueError(f"{directory}: no {MANIFEST} (expected a downloaded Kea-B or Kea-T model directory)")
    return json.loads(path.read_text())


# bytes per element of the safetensors dtype strings
_ST_DTYPE_BYTES = {"BOOL": 1, "U8": 1, "I8": 1, "F8_E4M3": 1, "F8_E5M2": 1, "U16": 2, "I16": 2, "F16": 2, "BF16": 2,
                   "U32": 4, "I32": 4, "F32": 4, "U64": 8, "I64": 8, "F64": 8}


def safetensors_header(path: Path) -> dict:
    """The header of a safetensors file without reading any tensor: its first 8 bytes are the little-endian length of
    a UTF-8 JSON object mapping each tensor name to {"dtype", "shape", "data_offsets"}, plus "__metadata__".

    The header is checked against the file as a safetensors reader checks it before handing out tensors: a JSON
    object; every tensor's byte range [begin, end) relative to the data buffer holds exactly its elements; the ranges,
    in order, tile the buffer from 0 to its end with no gap or overlap; and the buffer ends where the file ends (a
    truncated or extended file is rejected here, also when no SHA-256 is checked)."""
    path = Path(path)
    with open(path, "rb") as handle:
        raw = handle.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path}: not a safetensors file")
        (length,) = struct.unpack("<Q", raw)
        if length > (64 << 20):
            raise ValueError(f"{path}: implausible safetensors header length {length}")
        text = handle.read(length)
    if len(text) != length:
        raise ValueError(f"{path}: truncated safetensors header")
    try:
        header = json.loads(text)
    except ValueError as exc:
        raise ValueError(f"{path}: unreadable safetensors header") from exc
    if not isinstance(header, dict):
        raise ValueError(f"{path}: the safetensors header is not a JSON object")
    data_bytes = path.stat().st_size - 8 - length
    ranges = []
    for name, info in header.items():
        if name == "__metadata__":
            if info is not None and not isinstance(info, dict):
                raise ValueError(f"{path}: __metadata__ is not a JSON object")
            continue
        if not isinstance(info, dict):
            raise ValueError(f"{path}: tensor {name!r} has no dtype/shape/data_offsets")
        dtype, shape, offsets = info.get("dtype"), info.get("shape"), info.get("data_offsets")
        if (dtype not in _ST_DTYPE_BYTES or not isinstance(shape, list)
                or not all(isinstance(d, int) and d >= 0 for d in shape)
                or not isinstance(offsets, list) or len(offsets) != 2
                or not all(isinstance(o, int) for o in offsets)):
            raise ValueError(f"{path}: tensor {name!r} has an invalid dtype, shape or data_offsets")
        begin, end = offsets
        count = 1
        for d in shape:
            count *= d
        if not 0 <= begin <= end or end - begin != count * _ST_DTYPE_BYTES[dtype]:
            raise ValueError(f"{path}: tensor {name!r}: data_offsets {offsets} do not hold a {dtype} {shape}")
        ranges.append((begin, end, name))
    position = 0
    for begin, end, name in sorted(ranges):
        if begin != position:
            raise ValueError(f"{path}: tensor {name!r} starts at byte {begin} of the data, expected {position}")
        position = end
    if position != data_bytes:
        raise ValueError(f"{path}: the tensors cover {position} data bytes but the file holds {data_bytes} "
                         "(truncated or corrupt)")
    return header


# describe(): one handler per manifest format

def _describe_bundle(directory: Path, manifest: dict) -> ModelDir:
    """Kea-B 0.1: an 8-bit bundle whose compat/ directory is a binary export recording the bundle's hash."""
    compat = directory / COMPAT_DIR
    if not (compat / MANIFEST).is_file():
        raise ValueError(f"{directory}: a {BUNDLE_FORMAT} bundle without its {COMPAT_DIR}/ export; download the "
                         "whole repository")
    inner = describe(compat)
    if inner.kind != "binary":
        raise ValueError(f"{compat}: expected a {BINARY_FORMAT} export")
    keab = (read_manifest(compat).get("extra") or {}).get("keab") or {}
    if keab.get("bundle_sha256") != manifest.get("sha256"):
        raise ValueError(f"{compat}: its manifest does not record this directory's bundle")
    return inner


def _describe_binary(directory: Path, manifest: dict) -> ModelDir:
    # the compat export of a Kea-B 0.1 bundle carries extra.keab; its default mode is one part
    if (manifest.get("extra") or {}).get("keab"):
        return ModelDir("kea-b-0.1", "binary", directory, "x1")
    return ModelDir("kea-b", "binary", directory, "x2")


def _describe_ternary(directory: Path, manifest: dict) -> ModelDir:
    return ModelDir("kea-t", "ternary", directory, "x2")


_DESCRIBE = {BUNDLE_FORMAT: _describe_bundle, BINARY_FORMAT: _describe_binary, TERNARY_FORMAT: _describe_ternary}


def describe(directory) -> ModelDir:
    """Which model `directory` holds: a Kea-B 0.1 bundle, a Kea-B or Kea-T export, or an export inside a bundle."""
    directory = Path(directory).expanduser().resolve()
    manifest = read_manifest(directory)
    handler = _DESCRIBE.get(manifest.get("format"))
    if handler is None:
        raise ValueError(f"{directory}: unsupported format {manifest.get('format')!r} (expected {BINARY_FORMAT}, "
                         f"{TERNARY_FORMAT} or {BUNDLE_FORMAT})")
    return handler(directory, manifest)


# check_export(): the checks, in the order a broken export is reported

def _check_format(directory, manifest, layout, verify):
    if manifest.get("format") != layout.format:
        raise ValueError(f"{directory}: export format {manifest.get('format')!r}, expected {layout.format!r}")


def _check_files(directory, manifest, layout, verify):
    files = manifest.get("files") or {}
    if manifest.get("file") != FILE or FILE not in files:
        raise ValueError(f"{directory}: manifest does not list {FILE}")
    if not verify:
        return
    for rel, digest in files.items():
        path = directory / rel
        if not path.is_file() or sha256_file(path) != digest:
            raise ValueError(f"{path} does not match the manifest SHA-256")


def _check_target(directory, manifest, layout, verify):
    target = (manifest.get("config") or {}).get("target")
    if target != MODEL_TARGET:
        raise ValueError(f"{directory}: unexpected model target {target!r}")


def _check_layer_names(directory, manifest, layout, verify):
    names = list((manifest.get("quantized_layers") or {}).keys())
    if len(names) != EXPECTED_MODULES or any(QUANTIZED_PATTERN.fullmatch(name) is None for name in names):
        raise ValueError(f"{directory}: expected the {EXPECTED_MODULES} Parakeet quantized layers, got {len(names)}")


def _check_tensors(directory, manifest, layout, verify):
    header = safetensors_header(directory / FILE)
    if (header.get("__metadata__") or {}).get("format") != layout.format:
        raise ValueError(f"{directory}: safetensors metadata format is not {layout.format!r}")
    for name, info in manifest["quantized_layers"].items():
        if info.get("kind") not in _LAYER_KINDS:
            raise ValueError(f"{name}: unknown kind {info.get('kind')!r}")
        n, k = info["shape"]
        if f"{name}.weight" in header:
            raise ValueError(f"{name}: dense weight present in a quantized export")
        width = -(-k // layout.codes_per_byte)
        codes, scale = header.get(f"{name}.codes") or {}, header.get(f"{name}.scale") or {}
        if codes.get("dtype") != "U8" or codes.get("shape") != [n, width]:
            raise ValueError(f"{name}: codes must be uint8 [{n}, {width}]")
        if scale.get("dtype") != "F32" or scale.get("shape") != [n]:
            raise ValueError(f"{name}: scale must be FP32 [{n}]")
        if bool(info.get("bias")) != (f"{name}.bias" in header):
            raise ValueError(f"{name}: bias presence differs from the manifest")


_EXPORT_CHECKS = (_check_format, _check_files, _check_target, _check_layer_names, _check_tensors)


def check_export(directory, kind: str, *, verify_hashes: bool = True) -> dict:
    """The manifest of an intact parakeet-binary-v1 / parakeet-ternary-v1 export of the 264 Parakeet layers.

    Runs, in order: the manifest's format, the listed export file and (unless verify_hashes is False) every listed
    file's SHA-256, the model target, the 264 layer names, and each layer's kind and codes / scale / bias dtypes and
    shapes as the safetensors header records them. ValueError at the first failure."""
    if kind not in _LAYOUTS:
        raise ValueError(f"unknown export kind {kind!r} (binary or ternary)")
    directory = Path(directory)
    manifest = read_manifest(directory)
    for check in _EXPORT_CHECKS:
        check(directory, manifest, _LAYOUTS[kind], verify_hashes)
    return manifest


def build_nemo(manifest: dict, directory: Path):
    """An FP32 NeMo EncDecRNNTBPEModel from the manifest's config, pointed at the export's own tokenizer files and
    with no datasets (needs nemo_toolkit[asr] and omegaconf; RuntimeError without them)."""
    try:
        from nemo.collections.asr.models import EncDecRNNTBPEModel
        from omegaconf import OmegaConf
    except ImportError as exc:
        raise RuntimeError("building the NeMo model needs nemo_toolkit[asr] and omegaconf, which are not "
                           "installed") from exc
    cfg = copy.deepcopy(manifest["config"])
    tokenizer_dir = Path(directory) / TOKENIZER_DIR
    cfg["tokenizer"] = {**(cfg.get("tokenizer") or {}), "dir": str(tokenizer_dir),
                        **{key: str(tokenizer_dir / name) for key, name in TOKENIZER_FILES.items()}}
    cfg.update({section: None for section in ("train_ds", "validation_ds", "test_ds") if section in cfg})
    return EncDecRNNTBPEModel(cfg=OmegaConf.create(cfg))
