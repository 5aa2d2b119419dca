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

import hashlib
import json
import math
import re
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

@dataclass(frozen=True)
class ModelDir:
    """What a directory holds: the export the kernels read and its kind."""
    name: str            # "kea-b-0.1", "kea-b" or "kea-t"
    kind: str            # "binary" or "ternary"
    export: Path         # the parakeet-*-v1 export directory
    default_mode: str


def read_manifest(directory: Path) -> dict:
    path = Path(directory) / MANIFEST
    if not path.is_file():
        raise ValueError(f"{directory}: no {MANIFEST} (expected a downloaded Kea-B or Kea-T model directory)")
    return json.loads(path.read_text())


def describe(directory) -> ModelDir:
    """Which model `directory` holds: a Kea-B 0.1 bundle, a Kea-B or Kea-T export, or an export inside a bundle."""
    directory = Path(directory).expanduser().resolve()
    manifest = read_manifest(directory)
    fmt = manifest.get("format")
    if fmt == BUNDLE_FORMAT:
        compat = directory / COMPAT_DIR
        if not (compat / MANIFEST).is_file():
            raise ValueError(f"{directory}: a {BUNDLE_FORMAT} bundle without its {COMPAT_DIR}/ export; download the "
                             "whole repository")
        inner = describe(compat)
        if inner.kind != "binary":
            raise ValueError(f"{compat}: expected a {BINARY_FORMAT} export")
        recorded = ((read_manifest(compat).get("extra") or {}).get("keab") or {}).get("bundle_sha256")
        if recorded != manifest.get("sha256"):
            raise ValueError(f"{compat}: its manifest does not record this directory's bundle")
        return inner
    if fmt == BINARY_FORMAT:
        if (manifest.get("extra") or {}).get("keab"):
            return ModelDir("kea-b-0.1", "binary", directory, "x1")
        return ModelDir("kea-b", "binary", directory, "x2")
    if fmt == TERNARY_FORMAT:
        return ModelDir("kea-t", "ternary", directory, "x2")
    raise ValueError(f"{directory}: unsupported format {fmt!r} (expected {BINARY_FORMAT}, {TERNARY_FORMAT} or "
                     f"{BUNDLE_FORMAT})")


def check_export(directory, kind: str, *, verify_hashes: bool = True) -> dict:
    """The manifest of an intact parakeet-binary-v1 / parakeet-ternary-v1 export of the 264 Parakeet layers.

    Checks the format (manifest and safetensors metadata), every listed file's SHA-256 (unless verify_hashes is
    False), the 264 layer names and kinds, and each layer's codes / scale / bias dtype and shape without loading the
    tensors. ValueError otherwise (kk/formats.py:130-173)."""
    from safetensors import safe_open
    directory = Path(directory)
    manifest = read_manifest(directory)
    fmt = {"binary": BINARY_FORMAT, "ternary": TERNARY_FORMAT}[kind]
    if manifest.get("format") != fmt:
        raise ValueError(f"{directory}: export format {manifest.get('format')!r}, expected {fmt!r}")
    files = manifest.get("files", {})
    if manifest.get("file") != FILE or FILE not in files:
        raise ValueError(f"{directory}: manifest does not list {FILE}")
    if verify_hashes:
        for rel, digest in files.items():
            path = directory / rel
            if not path.is_file() or sha256_file(path) != digest:
                raise ValueError(f"{path} does not match the manifest SHA-256")
    if (manifest.get("config") or {}).get("target") != MODEL_TARGET:
        raise ValueError(f"{directory}: unexpected model target {(manifest.get('config') or {}).get('target')!r}")
    layers = manifest.get("quantized_layers") or {}
    if len(layers) != EXPECTED_MODULES or not all(QUANTIZED_PATTERN.fullmatch(name) for name in layers):
        raise ValueError(f"{directory}: expected the {EXPECTED_MODULES} Parakeet quantized layers, got {len(layers)}")
    per_byte = 8 if kind == "binary" else 4
    with safe_open(directory / FILE, framework="pt") as f:
        if (f.metadata() or {}).get("format") != fmt:
            raise ValueError(f"{directory}: safetensors metadata format is not {fmt!r}")
        keys = set(f.keys())
        for name, info in layers.items():
            if info.get("kind") not in ("linear", "pointwise_conv1d"):
                raise ValueError(f"{name}: unknown kind {info.get('kind')!r}")
            n, k = info["shape"]
            if f"{name}.weight" in keys:
                raise ValueError(f"{name}: dense weight present in a quantized export")
            codes, scale = f.get_slice(f"{name}.codes"), f.get_slice(f"{name}.scale")
            width = math.ceil(k / per_byte)
            if codes.get_dtype() != "U8" or codes.get_shape() != [n, width]:
                raise ValueError(f"{name}: codes must be uint8 [{n}, {width}]")
            if scale.get_dtype() != "F32" or scale.get_shape() != [n]:
                raise ValueError(f"{name}: scale must be FP32 [{n}]")
            if bool(info.get("bias")) != (f"{name}.bias" in keys):
                raise ValueError(f"{name}: bias presence differs from the manifest")
    return manifest


def build_nemo(manifest: dict, directory: Path):
    """An FP32 NeMo EncDecRNNTBPEModel from the manifest's config (needs nemo_toolkit, which this image lacks)."""
    try:
        from nemo.collections.asr.models import EncDecRNNTBPEModel
        from omegaconf import OmegaConf, open_dict
    except ImportError as exc:
        raise RuntimeError("building the NeMo model needs nemo_toolkit[asr] and omegaconf, which are not "
                           "installed") from exc
    directory = Path(directory)
    cfg = OmegaConf.create(manifest["config"])
    with open_dict(cfg):
        cfg.tokenizer.dir = str(directory / TOKENIZER_DIR)
        for key, filename in TOKENIZER_FILES.items():
            cfg.tokenizer[key] = str(directory / TOKENIZER_DIR / filename)
        for ds in ("train_ds", "validation_ds", "test_ds"):
            if ds in cfg:
                cfg[ds] = None
    return EncDecRNNTBPEModel(cfg=cfg)
