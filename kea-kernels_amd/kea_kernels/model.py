"""load / transcribe / close behind the reference's signatures (kk/model.py:34-272), on this build's GEMM path.

load() rejects a bad input at the same point as the reference (kk/model.py:86-114): the directory (describe), the
mode, the export (check_export, SHA-256 unless verify=False), the device, then the model. The model is NeMo's
EncDecRNNTBPEModel with the 264 quantized linears on this library's kernels; this build's image has no
nemo_toolkit, so here load() ends with formats.build_nemo's RuntimeError after every check before it. Transcription
(NeMo's preprocessor and greedy TDT decoder around the encoder) runs only where a NeMo model was loaded.
"""
from __future__ import annotations

import os
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np
import torch

from kea_kernels import formats

SAMPLE_RATE = 16000
MIN_DECODE_SAMPLES = 480     # 30 ms: shorter clips are zero-padded (kk/model.py:27-28)
SUPPORTED_ARCH = "gfx950"
_FEATURIZER_OVERRIDES = {"dither": 0.0, "pad_to": 0}  # deterministic features while a model is loaded


@dataclass
class Transcript:
    text: str
    tokens: list[int]        # SentencePiece token IDs
    timestamps: list[int]    # encoder frame of each token (80 ms per frame)


@dataclass
class Model:
    """A loaded model: `nemo` is the NeMo model whose quantized linears run on this library's kernels. close() (or
    leaving the context manager) runs `undo`, what load() registered to restore, latest first."""
    nemo: object
    name: str
    kind: str
    mode: str
    export: str
    device: torch.device
    undo: list = field(repr=False, default_factory=list)
    closed: bool = False

    def transcribe(self, audio, **kwargs):
        return transcribe(self, audio, **kwargs)

    def close(self) -> None:
        close(self)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        close(self)


def check_device(device) -> torch.device:
    """The ROCm GPU `device` as torch.device, or ValueError: the kernels are built for gfx950 (MI355X) only."""
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("kea-kernels runs on AMD MI355X GPUs only (device must be 'cuda' or 'cuda:N' under ROCm)")
    if not torch.cuda.is_available() or torch.version.hip is None:
        raise ValueError("no ROCm GPU is available to PyTorch (no AMD driver or a torch build without ROCm)")
    if device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    arch = torch.cuda.get_device_properties(device).gcnArchName.split(":")[0]
    if arch != SUPPORTED_ARCH:
        raise ValueError(f"this build targets AMD gfx950 (MI355X); {device} is {torch.cuda.get_device_name(device)} "
                         f"({arch}). The kernels use gfx950 instructions and tile tables, and no other GPU has been "
                         "tested.")
    return device


def _binary_nemo(export: Path, manifest: dict, device, mode: str):
    """1-bit layers at the mode's part count (x1, x2, x3)."""
    from kea_kernels.binary import provider
    from kea_kernels.binary.layer import Int8MmaLayer
    from kea_kernels.binary.layer_parts import LAYERS
    parts = int(mode[1])
    # three parts run on the full operator (its project() path), fewer on the P-part variants (kk/model.py:121-122)
    layer_cls = Int8MmaLayer if parts == 3 else LAYERS[parts]
    model, _space = provider.load_binary_model(export, manifest, layer_cls, device)
    return model


def _ternary_nemo(export: Path, manifest: dict, device, mode: str):
    from kea_kernels.ternary.runtime import load_packed
    return load_packed(export, manifest, device)


_BUILDERS = {"binary": _binary_nemo, "ternary": _ternary_nemo}


def load(path, device="cuda", mode: str | None = None, *, verify: bool = True) -> Model:
    """A downloaded Kea-B 0.1, Kea-B or Kea-T directory loaded onto `device` in `mode` (default: the model's own).

    verify: check the SHA-256 of every file the manifest lists. ValueError for a bad directory, mode, export or
    device; RuntimeError when nemo_toolkit is missing."""
    info = formats.describe(path)
    modes = formats.BINARY_MODES if info.kind == "binary" else formats.TERNARY_MODES
    mode = info.default_mode if mode is None else mode
    if mode not in modes:
        raise ValueError(f"{info.name} supports modes {modes}, got {mode!r}")
    manifest = formats.check_export(info.export, info.kind, verify_hashes=verify)
    device = check_device(device)
    torch.cuda.set_device(device)
    with torch.inference_mode():
        nemo = _BUILDERS[info.kind](info.export, manifest, device, mode).eval()
        undo = [_override_featurizer(nemo.preprocessor.featurizer)]
        torch.cuda.synchronize(device)
    return Model(nemo, info.name, info.kind, mode, str(info.export), device, undo)


def _override_featurizer(featurizer):
    """Sets the deterministic feature options and returns the callable that puts the previous values back."""
    saved = {key: getattr(featurizer, key) for key in _FEATURIZER_OVERRIDES}
    for key, value in _FEATURIZER_OVERRIDES.items():
        setattr(featurizer, key, value)
    return lambda: [setattr(featurizer, key, value) for key, value in saved.items()]


def close(model: Model) -> None:
    """Undo what load() set up. Idempotent."""
    if model.closed:
        return
    if torch.cuda.is_initialized():
        torch.cuda.synchronize(model.device)
    while model.undo:
        model.undo.pop()()
    model.closed = True


# --- audio --------------------------------------------------------------------------------------------------------

def read_audio(path) -> np.ndarray:
    """float32 mono samples of a 16 kHz audio file (channels averaged); needs the soundfile package."""
    try:
        import soundfile
    except ImportError as exc:
        raise RuntimeError("reading audio files needs the soundfile package, which is not installed") from exc
    samples, rate = soundfile.read(str(path), dtype="float32", always_2d=True)
    if rate != SAMPLE_RATE:
        raise ValueError(f"{path}: {rate} Hz; the models take 16 kHz audio "
                         f"(convert with: ffmpeg -i {path} -ar 16000 -ac 1 out.wav)")
    return samples.mean(axis=1, dtype=np.float32)


def as_clip(item) -> np.ndarray:
    """A path, or a 1-D array / tensor of 16 kHz samples, as float32 samples of at least 30 ms (zero-padded)."""
    if isinstance(item, (str, os.PathLike)):
        clip = read_audio(item)
    else:
        clip = np.asarray(item.detach().cpu() if isinstance(item, torch.Tensor) else item)
        if clip.ndim != 1:
            raise ValueError(f"in-memory audio must be 1-D mono 16 kHz samples, got shape {clip.shape}")
        clip = clip.astype(np.float32, copy=False)
    short = MIN_DECODE_SAMPLES - clip.shape[0]
    return np.concatenate([clip, np.zeros(short, np.float32)]) if short > 0 else clip


# --- transcription (NeMo's preprocessor and greedy TDT decoding around the encoder) ----------------------------------

def _ints(values) -> list[int]:
    if values is None:
        return []
    values = values.tolist() if hasattr(values, "tolist") else values
    return [int(v) for v in values] if all(isinstance(v, (int, float)) for v in values) else []


def _decode(model: Model, clip: np.ndarray) -> Transcript:
    nemo = model.nemo
    signal = torch.from_numpy(clip).unsqueeze(0).to(model.device)
    lengths = torch.tensor([clip.shape[0]], dtype=torch.long, device=model.device)
    encoded, encoded_lengths = nemo.forward(input_signal=signal, input_signal_length=lengths)
    out = nemo.decoding.rnnt_decoder_predictions_tensor(encoder_output=encoded, encoded_lengths=encoded_lengths,
                                                        return_hypotheses=True)
    hypothesis = (out[0] if isinstance(out, tuple) else out)[0]
    return Transcript(getattr(hypothesis, "text", str(hypothesis)), _ints(getattr(hypothesis, "y_sequence", None)),
                      _ints(getattr(hypothesis, "timestamp", None)))


def transcribe(model: Model, audio, *, return_tokens: bool = False):
    """Greedy TDT transcripts at batch 1: one item or a list of items (paths to 16 kHz audio files or 1-D sample
    arrays / tensors); a str per item (a Transcript with return_tokens), a list for a list."""
    if model.closed:
        raise ValueError("the model is closed")
    items = list(audio) if isinstance(audio, (list, tuple)) else [audio]
    with torch.inference_mode(), torch.autocast(model.device.type, enabled=False):
        model.nemo.eval()
        results = [_decode(model, as_clip(item)) for item in items]
    results = results if return_tokens else [r.text for r in results]
    return results if isinstance(audio, (list, tuple)) else results[0]


def decoder_graphs_mode(model: Model) -> str:
    """The TDT decoder's graph mode in use, as NeMo reports it."""
    computer = model.nemo.decoding.decoding.decoding_computer
    return str(getattr(computer, "cuda_graphs_mode", None))
