"""load / transcribe / close behind the reference's signatures (kk/model.py:34-272), on this build's GEMM path.

The loader follows the reference's order (kk/model.py:86-114): `formats.describe` names the model and its default
mode, the mode is checked against the model's modes, `formats.check_export` validates the export (SHA-256 unless
verify=False), the device is checked, and then the NeMo model is built with the 264 quantized linears on this
library's kernels (`provider.load_binary_model` with the part count of the mode, `ternary.runtime.load_packed`).
Building the NeMo model needs nemo_toolkit, which this build's image does not have: there `load` ends with the
RuntimeError of `formats.build_nemo` after every check that precedes it, so a caller sees the same errors, in the
same order, as with the reference. Transcription (NeMo's preprocessor and greedy TDT decoder around the encoder) is
the reference's and is not part of this build; `transcribe` runs it when a NeMo model was loaded.
"""
from __future__ import annotations

import contextlib
import os
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np
import torch

from kea_kernels import formats

SAMPLE_RATE = 16000
# Inputs shorter than 30 ms are zero-padded to 30 ms (kk/model.py:27-28).
MIN_DECODE_SAMPLES = 480
SUPPORTED_ARCH = "gfx950"


@dataclass
class Transcript:
    text: str
    tokens: list[int]        # SentencePiece token IDs
    timestamps: list[int]    # encoder frame of each token (80 ms per frame)


@dataclass
class Model:
    """A loaded model (kk/model.py:41-65): `nemo` is the NeMo EncDecRNNTBPEModel whose quantized linears run on this
    library's kernels. close() (or the context manager) releases what load() set up."""
    nemo: object
    name: str
    kind: str
    mode: str
    export: str
    device: torch.device
    _stack: contextlib.ExitStack = field(repr=False)
    _featurizer: dict = field(repr=False, default_factory=dict)
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
    """The GPU device, or ValueError: the kernels are built for gfx950 (MI355X) only (kk/model.py:68-83 checks SM120)."""
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("kea-kernels runs on AMD MI355X GPUs only (device must be 'cuda' or 'cuda:N' under ROCm)")
    if not torch.cuda.is_available() or torch.version.hip is None:
        raise ValueError("no ROCm GPU is available to PyTorch (no AMD driver or a torch build without ROCm)")
    if device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    arch = torch.cuda.get_device_properties(device).gcnArchName.split(":")[0]
    if arch != SUPPORTED_ARCH:
        name = torch.cuda.get_device_name(device)
        raise ValueError(f"this build targets AMD gfx950 (MI355X); {device} is {name} ({arch}). The kernels use "
                         "gfx950 instructions and tile tables, and no other GPU has been tested.")
    return device


def load(path, device="cuda", mode: str | None = None, *, verify: bool = True) -> Model:
    """Load a downloaded Kea-B 0.1, Kea-B or Kea-T directory onto `device` in `mode` (default: the model's own).

    verify: check the SHA-256 of every file the manifest lists. Raises ValueError for a bad directory, mode, export
    or device, and RuntimeError when nemo_toolkit is missing."""
    info = formats.describe(path)
    modes = formats.BINARY_MODES if info.kind == "binary" else formats.TERNARY_MODES
    mode = info.default_mode if mode is None else mode
    if mode not in modes:
        raise ValueError(f"{info.name} supports modes {modes}, got {mode!r}")
    manifest = formats.check_export(info.export, info.kind, verify_hashes=verify)
    device = check_device(device)
    torch.cuda.set_device(device)
    stack = contextlib.ExitStack()
    with torch.inference_mode():
        try:
            if info.kind == "binary":
                nemo = _load_binary(info.export, manifest, device, mode)
            else:
                nemo = _load_ternary(info.export, manifest, device, mode)
        except BaseException:
            stack.close()
            raise
        featurizer = nemo.preprocessor.featurizer
        saved = {k: getattr(featurizer, k) for k in ("dither", "pad_to")}
        featurizer.dither, featurizer.pad_to = 0.0, 0
        torch.cuda.synchronize(device)
    return Model(nemo, info.name, info.kind, mode, str(info.export), device, stack, saved)


def _load_binary(export: Path, manifest: dict, device, mode: str):
    """The 1-bit layers at the mode's part count: x1 / x2 through PartCount, x3 at the reference's three parts."""
    from kea_kernels.binary import provider as P
    from kea_kernels.binary.layer import Int8MmaLayer
    from kea_kernels.binary.layer_parts import LAYERS
    parts = int(mode[1])
    layer_cls = Int8MmaLayer if parts == 3 else LAYERS[parts]
    model, _table = P.load_binary_model(export, manifest, layer_cls, device)
    return model.eval()


def _load_ternary(export: Path, manifest: dict, device, mode: str):
    from kea_kernels.ternary.runtime import load_packed
    return load_packed(export, manifest, device).eval()


def close(model: Model) -> None:
    """Undo what load() set up. Idempotent."""
    if model.closed:
        return
    with torch.inference_mode():
        if torch.cuda.is_initialized():
            torch.cuda.synchronize(model.device)
        model._stack.close()
        for k, v in model._featurizer.items():
            setattr(model.nemo.preprocessor.featurizer, k, v)
    model.closed = True


# --- transcription ------------------------------------------------------------------------------------------------

def read_audio(path) -> np.ndarray:
    """float32 mono samples of a 16 kHz audio file; multichannel files are averaged to mono (kk/model.py:184-191)."""
    try:
        import soundfile
    except ImportError as exc:
        raise RuntimeError("reading audio files needs the soundfile package, which is not installed") from exc
    audio, rate = soundfile.read(str(path), dtype="float32", always_2d=True)
    if rate != SAMPLE_RATE:
        raise ValueError(f"{path}: {rate} Hz; the models take 16 kHz audio "
                         f"(convert with: ffmpeg -i {path} -ar 16000 -ac 1 out.wav)")
    return audio.mean(axis=1) if audio.shape[1] > 1 else audio[:, 0]


def as_clip(item) -> np.ndarray:
    """A path or a 1-D array / tensor of 16 kHz samples as float32, zero-padded to 30 ms (kk/model.py:194-204)."""
    if isinstance(item, (str, os.PathLike)):
        clip = read_audio(item)
    else:
        clip = item.detach().cpu().numpy() if isinstance(item, torch.Tensor) else np.asarray(item)
        if clip.ndim != 1:
            raise ValueError(f"in-memory audio must be 1-D mono 16 kHz samples, got shape {clip.shape}")
        clip = clip.astype(np.float32, copy=False)
    if len(clip) < MIN_DECODE_SAMPLES:
        clip = np.pad(clip, (0, MIN_DECODE_SAMPLES - len(clip)))
    return clip


def _transcribe_one(model: Model, clip: np.ndarray) -> Transcript:
    nemo = model.nemo
    audio = torch.from_numpy(clip).unsqueeze(0).to(model.device)
    length = torch.tensor([len(clip)], dtype=torch.long, device=model.device)
    enc, enc_len = nemo.forward(input_signal=audio, input_signal_length=length)
    hyps = nemo.decoding.rnnt_decoder_predictions_tensor(encoder_output=enc, encoded_lengths=enc_len,
                                                         return_hypotheses=True)
    h = (hyps[0] if isinstance(hyps, tuple) else hyps)[0]
    seq = getattr(h, "y_sequence", None)
    tokens = [int(t) for t in (seq.tolist() if hasattr(seq, "tolist") else (seq or []))]
    ts = getattr(h, "timestamp", None)
    stamps = [int(t) for t in ts.tolist()] if hasattr(ts, "tolist") else (
        list(ts) if isinstance(ts, list) and all(isinstance(t, int) for t in ts) else [])
    return Transcript(h.text if hasattr(h, "text") else str(h), tokens, stamps)


def transcribe(model: Model, audio, *, return_tokens: bool = False):
    """Greedy TDT transcripts at batch 1 (kk/model.py:246-265): one item or a list of items, each a path to a 16 kHz
    audio file or a 1-D float array / tensor; a str per item (a Transcript when return_tokens), a list for a list."""
    if model.closed:
        raise ValueError("the model is closed")
    single = not isinstance(audio, (list, tuple))
    items = [audio] if single else list(audio)
    out = []
    with torch.inference_mode(), torch.autocast(model.device.type, enabled=False):
        model.nemo.eval()
        for item in items:
            result = _transcribe_one(model, as_clip(item))
            out.append(result if return_tokens else result.text)
    return out[0] if single else out


def decoder_graphs_mode(model: Model) -> str:
    """The TDT decoder's graph mode in use, as NeMo reports it (kk/model.py:268-272)."""
    comp = model.nemo.decoding.decoding.decoding_computer
    return str(getattr(comp, "cuda_graphs_mode", None))
