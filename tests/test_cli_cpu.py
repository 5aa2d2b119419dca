"""The package-level API and the `python -m kea_kernels` command line as a drop-in (kk/__main__.py:13-51,
kk/model.py:86-114, :194-204, :246-265): arguments, the order of the load-time checks, the error lines and the exit
codes. Transcription itself needs nemo_toolkit (absent here), so every run ends in an error line; which one, and
in what order the checks reject a bad input, is what these tests pin."""
from __future__ import annotations

import json
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import kea_kernels
from kea_kernels import __main__ as cli
from kea_kernels import formats, model
from test_api_cpu import write_fake_export

ROOT = Path(__file__).resolve().parents[1]


def _run(argv, capsys):
    code = cli.main(argv)
    return code, capsys.readouterr()


def test_arguments_and_usage_errors(capsys):
    with pytest.raises(SystemExit) as e:
        cli.main([])
    assert e.value.code == 2
    args = cli.parser().parse_args(["m", "a.wav", "b.wav", "--mode", "x2", "--tokens", "--no-verify"])
    assert (args.model, args.audio, args.mode, args.device, args.tokens, args.no_verify) == \
        ("m", ["a.wav", "b.wav"], "x2", "cuda", True, True)


def test_missing_directory_is_an_error_line(tmp_path, capsys):
    code, out = _run([str(tmp_path / "nope"), "clip.wav"], capsys)
    assert code == 1 and out.out == ""
    assert out.err.startswith("error: ") and "manifest.json" in out.err


def test_mode_is_checked_before_the_export(tmp_path, capsys):
    d = write_fake_export(tmp_path / "b", "binary")
    (d / formats.FILE).write_bytes(b"corrupt")  # the export check would fail too: the mode error comes first
    code, out = _run([str(d), "clip.wav", "--mode", "compact"], capsys)
    assert code == 1 and "kea-b supports modes ('x2', 'x3', 'x1'), got 'compact'" in out.err
    code, out = _run([str(d), "clip.wav"], capsys)
    assert code == 1 and "does not match the manifest SHA-256" in out.err


def test_export_is_checked_before_the_device(tmp_path, capsys):
    d = write_fake_export(tmp_path / "t", "ternary")
    code, out = _run([str(d), "clip.wav", "--device", "cpu"], capsys)
    assert code == 1 and "AMD MI355X GPUs only" in out.err
    manifest = json.loads((d / formats.MANIFEST).read_text())
    manifest["quantized_layers"].popitem()
    (d / formats.MANIFEST).write_text(json.dumps(manifest))
    code, out = _run([str(d), "clip.wav", "--device", "cpu", "--no-verify"], capsys)
    assert code == 1 and "expected the 264 Parakeet quantized layers" in out.err


def test_valid_export_ends_at_the_device_or_nemo(tmp_path, capsys):
    d = write_fake_export(tmp_path / "b01", "binary", extra={"keab": {"v": 1}})
    assert formats.describe(d).name == "kea-b-0.1"
    code, out = _run([str(d), "clip.wav"], capsys)
    assert code == 1 and out.err.startswith("error: ")
    # without a gfx950 GPU the device check rejects; with one, building the NeMo model does
    assert ("no ROCm GPU" in out.err) or ("gfx950" in out.err) or ("nemo_toolkit" in out.err)


def test_api_surface_and_clip_handling(tmp_path):
    assert set(kea_kernels.__all__) >= {"Model", "Transcript", "load", "transcribe", "close", "decoder_graphs_mode"}
    assert kea_kernels.load is model.load and kea_kernels.Transcript is model.Transcript
    with pytest.raises(ValueError, match="supports modes"):
        kea_kernels.load(write_fake_export(tmp_path / "t", "ternary"), mode="x1")
    # only None means "the model's own mode" (kk/model.py:92): an empty mode is a bad mode, not the default
    with pytest.raises(ValueError, match="supports modes"):
        kea_kernels.load(write_fake_export(tmp_path / "b", "binary"), mode="")
    with pytest.raises(ValueError, match="AMD MI355X GPUs only"):
        model.check_device("cpu")
    short = model.as_clip(np.ones(100, dtype=np.float64))
    assert short.dtype == np.float32 and short.shape == (model.MIN_DECODE_SAMPLES,) and short[100:].sum() == 0
    assert model.as_clip(torch.zeros(1000)).shape == (1000,)
    with pytest.raises(ValueError, match="1-D mono"):
        model.as_clip(np.zeros((2, 10)))


class _Featurizer:
    dither, pad_to = 1e-5, 16


class _Nemo:
    class preprocessor:
        featurizer = _Featurizer()


def test_closed_model_and_idempotent_close():
    calls = []
    featurizer = _Nemo.preprocessor.featurizer
    featurizer.dither = 0.5
    undo = [lambda: calls.append("first"), model._override_featurizer(featurizer), lambda: calls.append("last")]
    assert featurizer.dither == 0.0 and featurizer.pad_to == 0
    m = model.Model(_Nemo(), "kea-b", "binary", "x2", "/x", torch.device("cpu"), undo)
    with m:
        pass
    assert m.closed and calls == ["last", "first"] and featurizer.dither == 0.5
    m.close()
    assert calls == ["last", "first"]
    with pytest.raises(ValueError, match="closed"):
        kea_kernels.transcribe(m, np.zeros(480, np.float32))


def test_output_lines():
    r = model.Transcript("hello world", [5, 6], [0, 3])
    m = type("M", (), {"name": "kea-b", "mode": "x2"})()
    assert cli.line("a.wav", r, m, tokens=False, many=False) == "hello world"
    assert cli.line("a.wav", r, m, tokens=False, many=True) == "a.wav\thello world"
    assert json.loads(cli.line("a.wav", r, m, tokens=True, many=False)) == {
        "audio": "a.wav", "text": "hello world", "tokens": [5, 6], "timestamps": [0, 3], "model": "kea-b",
        "mode": "x2"}


def test_module_entry_point(tmp_path):
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([str(ROOT / "kea-kernels_amd"), str(ROOT)]))
    p = subprocess.run([sys.executable, "-m", "kea_kernels", str(tmp_path / "missing"), "x.wav"], env=env,
                       capture_output=True, text=True, timeout=300)
    assert p.returncode == 1 and p.stderr.startswith("error: ") and p.stdout == ""
