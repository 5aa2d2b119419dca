"""Shared test setup. GPU tests are marked `gpu` and skipped unless a gfx950 (MI355X) GPU is visible."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "kea-kernels_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X (gfx950) GPU; skipped elsewhere")


def gfx950() -> bool:
    import torch
    if not torch.cuda.is_available() or torch.version.hip is None:
        return False
    return torch.cuda.get_device_properties(0).gcnArchName.split(":")[0] == "gfx950"


def pytest_collection_modifyitems(config, items):
    if not any("gpu" in item.keywords for item in items) or gfx950():
        return
    skip = pytest.mark.skip(reason="needs an AMD MI355X (gfx950) GPU")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
