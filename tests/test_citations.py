"""Every `kk/<file>:<a>-<b>` citation in the library, its C headers and the tests names lines that exist in the
reference file it cites (kk/ = the reference's src/kea_kernels/). Reads the reference's sources as text; skipped where
the reference tree is absent (the GPU box)."""
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
REF = Path("/root/reference")
CITE = re.compile(r"\b(kk/[\w/]+\.py|tests/test_[\w]+\.py)((?::\d+(?:-\d+)?)(?:,\s*:?\d+(?:-\d+)?)*)")


def _sources():
    for sub in ("include", "kea-kernels_amd", "oracle", "tests"):
        for path in sorted((ROOT / sub).rglob("*")):
            if path.is_file() and path.suffix in (".py", ".h", ".hip", ".cpp", ".c") and "_build" not in path.parts:
                yield path


@pytest.mark.skipif(not REF.is_dir(), reason="the reference tree is not present on this machine")
def test_every_citation_lies_inside_its_file():
    bad = []
    for path in _sources():
        for ln, line in enumerate(path.read_text(errors="ignore").splitlines(), 1):
            for m in CITE.finditer(line):
                rel = m.group(1)
                target = REF / "src" / "kea_kernels" / rel[3:] if rel.startswith("kk/") else REF / rel
                if not target.is_file():
                    if not rel.startswith("kk/") and (ROOT / rel).is_file():
                        continue  # one of this build's own tests
                    bad.append(f"{path.relative_to(ROOT)}:{ln}: no file {rel}")
                    continue
                lines = len(target.read_text(errors="ignore").splitlines())
                for lo, hi in re.findall(r"(\d+)(?:-(\d+))?", m.group(2)):
                    if not 1 <= int(lo) <= int(hi or lo) <= lines:
                        bad.append(f"{path.relative_to(ROOT)}:{ln}: {rel}:{lo}-{hi or lo} (file has {lines} lines)")
    assert not bad, "\n".join(bad)
