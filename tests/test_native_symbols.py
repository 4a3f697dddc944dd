"""The C-ABI libraries load (no GPU needed) and export every function their headers declare;
nothing else leaks from libpinfer.so (its version script exports pinfer_* only, like the
reference's engine/pkg/pinfer.map:3-8); the synthetic-model tools live in libpqtool.so."""
from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "nibblemac_amd" / "lib"


def declared(header: str, prefix: str) -> set[str]:
    text = (ROOT / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(rf"\b({prefix}\w+)\s*\(", text)) - {"PINFER_H"}


def exported(lib: Path) -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True,
                         check=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if " T " in ln}


@pytest.mark.parametrize("lib,header,prefix", [("libnmx.so", "nmx.h", "nmx_"),
                                               ("libpqtool.so", "pqtool.h", "pqt_"),
                                               ("libpinfer.so", "pinfer.h", "pinfer_")])
def test_headers_fully_exported(lib, header, prefix):
    path = LIB / lib
    assert path.exists(), f"{path} missing: build first"
    if not (ROOT / "include" / header).exists():
        pytest.skip(f"{header} not present")
    ctypes.CDLL(str(path))  # loads without a GPU
    missing = declared(header, prefix) - exported(path)
    assert not missing, f"{lib} lacks {sorted(missing)}"


def test_pinfer_exports_only_its_prefixes():
    syms = exported(LIB / "libpinfer.so")
    assert all(s.startswith("pinfer_") for s in syms), sorted(syms)[:20]
