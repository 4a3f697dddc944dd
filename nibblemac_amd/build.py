"""Build the native libraries of nibblemac_amd in-tree.

    python -m nibblemac_amd.build          # libnmx.so (HIP, gfx950), libpinfer.so, libpqtool.so

libnmx.so   hand-written HIP kernels for gfx950 behind the C ABI of include/nmx.h
libpinfer.so the C11 host engine exporting the pinfer_* API of include/pinfer.h; it calls the
             device only through libnmx.so
libpqtool.so seeded synthetic weights and the Q4K_G32 packer (include/pqtool.h), host only

Both land in nibblemac_amd/lib/. Every call recompiles (sources are few and hipcc
cross-compiles gfx950 without a GPU).
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
INCLUDE = ROOT / "include"
HIP_DIR = PKG / "csrc" / "hip"
HOST_DIR = PKG / "csrc" / "host"
TOOL_DIR = PKG / "csrc" / "tool"
LIB_DIR = PKG / "lib"
OBJ_DIR = PKG / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CC = os.environ.get("CC", "gcc")
ARCH = "gfx950"

# Device numerics: no contraction (the reference rounds every multiply and add separately
# except where it calls fmaf), IEEE fp32 denormals, correctly rounded divide / sqrt (the
# hipcc default, kept), and no packed-fp32 code generation. Kernel arguments preloaded into
# SGPRs (the leading pointer / integer arguments, up to 16 SGPRs; the code object keeps the
# loading prologue for firmware without preloading), so a kernel's first memory requests do
# not wait for a load from the argument segment.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall", "-Wno-unused-function", f"-I{INCLUDE}", f"-I{HIP_DIR}",
]
C_FLAGS = ["-O2", "-std=c11", "-ffp-contract=off", "-fPIC", "-Wall", "-Wextra",
           "-Wno-unused-parameter", f"-I{INCLUDE}", f"-I{HOST_DIR}", "-pthread"]


def _run(cmd: list[str]) -> None:
    p = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(ln for ln in p.stderr.splitlines() if "packed-fp32-ops" not in ln)
    if p.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build_nmx() -> Path:
    """Compile every csrc/hip/*.hip for gfx950 and link libnmx.so."""
    OBJ_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    srcs = sorted(HIP_DIR.glob("*.hip"))
    objs = [OBJ_DIR / (s.stem + ".o") for s in srcs]
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(lambda so: _run([HIPCC, *HIP_FLAGS, "-c", str(so[0]), "-o", str(so[1])]),
                    zip(srcs, objs)))
    out = LIB_DIR / "libnmx.so"
    tmp = out.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    tmp.replace(out)
    return out


def build_pinfer() -> Path | None:
    """Compile csrc/host/*.c (C11) into libpinfer.so linked against libnmx.so."""
    srcs = sorted(HOST_DIR.glob("*.c"))
    if not srcs:
        return None
    out = LIB_DIR / "libpinfer.so"
    tmp = out.with_suffix(".so.tmp")
    _run([CC, *C_FLAGS, "-shared", *map(str, srcs), f"-L{LIB_DIR}", "-lnmx",
          "-Wl,-rpath,$ORIGIN", f"-Wl,--version-script={HOST_DIR / 'pinfer.map'}",
          "-lm", "-o", str(tmp)])
    tmp.replace(out)
    return out


def build_pqtool() -> Path:
    """Compile csrc/tool/*.c (C11) into libpqtool.so (no device code)."""
    LIB_DIR.mkdir(exist_ok=True)
    out = LIB_DIR / "libpqtool.so"
    tmp = out.with_suffix(".so.tmp")
    _run([CC, *C_FLAGS, "-shared", *map(str, sorted(TOOL_DIR.glob("*.c"))), "-lm", "-o", str(tmp)])
    tmp.replace(out)
    return out


def build_all() -> list[Path]:
    outs = [build_nmx()]
    p = build_pinfer()
    if p:
        outs.append(p)
    outs.append(build_pqtool())
    return outs


if __name__ == "__main__":
    for path in build_all():
        print(path)
