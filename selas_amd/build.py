"""Builds libselas_amd.so (the gfx950 kernels behind include/selas_amd.h) in-tree with hipcc.

Run as ``python -m selas_amd.build``. Every source under ``selas_amd/csrc`` is
compiled to an object in ``selas_amd/_build`` (in parallel) and linked into
``selas_amd/libselas_amd.so`` next to this file.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libselas_amd.so"
SOURCES = ("errors.hip", "nf4_codec.hip", "int8_row_codec.hip", "nf4_linear.hip", "segments.hip", "attention.hip")
ARCH = "gfx950"

# Packed-fp32 instructions are switched off for all device code: hipcc still
# vectorises ordinary float code, only without the v_pk_*_f32 forms.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build selas_amd")


def _compile(src: Path, obj: Path, cc: str) -> None:
    cmd = [cc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr}")
    for line in r.stderr.splitlines():  # the host pass does not know the packed-fp32 feature: harmless
        if line.strip() and "packed-fp32-ops" not in line and "is not a recognized feature" not in line:
            print(line, file=sys.stderr)


def build(verbose: bool = True) -> Path:
    """Compiles every source and links the shared library; returns its path."""
    cc = hipcc()
    OBJ.mkdir(exist_ok=True)
    srcs = [CSRC / s for s in SOURCES]
    objs = [OBJ / (s.stem + ".o") for s in srcs]
    with ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 1)) as ex:
        list(ex.map(lambda so: _compile(so[0], so[1], cc), zip(srcs, objs)))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)  # atomic: a process that loaded the old library keeps its mapping
    if verbose:
        print(f"built {LIB} ({LIB.stat().st_size // 1024} KiB)")
    return LIB


if __name__ == "__main__":
    build()
