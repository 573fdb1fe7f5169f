"""Builds libspissa_hip.so (the gfx950 attention path behind include/spissa_hip.h).

Every .hip file under csrc/ is compiled with hipcc for gfx950 into _build/,
then linked in-tree into spissa_amd/_lib/libspissa_hip.so so that the library
travels with the source tree. Packed-FP32 instruction selection is disabled
for all device code.

Usage: python -m spissa_amd.build [-v]
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIBDIR = PKG / "_lib"
LIB = LIBDIR / "libspissa_hip.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{PKG.parent / 'include'}",
]


# Per-source additions. prefill.hip keeps MFMA results in VGPRs: its score
# accumulators feed VALU code, and the AGPR form round-trips them.
EXTRA = {
    "prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}

# The link line: flags before the objects, libraries after them.
LINK = [f"--offload-arch={ARCH}", "-shared", "-fPIC"]
LINK_LIBS = ["-lpthread"]


def _compile(src: Path, verbose: bool) -> Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *COMMON, *EXTRA.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    warn = "\n".join(
        line for line in res.stderr.splitlines() if "packed-fp32-ops" not in line and line.strip()
    )
    if verbose and warn:
        print(warn, flush=True)
    return obj


def build(verbose: bool = False) -> Path:
    """Compiles every HIP source and links the shared library; returns its path."""
    OBJ.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, *LINK, "-o", str(tmp), *map(str, objs), *LINK_LIBS]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
