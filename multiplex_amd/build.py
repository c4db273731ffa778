"""Builds ``multiplex_amd/libgdn.so`` (gfx950) with hipcc, in-tree.

Usage: ``python -m multiplex_amd.build`` (or ``build()`` from Python).  The
library links only the HIP runtime; it has no torch or Python dependency.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_PATH = PKG_DIR / "libgdn.so"
SOURCES = [
    "gdn_api.hip",
    "gdn_recurrent.hip",
    "gdn_prologue.hip",
    "gdn_chunk.hip",
    "gdn_epilogue.hip",
    "gdn_attention.hip",
    "gdn_linear.hip",
]
ARCH = "gfx950"

# Packed-FP32 VALU ops are disabled for all device code; hipcc -O3 would
# otherwise form v_pk_{add,mul,fma}_f32 from ordinary float code.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in ordinary VGPRs (no accumulator-register round trips)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
]


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libgdn.so)")


def build(verbose: bool = False, jobs: int = 4) -> Path:
    """Compiles every HIP source to an object, then links the shared library."""
    hipcc = hipcc_path()
    obj_dir = PKG_DIR / "_build"
    obj_dir.mkdir(exist_ok=True)
    procs = []
    objs = []
    for src in SOURCES:
        obj = obj_dir / (Path(src).stem + ".o")
        objs.append(obj)
        cmd = [hipcc, *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        if len(procs) >= jobs:
            _wait(procs.pop(0), verbose)
    for p in procs:
        _wait(p, verbose)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(link), flush=True)
    out = subprocess.run(link, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if out.returncode != 0:
        raise RuntimeError(f"link failed:\n{out.stdout}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def _wait(item, verbose):
    src, proc = item
    out, _ = proc.communicate()
    text = out.decode(errors="replace")
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{text}")
    if verbose and text.strip():
        print(text)


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
