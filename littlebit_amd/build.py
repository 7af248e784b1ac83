"""Compile the gfx950 HIP library in-tree with hipcc.

``python -m littlebit_amd.build`` (or ``__graft_entry__.build()``) writes
``littlebit_amd/_lib/liblittlebit_amd.so``.  hipcc cross-compiles, so this
runs on a machine without a GPU.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
SRC = PKG_DIR / "csrc" / "littlebit_amd.hip"
INCLUDE_DIR = REPO_DIR / "include"
LIB_DIR = PKG_DIR / "_lib"
LIB_PATH = LIB_DIR / "liblittlebit_amd.so"
ARCH = "gfx950"

# -packed-fp32-ops: keep hipcc from emitting packed fp32 VALU instructions.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc_path() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def build(verbose: bool = False) -> Path:
    """Compile the library; returns its path.  Always recompiles."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc_path(), *HIP_FLAGS, "-I", str(INCLUDE_DIR), str(SRC), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}\n{proc.stdout}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
