"""Compile the reference's AVX2/OpenMP CPU kernels into oracle/_ref/.

TEST INFRASTRUCTURE ONLY (the CPU baseline that bench.py times and a
cross-check of the oracle).  The source is compiled where it lies,
/root/reference/patches/littlebit_cpu_optimized.cpp, by one g++ command
against the ATen headers of the installed torch; nothing of the reference is
copied into this repository.  The reference builds the same file with
torch.utils.cpp_extension.load and -march=native (cpu_draft_model.py:85-94);
this recipe uses -mavx2 -mfma instead so that the library also runs on the
GPU box's host CPU.  The output, oracle/_ref/littlebit_cpu_ref.so, registers
torch.ops.littlebit_cpu_ops.* when loaded with torch.ops.load_library.

Run:  python oracle/build_ref.py       (needs /root/reference; a no-op without it)
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT_DIR = HERE / "_ref"
OUT = OUT_DIR / "littlebit_cpu_ref.so"
SRC = Path("/root/reference/patches/littlebit_cpu_optimized.cpp")


def build(verbose: bool = True) -> Path | None:
    if not SRC.exists():
        if verbose:
            print(f"[build_ref] {SRC} not present; skipping", flush=True)
        return None
    import torch
    import torch.utils.cpp_extension as ext

    OUT_DIR.mkdir(parents=True, exist_ok=True)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O3", "-mavx2", "-mfma", "-mf16c", "-fopenmp", "-std=c++17", "-fPIC", "-shared",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}"]
    for inc in ext.include_paths():
        cmd += ["-isystem", inc]
    cmd += [str(SRC), "-o", str(OUT) + ".tmp"]
    for lib in ext.library_paths():
        cmd += [f"-L{lib}", f"-Wl,-rpath,{lib}"]
    cmd += ["-lc10", "-ltorch_cpu", "-lgomp"]
    if verbose:
        print("[build_ref] " + " ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"g++ failed ({proc.returncode}):\n{proc.stderr[-4000:]}")
    os.replace(str(OUT) + ".tmp", OUT)
    return OUT


def load():
    """Load the built library (registers torch.ops.littlebit_cpu_ops)."""
    import torch

    if not OUT.exists():
        raise FileNotFoundError(f"{OUT} not built (python oracle/build_ref.py)")
    if not hasattr(torch.ops, "littlebit_cpu_ops") or not hasattr(torch.ops.littlebit_cpu_ops, "littlebit_linear"):
        torch.ops.load_library(str(OUT))
    return torch.ops.littlebit_cpu_ops


if __name__ == "__main__":
    path = build()
    print(f"[build_ref] {path}")
    sys.exit(0)
