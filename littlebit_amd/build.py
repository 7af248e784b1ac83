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
import tempfile
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
SRC = PKG_DIR / "csrc" / "littlebit_amd.hip"
INCLUDE_DIR = REPO_DIR / "include"
LIB_DIR = PKG_DIR / "_lib"
LIB_PATH = LIB_DIR / "liblittlebit_amd.so"
# measurement programs bench.py runs (`--only handoff`, `--only issue`), not part of the library
PROBE_SRC = PKG_DIR / "csrc" / "handoff_probe.hip"
PROBE_PATH = LIB_DIR / "handoff_probe"
ISSUE_PROBE_SRC = PKG_DIR / "csrc" / "mfma_issue_probe.hip"
ISSUE_PROBE_PATH = LIB_DIR / "mfma_issue_probe"
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


def inline_asm_instructions(asm: str) -> list:
    """Instructions the device assembly holds inside inline asm blocks.

    The library's inline asm only pins values in registers or orders memory
    (empty blocks).  An instruction inside one is invisible to the compiler's
    hazard recognizer: a VALU result written there and read by an MFMA gets no
    wait states, which made MFMAs read stale operands on gfx950.  The build
    refuses device code that has any.
    """
    bad, func, inside = [], "?", False
    for line in asm.splitlines():
        if line and not line[0].isspace() and line.startswith("_Z") and ":" in line:
            func = line.split(":", 1)[0]
        s = line.strip()
        if s.startswith(";;#ASMSTART"):
            inside = True
        elif s.startswith(";;#ASMEND"):
            inside = False
        elif inside and s and not s.startswith(";"):
            bad.append(f"{func}: {s}")
    return bad


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)


def _finish(proc, what):
    out, err = proc.communicate()
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(line for line in err.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc ({what}) failed ({proc.returncode}):\n{err}\n{out}")
    return err


def build(verbose: bool = False) -> Path:
    """Compile the library and check its device code; returns its path.
    Always recompiles.  The device assembly (for the inline asm check) is
    compiled in parallel with the library."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    with tempfile.TemporaryDirectory() as td:
        asm_path = Path(td) / "device.s"
        lib_proc = _run([hipcc_path(), *HIP_FLAGS, "-I", str(INCLUDE_DIR), str(SRC), "-o", str(tmp)], verbose)
        flags = [f for f in HIP_FLAGS if f != "-shared"]
        asm_proc = _run([hipcc_path(), *flags, "--cuda-device-only", "-S", "-I", str(INCLUDE_DIR), str(SRC),
                         "-o", str(asm_path)], verbose)
        probe_tmp = PROBE_PATH.with_suffix(".tmp")
        probe_flags = [f for f in HIP_FLAGS if f not in ("-shared", "-fPIC")]
        probe_proc = _run([hipcc_path(), *probe_flags, str(PROBE_SRC), "-o", str(probe_tmp)], verbose)
        issue_tmp = ISSUE_PROBE_PATH.with_suffix(".tmp")
        issue_proc = _run([hipcc_path(), *probe_flags, str(ISSUE_PROBE_SRC), "-o", str(issue_tmp)], verbose)
        err = _finish(lib_proc, "library")
        _finish(asm_proc, "device assembly")
        _finish(probe_proc, "handoff probe")
        _finish(issue_proc, "MFMA issue probe")
        os.replace(probe_tmp, PROBE_PATH)
        os.replace(issue_tmp, ISSUE_PROBE_PATH)
        bad = inline_asm_instructions(asm_path.read_text())
    if bad:
        tmp.unlink(missing_ok=True)
        raise RuntimeError(f"{len(bad)} instructions inside inline asm, e.g.\n" + "\n".join(bad[:5]))
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
