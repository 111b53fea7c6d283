"""Build the gfx950 HIP library ``_lib/libgptqplus_hip.so`` in-tree with hipcc.

Usage: ``python -m gptq_plus_mp_quant_amd.build`` (or ``build()`` from Python).
Every translation unit is compiled for gfx950 only, without fp contraction (the column loop
must round like the reference's separate multiply / add / subtract), with packed-fp32 code
generation disabled, and linked into one shared object exporting the C ABI declared in
``include/gptqplus_hip.h``.
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
LIBDIR = PKG / "_lib"
LIB = LIBDIR / "libgptqplus_hip.so"
SOURCES = ["hessian.hip", "params.hip", "argsort.hip", "chol.hip", "terms.hip", "colloop.hip", "pack.hip",
           "blockgd.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("command failed: " + " ".join(cmd) + "\n" + res.stdout + res.stderr)
    return res


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link the shared library.  Always recompiles."""
    if not Path(HIPCC).exists() and shutil.which(HIPCC) is None:
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    objdir = LIBDIR / "obj"
    objdir.mkdir(parents=True, exist_ok=True)
    objs = []

    def compile_one(src):
        out = objdir / (Path(src).stem + ".o")
        _run([HIPCC, *FLAGS, "-I", str(CSRC), "-c", str(CSRC / src), "-o", str(out)])
        if verbose:
            print(f"compiled {src}", flush=True)
        return out

    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    if verbose:
        print(f"linked {LIB}", flush=True)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
