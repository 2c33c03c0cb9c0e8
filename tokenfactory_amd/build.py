"""Builds ``libtf_attn.so`` (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

Usage: ``python -m tokenfactory_amd.build`` (or ``__graft_entry__.build()``).
The library lands in ``tokenfactory_amd/_lib/`` next to the sources so that it
travels with the source tree; nothing is installed elsewhere.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
LIB_DIR = PKG_DIR / "_lib"
LIB_PATH = LIB_DIR / "libtf_attn.so"
SOURCES = ["abi.hip", "decode.hip", "extend.hip", "kv_ops.hip", "qk_prep.hip"]
ARCH = "gfx950"


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm at /opt/rocm)")


def compile_flags() -> list:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Wall",
        "-Wno-unused-function",
        # Keep the compiler from emitting packed-fp32 VALU ops (v_pk_*_f32).
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{REPO_DIR / 'include'}",
        f"-I{CSRC}",
    ]


def build_library(verbose: bool = False) -> Path:
    """Compile every source into one shared library; returns its path."""
    LIB_DIR.mkdir(exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc_path(), *compile_flags(), "-shared", "-o", str(tmp),
           *[str(CSRC / s) for s in SOURCES]]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    if verbose and res.stderr.strip():
        # hipcc's host pass warns about the device-only target feature; show
        # anything else.
        lines = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln]
        if any(ln.strip() for ln in lines):
            print("\n".join(lines), file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose=True))
