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
import tempfile
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
LIB_DIR = PKG_DIR / "_lib"
LIB_PATH = LIB_DIR / "libtf_attn.so"
SOURCES = ["abi.hip", "attn_generic.hip", "decode.hip", "extend.hip", "fp8_linear.hip",
           "gdn.hip", "kv_ops.hip", "plan.hip", "qk_prep.hip"]
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


# Per-file flags on top of compile_flags(): MFMA accumulators in VGPRs.
# extend.hip: two waves per SIMD, O^T, Q^T and S^T all in the 256 VGPRs
# of a wave.  fp8_linear.hip: the GEMM folds each MFMA product into fp32
# accumulators with a VALU FMA, which reads VGPRs only.  gdn.hip: the chunked
# recurrence feeds its accumulators (state, P, Delta) back to VALU work and
# MFMA operands.
EXTRA_FLAGS = {"extend.hip": ["-mllvm", "--amdgpu-mfma-vgpr-form=1"],
               "fp8_linear.hip": ["-mllvm", "--amdgpu-mfma-vgpr-form=1"],
               "gdn.hip": ["-mllvm", "--amdgpu-mfma-vgpr-form=1"]}


def _filter_stderr(text: str) -> str:
    # hipcc's host pass warns about the device-only target feature; keep the rest.
    return "\n".join(ln for ln in text.splitlines() if "packed-fp32-ops" not in ln).strip()


def build_library(verbose: bool = False) -> Path:
    """Compile every source (in parallel) and link one shared library; returns its path."""
    LIB_DIR.mkdir(exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    with tempfile.TemporaryDirectory(prefix="tf_attn_build_") as objdir:
        procs = []
        for src in SOURCES:
            obj = Path(objdir) / (Path(src).stem + ".o")
            cmd = [hipcc_path(), *compile_flags(), *EXTRA_FLAGS.get(src, []), "-c",
                   str(CSRC / src), "-o", str(obj)]
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append((src, obj, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                                     stderr=subprocess.PIPE, text=True)))
        objs, failures = [], []
        for src, obj, proc in procs:
            out, err = proc.communicate()
            if proc.returncode != 0:
                failures.append(f"{src}: hipcc failed ({proc.returncode}):\n{out}\n{err}")
            elif verbose and _filter_stderr(err):
                print(_filter_stderr(err), file=sys.stderr)
            objs.append(str(obj))
        if failures:
            raise RuntimeError("\n".join(failures))
        cmd = [hipcc_path(), f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *objs]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose=True))
