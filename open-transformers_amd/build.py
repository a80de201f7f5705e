"""Builds libotx_attn.so (the gfx950 kernels and their C ABI) in place.

The library is compiled with hipcc for gfx950 only.  Flags that matter for
the bit-level contract:
  -ffp-contract=off   no compiler-formed fma: every a*b+c in the source is two
                      roundings unless written as an explicit fma
  (no -ffast-math, no -fgpu-flush-denormals-to-zero: binary32 denormals stay on)
  -Xclang -target-feature -Xclang -packed-fp32-ops
                      no v_pk_{add,mul,fma}_f32 anywhere
"""

from __future__ import annotations

import os
import pathlib
import shutil
import subprocess

PKG_DIR = pathlib.Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
LIB_NAME = "libotx_attn.so"
SOURCES = ["attn_fwd.hip", "attn_bwd.hip", "gemm.hip", "norm_act.hip", "loss.hip", "embedding.hip", "otx_capi.hip"]

HIPCC_FLAGS = [
    "-std=c++17",
    "-O3",
    "--offload-arch=gfx950",
    "-ffp-contract=off",
    "-fPIC",
    "-shared",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libotx_attn.so")


def build(verbose: bool = False) -> pathlib.Path:
    """Compile every HIP source into PKG_DIR/libotx_attn.so; returns the path."""
    out = PKG_DIR / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc_path(), *HIPCC_FLAGS, f"-I{CSRC}", f"-I{INCLUDE}"]
    cmd += [str(CSRC / s) for s in SOURCES]
    cmd += ["-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-4000:]}")
    if verbose and res.stderr:
        print(res.stderr)
    os.replace(tmp, out)
    build_host_math()
    return out


HOST_MATH_LIB = "libotx_math_host.so"


def build_host_math() -> pathlib.Path:
    """Host build of the kernels' exp/log/bf16/division (csrc/otx_math_host.cpp)
    so that the CPU test suite can check the exact device source without a GPU."""
    out = PKG_DIR / HOST_MATH_LIB
    tmp = out.with_suffix(".so.tmp")
    cxx = shutil.which("g++") or "g++"
    cmd = [cxx, "-O2", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-fPIC", "-shared", f"-I{CSRC}",
           str(CSRC / "otx_math_host.cpp"), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed ({res.returncode}):\n{res.stderr[-4000:]}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
