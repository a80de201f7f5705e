"""Builds libotx_attn.so (the gfx950 kernels and their C ABI) in place.

The library is compiled with hipcc for gfx950 only.  Flags that matter for
the bit-level contract:
  -ffp-contract=off   no compiler-formed fma: every a*b+c in the source is two
                      roundings unless written as an explicit fma
  (no -ffast-math, no -fgpu-flush-denormals-to-zero: binary32 denormals stay on)
  -Xclang -target-feature -Xclang -packed-fp32-ops
                      no v_pk_{add,mul,fma}_f32 anywhere

Each HIP source compiles to its own object under ``_build/`` (in parallel);
the objects are linked with the provenance stamp (``csrc/otx_stamp.cpp``:
commit, dirty flag and a digest of the compiled sources and flags, the
analogue of ``repop.build_info()["commit"]`` that the reference's audit replay
records, src/pretrain/cli/audit_replay.py:1508-1511).
"""

from __future__ import annotations

import concurrent.futures
import hashlib
import os
import pathlib
import shutil
import subprocess

PKG_DIR = pathlib.Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
OBJ_DIR = PKG_DIR / "_build"
LIB_NAME = "libotx_attn.so"
SOURCES = ["attn_fwd.hip", "attn_bwd.hip", "gemm.hip", "norm_act.hip", "rope.hip", "loss.hip", "embedding.hip",
           "otx_capi.hip"]
STAMP_SOURCE = "otx_stamp.cpp"

HIPCC_FLAGS = [
    "-std=c++17",
    "-O3",
    "--offload-arch=gfx950",
    "-ffp-contract=off",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]
STAMP_FLAGS = ["-std=c++17", "-O2", "-fPIC"]
# Paths whose state decides the stamp's dirty flag (relative to the repository root).
STAMP_PATHS = ("open-transformers_amd/csrc", "include", "open-transformers_amd/build.py")


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libotx_attn.so")


def sources_digest() -> str:
    """blake2b-16 (hex) over the library's sources, every header they can
    include and the compile flags: equal digests mean the same inputs."""
    h = hashlib.blake2b(digest_size=16)
    files = [CSRC / s for s in SOURCES] + sorted(CSRC.glob("*.h")) + sorted(INCLUDE.glob("*.h"))
    for p in files:
        h.update(p.name.encode() + b"\0" + p.read_bytes() + b"\0")
    h.update(" ".join(HIPCC_FLAGS + SOURCES).encode())
    return h.hexdigest()


def tree_stamp() -> dict:
    """{"commit": 12-hex HEAD or "unknown", "dirty": bool or None} of the checkout
    holding this package; dirty means a stamped path differs from HEAD or holds
    untracked files."""
    root = PKG_DIR.parent

    def git(*args):
        return subprocess.run(["git", "-C", str(root), *args], capture_output=True, text=True, timeout=30)

    try:
        head = git("rev-parse", "--short=12", "HEAD")
        if head.returncode != 0 or not head.stdout.strip():
            return {"commit": "unknown", "dirty": None}
        st = git("status", "--porcelain", "--", *STAMP_PATHS)
        dirty = None if st.returncode != 0 else bool(st.stdout.strip())
        return {"commit": head.stdout.strip(), "dirty": dirty}
    except (OSError, subprocess.SubprocessError):
        return {"commit": "unknown", "dirty": None}


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{cmd[0]} failed ({res.returncode}):\n{res.stderr[-4000:]}")
    return res


def compile_objects(jobs: int | None = None) -> list[pathlib.Path]:
    """Compile every HIP source to OBJ_DIR/<name>.o (always, in parallel)."""
    OBJ_DIR.mkdir(exist_ok=True)
    hipcc = hipcc_path()
    jobs = jobs or max(1, min(len(SOURCES), os.cpu_count() or 1))

    def one(src):
        obj = OBJ_DIR / (pathlib.Path(src).stem + ".o")
        tmp = obj.with_suffix(".o.tmp")
        _run([hipcc, *HIPCC_FLAGS, "-c", f"-I{CSRC}", f"-I{INCLUDE}", str(CSRC / src), "-o", str(tmp)])
        os.replace(tmp, obj)
        return obj

    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        return list(ex.map(one, SOURCES))


def link(out: pathlib.Path, stamp: dict | None = None, digest: str | None = None) -> pathlib.Path:
    """Compile the provenance stamp and link it with the objects in OBJ_DIR into ``out``."""
    objs = [OBJ_DIR / (pathlib.Path(s).stem + ".o") for s in SOURCES]
    missing = [o.name for o in objs if not o.exists()]
    if missing:
        raise RuntimeError(f"objects not built: {missing} (run build())")
    stamp = tree_stamp() if stamp is None else stamp
    digest = sources_digest() if digest is None else digest
    dirty = {True: "true", False: "false", None: "null"}[stamp["dirty"]]
    out = pathlib.Path(out)
    stamp_obj = out.parent / (out.stem + ".stamp.o")
    cxx = shutil.which("g++") or "g++"
    _run([cxx, *STAMP_FLAGS, f'-DOTX_STAMP_COMMIT="{stamp["commit"]}"', f'-DOTX_STAMP_DIRTY="{dirty}"',
          f'-DOTX_STAMP_SOURCES="{digest}"', "-c", str(CSRC / STAMP_SOURCE), "-o", str(stamp_obj)])
    tmp = out.with_suffix(".so.tmp")
    try:
        _run([hipcc_path(), "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), str(stamp_obj), "-o", str(tmp)])
    finally:
        stamp_obj.unlink(missing_ok=True)
    os.replace(tmp, out)
    return out


def check_isa(lib: pathlib.Path) -> None:
    """Refuse a library whose code touches a register while an LDS load into it
    is still in flight (isa_check.py: the hand-counted LDS reads of the matrix
    chains are invisible to the compiler, which may copy their destinations
    early)."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("_otx_isa_check", PKG_DIR / "isa_check.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    hazards = mod.check_library(lib)
    if hazards:
        lines = [f"{fn}: {len(v)} instruction(s), first {v[0][0]!r} touches {v[0][1]}" for fn, v in hazards.items()]
        raise RuntimeError("registers touched while their LDS loads are in flight:\n" + "\n".join(lines))


def build(verbose: bool = False) -> pathlib.Path:
    """Compile every HIP source and link PKG_DIR/libotx_attn.so; returns the path."""
    compile_objects()
    tmp = link(PKG_DIR / "libotx_attn.unchecked.so")
    try:
        check_isa(tmp)
    except BaseException:
        tmp.unlink(missing_ok=True)
        raise
    out = PKG_DIR / LIB_NAME
    os.replace(tmp, out)
    if verbose:
        print(out, tree_stamp(), sources_digest())
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
