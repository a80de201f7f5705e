"""ctypes wrapper of the CPU oracle (oracle/attn_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as the
checker and by bench.py's CPU-baseline leg.  The product never imports it.
"""

from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "liborc.so"

_LIB = None
_fp = ctypes.POINTER(ctypes.c_float)
_i = ctypes.c_int


def build() -> pathlib.Path:
    res = subprocess.run(["make", "-s", "-f", str(HERE / "Makefile")], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stderr[-4000:]}")
    return LIB_PATH


def load() -> ctypes.CDLL:
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.orc_expf.restype = ctypes.c_float
    lib.orc_expf.argtypes = [ctypes.c_float]
    lib.orc_logf.restype = ctypes.c_float
    lib.orc_logf.argtypes = [ctypes.c_float]
    lib.orc_expf_quad.restype = ctypes.c_float
    lib.orc_expf_quad.argtypes = [ctypes.c_float]
    lib.orc_logf_quad.restype = ctypes.c_float
    lib.orc_logf_quad.argtypes = [ctypes.c_float]
    lib.orc_scale.restype = ctypes.c_float
    lib.orc_scale.argtypes = [_i]
    lib.orc_round_bf16.restype = ctypes.c_float
    lib.orc_round_bf16.argtypes = [ctypes.c_float]
    lib.orc_verify_math.restype = ctypes.c_uint64
    lib.orc_verify_math.argtypes = [ctypes.c_uint32, ctypes.c_uint32, _i]
    lib.orc_math_checksum.restype = ctypes.c_uint64
    lib.orc_math_checksum.argtypes = [_i, ctypes.c_uint64, ctypes.c_uint64]
    lib.orc_fmaf_batch.restype = None
    lib.orc_fmaf_batch.argtypes = [_fp, _fp, _fp, _fp, ctypes.c_long]
    lib.orc_attn_fwd.restype = _i
    lib.orc_attn_fwd.argtypes = [_fp] * 5 + [_i] * 8
    lib.orc_attn_bwd.restype = _i
    lib.orc_attn_bwd.argtypes = [_fp] * 9 + [_i] * 8
    _LIB = lib
    return lib


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_fp)


def expf(x: float) -> float:
    return load().orc_expf(x)


def logf(x: float) -> float:
    return load().orc_logf(x)


def scale(D: int) -> float:
    return load().orc_scale(D)


def math_checksum(which: int, lo: int, count: int) -> int:
    """sum mod 2^64 of mix(x, f(x)) over bit patterns [lo, lo+count); f = exp (0) / log (1)."""
    return int(load().orc_math_checksum(which, lo, count))


def fmaf(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    a, b, c = (np.ascontiguousarray(x, dtype=np.float32) for x in (a, b, c))
    out = np.empty_like(a)
    load().orc_fmaf_batch(_f(a), _f(b), _f(c), _f(out), a.size)
    return out


def attn_fwd(q, k, v, window: int = 0, out_bf16: bool = False, nthreads: int = 0):
    """q [B,H,S,D], k/v [B,Hkv,S,D] binary32 -> (o, lse)."""
    q, k, v = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v))
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    o = np.empty_like(q)
    lse = np.empty((B, H, S), dtype=np.float32)
    rc = load().orc_attn_fwd(_f(q), _f(k), _f(v), _f(o), _f(lse), B, H, Hkv, S, D, window, int(out_bf16), nthreads)
    if rc != 0:
        raise ValueError("oracle rejected the shape")
    return o, lse


def attn_bwd(q, k, v, o, lse, do, window: int = 0, out_bf16: bool = False, nthreads: int = 0):
    q, k, v, o, do = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v, o, do))
    lse = np.ascontiguousarray(lse, dtype=np.float32)
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    dq = np.empty_like(q)
    dk = np.empty_like(k)
    dv = np.empty_like(v)
    rc = load().orc_attn_bwd(
        _f(q), _f(k), _f(v), _f(o), _f(lse), _f(do), _f(dq), _f(dk), _f(dv), B, H, Hkv, S, D, window,
        int(out_bf16), nthreads,
    )
    if rc != 0:
        raise ValueError("oracle rejected the shape")
    return dq, dk, dv
