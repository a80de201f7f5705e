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
    srcs = [HERE / "attn_oracle.c", HERE / "layer_oracle.c", HERE / "int8pv_oracle.c", HERE / "loss_oracle.c",
            HERE / "Makefile"]
    if not LIB_PATH.exists() or any(p.stat().st_mtime > LIB_PATH.stat().st_mtime for p in srcs if p.exists()):
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
    lib.orc_cos_sin_quad_batch.restype = None
    lib.orc_cos_sin_quad_batch.argtypes = [_fp, _fp, _fp, ctypes.c_long]
    lib.orc_fmaf_batch.restype = None
    lib.orc_fmaf_batch.argtypes = [_fp, _fp, _fp, _fp, ctypes.c_long]
    lib.orc_attn_fwd.restype = _i
    lib.orc_attn_fwd.argtypes = [_fp] * 5 + [_i] * 8
    lib.orc_attn_bwd.restype = _i
    lib.orc_attn_bwd.argtypes = [_fp] * 9 + [_i] * 8
    _l = ctypes.c_long
    lib.orc_rsqrtf.restype = ctypes.c_float
    lib.orc_rsqrtf.argtypes = [ctypes.c_float]
    lib.orc_gemm.restype = _i
    lib.orc_gemm.argtypes = [_fp, _l, _l, _fp, _l, _l, _fp, _l, _i, _i, _i, _i, _i]
    lib.orc_rmsnorm_fwd.restype = _i
    lib.orc_rmsnorm_fwd.argtypes = [_fp, _fp, _fp, _fp, _l, _i, ctypes.c_float, _i, _i]
    lib.orc_rmsnorm_bwd.restype = _i
    lib.orc_rmsnorm_bwd.argtypes = [_fp, _fp, _fp, _fp, _fp, _fp, _l, _i, _i, _i]
    lib.orc_silu_fwd.restype = _i
    lib.orc_silu_fwd.argtypes = [_fp, _fp, _l, _i]
    lib.orc_silu_bwd.restype = _i
    lib.orc_silu_bwd.argtypes = [_fp, _fp, _fp, _l, _i]
    _vp = ctypes.c_void_p
    lib.orc_quantize_v.restype = _i
    lib.orc_quantize_v.argtypes = [_fp, _vp, _fp, _i, _i, _i, _i]
    lib.orc_attn_fwd_int8pv.restype = _i
    lib.orc_attn_fwd_int8pv.argtypes = [_fp] * 5 + [_i] * 8
    lib.orc_embedding_bwd.restype = _i
    lib.orc_embedding_bwd.argtypes = [_vp, _fp, _fp, _l, _i, _i, _i]
    lib.orc_fold32t.restype = ctypes.c_float
    lib.orc_fold32t.argtypes = [_fp, _l]
    lib.orc_ce_zloss_fwd.restype = _i
    lib.orc_ce_zloss_fwd.argtypes = [_fp, _vp, _l, _i, ctypes.c_double, _fp, _fp, _i]
    lib.orc_ce_zloss_bwd.restype = _i
    lib.orc_ce_zloss_bwd.argtypes = [_fp, _vp, _fp, ctypes.c_float, ctypes.c_float, _l, _l, _i, ctypes.c_double,
                                     _fp, _i, _i]
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
    """sum mod 2^64 of mix(x, f(x)) over bit patterns [lo, lo+count); f = exp (0) / log (1) /
    round to the nearest-even bf16 value (4) / rint (5, the int8-PV quantizer's rounding on [+0, 128))."""
    return int(load().orc_math_checksum(which, lo, count))


def cos_sin_quad(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """binary32 cos, sin of binary32 angles, rounded once from libquadmath's cosq / sinq."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    c = np.empty_like(x)
    s = np.empty_like(x)
    load().orc_cos_sin_quad_batch(_f(x), _f(c), _f(s), x.size)
    return c, s


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


def quantize_v(v):
    """v [B,Hkv,S,D] -> (qv int8 [B,Hkv,S,D], sv binary32 [B,Hkv,S/32,D]) of the int8-PV contract."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    B, Hkv, S, D = v.shape
    qv = np.empty(v.shape, dtype=np.int8)
    sv = np.empty((B, Hkv, S // 32, D), dtype=np.float32)
    if load().orc_quantize_v(_f(v), qv.ctypes.data, _f(sv), B, Hkv, S, D) != 0:
        raise ValueError("oracle rejected the shape")
    return qv, sv


def attn_fwd_int8pv(q, k, v, window: int = 0, out_bf16: bool = True, nthreads: int = 0):
    """int8-PV forward: q [B,H,S,D], k/v [B,Hkv,S,D] -> (o, lse)."""
    q, k, v = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v))
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    o = np.empty_like(q)
    lse = np.empty((B, H, S), dtype=np.float32)
    rc = load().orc_attn_fwd_int8pv(_f(q), _f(k), _f(v), _f(o), _f(lse), B, H, Hkv, S, D, window, int(out_bf16),
                                    nthreads)
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


def rsqrtf(x: float) -> float:
    return load().orc_rsqrtf(x)


def gemm(a: np.ndarray, b: np.ndarray, out_bf16: bool = True, nthreads: int = 0) -> np.ndarray:
    """C = a @ b.T with the serial binary32 fold over the shared last axis.

    a [M, R] and b [N, R] (binary32 arrays holding bf16 values); any axis
    layout is handled through strides by the C code, numpy views are made
    contiguous first."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    M, R = a.shape
    N, R2 = b.shape
    assert R == R2
    c = np.empty((M, N), dtype=np.float32)
    rc = load().orc_gemm(_f(a), R, 1, _f(b), R, 1, _f(c), N, M, N, R, int(out_bf16), nthreads)
    if rc != 0:
        raise ValueError("oracle rejected the GEMM")
    return c


def rmsnorm_fwd(x: np.ndarray, w: np.ndarray, eps: float, out_bf16: bool = True, nthreads: int = 0):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    D = x.shape[-1]
    rows = x.size // D
    y = np.empty_like(x)
    rstd = np.empty(x.shape[:-1], dtype=np.float32)
    rc = load().orc_rmsnorm_fwd(_f(x), _f(w), _f(y), _f(rstd), rows, D, eps, int(out_bf16), nthreads)
    if rc != 0:
        raise ValueError("oracle rejected the RMSNorm shape")
    return y, rstd


def rmsnorm_bwd(x, w, rstd, dy, out_bf16: bool = True, nthreads: int = 0):
    x, w, rstd, dy = (np.ascontiguousarray(t, dtype=np.float32) for t in (x, w, rstd, dy))
    D = x.shape[-1]
    rows = x.size // D
    dx = np.empty_like(x)
    dw = np.empty(D, dtype=np.float32)
    rc = load().orc_rmsnorm_bwd(_f(x), _f(w), _f(rstd), _f(dy), _f(dx), _f(dw), rows, D, int(out_bf16), nthreads)
    if rc != 0:
        raise ValueError("oracle rejected the RMSNorm shape")
    return dx, dw


def silu_fwd(x: np.ndarray, out_bf16: bool = True) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    load().orc_silu_fwd(_f(x), _f(y), x.size, int(out_bf16))
    return y


def silu_bwd(x: np.ndarray, dy: np.ndarray, out_bf16: bool = True) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    dy = np.ascontiguousarray(dy, dtype=np.float32)
    dx = np.empty_like(x)
    load().orc_silu_bwd(_f(x), _f(dy), _f(dx), x.size, int(out_bf16))
    return dx


def fold32t(a: np.ndarray) -> float:
    """Recursive chunk-32 fold of a binary32 vector (the loss reductions' order)."""
    a = np.ascontiguousarray(a, dtype=np.float32).ravel()
    return float(np.float32(load().orc_fold32t(_f(a), a.size)))


def ce_zloss_fwd(logits: np.ndarray, labels: np.ndarray, coeff: float, nthreads: int = 0):
    """logits [N, V] (binary32 values), labels [N] int64 -> (ce, z, stats [5, N])."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    lab = np.ascontiguousarray(labels, dtype=np.int64)
    N, V = x.shape
    stats = np.empty((5, N), dtype=np.float32)
    loss = np.empty(2, dtype=np.float32)
    if load().orc_ce_zloss_fwd(_f(x), lab.ctypes.data, N, V, coeff, _f(stats), _f(loss), nthreads) != 0:
        raise ValueError("oracle rejected the loss shape")
    return loss[0], loss[1], stats


def ce_zloss_bwd(logits, labels, stats, coeff: float, gce: float = 1.0, gz: float = 1.0, out_bf16: bool = True,
                 nthreads: int = 0, n_total: int | None = None) -> np.ndarray:
    """Logit gradient of rows [0, N) of a batch of ``n_total`` rows (default N);
    ``stats`` holds those rows' [5, N] statistics."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    lab = np.ascontiguousarray(labels, dtype=np.int64)
    st = np.ascontiguousarray(stats, dtype=np.float32)
    N, V = x.shape
    g = np.empty_like(x)
    if load().orc_ce_zloss_bwd(_f(x), lab.ctypes.data, _f(st), gce, gz, N, n_total or N, V, coeff, _f(g),
                               int(out_bf16), nthreads) != 0:
        raise ValueError("oracle rejected the loss shape")
    return g


def embedding_bwd(ids: np.ndarray, g: np.ndarray, V: int, out_bf16: bool = True) -> np.ndarray:
    """grad of weight [V, D] from ids [npos] and grad_out [npos, D] (position-ordered fold per id)."""
    ids = np.ascontiguousarray(ids, dtype=np.int64).ravel()
    g = np.ascontiguousarray(g, dtype=np.float32).reshape(ids.size, -1)
    gw = np.empty((V, g.shape[1]), dtype=np.float32)
    if load().orc_embedding_bwd(ids.ctypes.data, _f(g), _f(gw), ids.size, V, g.shape[1], int(out_bf16)) != 0:
        raise ValueError("oracle rejected the embedding shape")
    return gw
