"""Seeded synthetic attention inputs (host side, numpy).

Values are drawn per (seed, tensor, batch index) from a Philox4x32-10 stream
(numpy.random.Philox keyed by (seed, tensor id << 32 | batch index)), so the
content of sequence b does not depend on the batch size B.  Draws are
numpy's binary32 standard normals (Generator.standard_normal with
dtype=float32, a ziggurat); bf16 tensors are the round-to-nearest-even bf16
values of those draws.  The optional RoPE step follows the reference's
apply_rope (src/pretrain/model/modules/rope.py:103-125: interleaved pairs,
rx1 = x1*cos - x2*sin, rx2 = x1*sin + x2*cos, each product and sum rounded to
binary32) with the reference's tables (rope.py:21-31; see rope.py of this
package: torch binary32 inv_freq, correctly rounded cos/sin).
"""

from __future__ import annotations

import numpy as np

from . import rope as _rope

TENSOR_IDS = {"q": 1, "k": 2, "v": 3, "do": 4}


def normal_f32(seed: int, tensor: str, B: int, H: int, S: int, D: int) -> np.ndarray:
    out = np.empty((B, H, S, D), dtype=np.float32)
    tid = TENSOR_IDS[tensor]
    for b in range(B):
        key = np.array([seed & 0xFFFFFFFFFFFFFFFF, (tid << 32) | b], dtype=np.uint64)
        gen = np.random.Generator(np.random.Philox(key=key))
        out[b] = gen.standard_normal((H, S, D), dtype=np.float32)
    return out


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """binary32 -> nearest-even bf16 value (returned as binary32)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) & np.uint32(0xFFFF0000)
    r = np.where(nan, (u | np.uint32(0x00400000)) & np.uint32(0xFFFF0000), r)
    return r.astype(np.uint32).view(np.float32)


def rope_tables(S: int, D: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """The reference's RoPE tables (rope.py:21-31), shared with the decoder layer."""
    return _rope.rope_tables(S, D, theta)


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x [B, H, S, D] binary32; cos/sin [S, D/2]."""
    x1 = x[..., 0::2]
    x2 = x[..., 1::2]
    c = cos[None, None]
    s = sin[None, None]
    rx1 = (x1 * c).astype(np.float32) - (x2 * s).astype(np.float32)
    rx2 = (x1 * s).astype(np.float32) + (x2 * c).astype(np.float32)
    out = np.empty_like(x)
    out[..., 0::2] = rx1
    out[..., 1::2] = rx2
    return out


def make_inputs(
    B: int,
    H: int,
    Hkv: int,
    S: int,
    D: int,
    dtype: str = "bf16",
    seed: int = 0,
    rope_theta: float | None = None,
    qk_scale: float | None = None,
    with_grad: bool = True,
) -> dict[str, np.ndarray]:
    """binary32 arrays q, k, v (and do) whose values are representable in ``dtype``."""
    q = normal_f32(seed, "q", B, H, S, D)
    k = normal_f32(seed, "k", B, Hkv, S, D)
    v = normal_f32(seed, "v", B, Hkv, S, D)
    if rope_theta is not None:
        cos, sin = rope_tables(S, D, rope_theta)
        q = apply_rope(q, cos, sin)
        k = apply_rope(k, cos, sin)
    if qk_scale is not None:
        q = (q * np.float32(qk_scale)).astype(np.float32)
        k = (k * np.float32(qk_scale)).astype(np.float32)
    out = {"q": q, "k": k, "v": v}
    if with_grad:
        out["do"] = normal_f32(seed, "do", B, H, S, D)
    if dtype == "bf16":
        out = {name: round_to_bf16(a) for name, a in out.items()}
    elif dtype != "f32":
        raise ValueError(f"dtype {dtype!r} not supported")
    return out


# The BASELINE configurations (shapes and input recipes).
CONFIGS = {
    "c1": dict(B=1, H=4, Hkv=4, S=256, D=64, dtype="f32", rope_theta=None, qk_scale=None),
    "c2": dict(B=4, H=16, Hkv=16, S=2048, D=128, dtype="bf16", rope_theta=10000.0, qk_scale=None),
    "c3": dict(B=1, H=16, Hkv=16, S=8192, D=128, dtype="bf16", rope_theta=None, qk_scale=3.0),
    "c4": dict(B=1, H=16, Hkv=16, S=1024, D=128, dtype="bf16", rope_theta=None, qk_scale=None),
}


def causal_pairs(B: int, H: int, S: int, window: int = 0) -> int:
    """Number of unmasked (query, key) pairs."""
    if window <= 0:
        return B * H * S * (S + 1) // 2
    n = 0
    for i in range(S):
        n += min(i + 1, window)
    return B * H * n


def attention_flops(B: int, H: int, S: int, D: int, window: int = 0, backward: bool = True) -> float:
    """FlashAttention convention: 4*D per unmasked pair forward, +10*D backward."""
    per_pair = (14 if backward else 4) * D
    return float(causal_pairs(B, H, S, window) * per_pair)
