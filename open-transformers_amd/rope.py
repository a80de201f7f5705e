"""RoPE tables of the reference's RoPE module (host side, computed once).

The recipe is the reference's _build_inv_freq / _build_tables
(src/pretrain/model/modules/rope.py:21-31):

    inv_freq = 1.0 / (theta ** (arange(0, D, 2, float32) / D))   torch binary32 ops
    freqs    = outer(arange(S, float32), inv_freq)                binary32 products
    cos, sin = repop.ops.cos(freqs), repop.ops.sin(freqs)         correctly rounded binary32

inv_freq is computed with torch's own binary32 operations, exactly as the
reference computes it.  repop's cos/sin are correctly rounded
(docs/unified-audit-results.md:25 of the reference), so the table entries are
fixed by mathematics: each is the binary32 value nearest to the exact cosine
or sine of the binary32 angle.  They are evaluated in binary64 (the host
libm, within one binary64 ulp) and rounded once; where that binary64 value
lies too close to a binary32 rounding boundary for the rounding to be
certain, the entry is recomputed with 60 significant decimal digits.  No entry
depends on the host's libm.
"""

from __future__ import annotations

import decimal
import functools

import numpy as np

_F32 = np.float32
# pi to 80 significant digits
_PI = decimal.Decimal("3.1415926535897932384626433832795028841971693993751058209749445923078164062862089986")


def inv_freq(head_dim: int, theta: float) -> np.ndarray:
    """1 / theta^(2i/D), i < D/2, with the reference's torch binary32 operations."""
    import torch

    return (1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))).numpy()


def angles(seq_len: int, head_dim: int, theta: float) -> np.ndarray:
    """freqs [seq_len, head_dim/2] = pos * inv_freq, each product rounded to binary32."""
    pos = np.arange(seq_len, dtype=_F32)
    return (pos[:, None] * inv_freq(head_dim, theta)[None, :]).astype(_F32)


def _hp_cos_sin(x: float) -> tuple[decimal.Decimal, decimal.Decimal]:
    """cos and sin of the binary32 value x to about 60 significant digits."""
    if x == 0:
        return decimal.Decimal(1), decimal.Decimal(float(x))  # sin(+-0) = +-0
    with decimal.localcontext() as ctx:
        ctx.prec = 75
        X = decimal.Decimal(float(x))  # exact
        two_pi = 2 * _PI
        r = X - (X / two_pi).to_integral_value(rounding=decimal.ROUND_HALF_EVEN) * two_pi  # |r| <= pi
        r2 = r * r
        c, s = decimal.Decimal(0), decimal.Decimal(0)
        term_c, term_s = decimal.Decimal(1), r
        n = 0
        eps = decimal.Decimal(10) ** -70
        while abs(term_c) > eps or abs(term_s) > eps:
            c += term_c
            s += term_s
            term_c = -term_c * r2 / ((2 * n + 1) * (2 * n + 2))
            term_s = -term_s * r2 / ((2 * n + 2) * (2 * n + 3))
            n += 1
        return +c, +s


def _round_decimal_f32(y: decimal.Decimal) -> np.float32:
    """The binary32 value nearest to y (ties to even)."""
    f = _F32(float(y))  # within one binary32 step of y
    best = f
    with decimal.localcontext() as ctx:
        ctx.prec = 75
        for cand in (np.nextafter(f, _F32(-np.inf)), f, np.nextafter(f, _F32(np.inf))):
            dc = abs(decimal.Decimal(float(cand)) - y)
            db = abs(decimal.Decimal(float(best)) - y)
            if dc < db or (dc == db and (int(np.asarray(cand).view(np.uint32)) & 1) == 0):
                best = cand
    return _F32(best)


def _round_checked(y64: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Round binary64 values known to within 2^-52 (relative) to binary32; ok
    marks the entries whose rounding that error cannot change."""
    e = np.abs(y64) * 2.0**-50
    lo = (y64 - e).astype(_F32)
    hi = (y64 + e).astype(_F32)
    return lo, lo == hi


def cos_sin_f32(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Correctly rounded binary32 cos and sin of binary32 angles."""
    x = np.ascontiguousarray(x, dtype=_F32)
    x64 = x.astype(np.float64)
    c, okc = _round_checked(np.cos(x64))
    s, oks = _round_checked(np.sin(x64))
    for idx in np.argwhere(~(okc & oks)):
        t = tuple(idx)
        hc, hs = _hp_cos_sin(float(x[t]))
        c[t] = _round_decimal_f32(hc)
        s[t] = _round_decimal_f32(hs)
    return c, s


@functools.lru_cache(maxsize=16)
def _tables(seq_len: int, head_dim: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    c, s = cos_sin_f32(angles(seq_len, head_dim, theta))
    c.setflags(write=False)
    s.setflags(write=False)
    return c, s


def rope_tables(seq_len: int, head_dim: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """cos, sin tables [seq_len, head_dim/2] (binary32, read-only arrays)."""
    return _tables(int(seq_len), int(head_dim), float(theta))
