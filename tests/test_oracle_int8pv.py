"""CPU pins of the int8-PV oracle (oracle/int8pv_oracle.c).

repop's int8pv_causal_flash_attention is closed and absent and the reference's
tests hold no vectors for it, so each check is fixed by something other than
the oracle's code:

  quantizer       V: per (key block, column) the largest magnitude maps to
                  +-127 exactly, every value is within half a step of its
                  quantized value (round to nearest, not floor), exact ties go
                  to the even neighbour, zero columns stay zero, non-finite
                  columns become NaN.
  closed forms    q = 0 (every visible key has probability 1, so qp = 127) with
                  V on an exact int8 grid (k * 2^e, max |k| = 127 in each
                  block column): the int8 path is exact up to the rounding of
                  RN(1/127) and the fma chain, so O is the running mean of the
                  visible V rows to 2^-20 relative.  With V off the grid, the
                  error of that mean is bounded by half a quantization step.
  invariants      LSE is bit-identical to the binary32 forward (l sums the
                  unquantized probabilities); the causal mask and sliding
                  window act exactly as in the binary32 forward.
  mathematics     random inputs against float64 softmax attention, within an
                  error bound computed per element from the quantization steps
                  (|sp qp - p| <= sp/2, |sv qv - v| <= sv/2); the observed
                  error is also required to be a sizeable part of that bound,
                  so the quantization really happens.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from attn_util import assert_bits_equal, make
from oracle import oracle as orc
from open_transformers_amd import synthetic


def _grid_v(rng, B, Hkv, S, D, e=-6):
    """V = k * 2^e with integer k in [-127, 127] and max |k| = 127 in every
    (key block, column); returns the values."""
    k = rng.integers(-127, 128, (B, Hkv, S // 32, 32, D))
    j = rng.integers(0, 32, (B, Hkv, S // 32, D))
    sign = rng.choice([-1, 1], (B, Hkv, S // 32, D))
    np.put_along_axis(k, j[:, :, :, None, :], (127 * sign)[:, :, :, None, :], axis=3)
    return (k * 2.0 ** e).reshape(B, Hkv, S, D).astype(np.float32)


def test_quantize_v_steps_and_extremes():
    rng = np.random.default_rng(3)
    B, Hkv, S, D = 2, 2, 128, 64
    v = synthetic.round_to_bf16(rng.standard_normal((B, Hkv, S, D)).astype(np.float32) * 3)
    v[0, 0, 0:32, 5] = 0.0  # an all-zero block column
    qv, sv = orc.quantize_v(v)
    vb = v.reshape(B, Hkv, S // 32, 32, D).astype(np.float64)
    qb = qv.reshape(B, Hkv, S // 32, 32, D).astype(np.int64)
    amax = np.abs(vb).max(axis=3)
    # the largest magnitude of each block column maps to +-127, signs are kept
    assert np.all(np.abs(qb).max(axis=3)[amax > 0] == 127)
    assert np.all(np.sign(qb) * np.sign(vb) >= 0)
    # scale = amax / 127 to binary32 precision; zero column -> zero scale and values
    nz = amax > 0
    assert np.all(np.abs(sv[nz] - amax[nz] / 127) <= amax[nz] / 127 * 2.0 ** -23)
    assert sv[0, 0, 0, 5] == 0.0 and np.all(qb[0, 0, 0, :, 5] == 0)
    # round to nearest: within half a step (plus binary32 slack)
    step = (amax / 127)[:, :, :, None, :]
    assert np.all(np.abs(qb * step - vb) <= step * (0.5 + 2.0 ** -18))
    # ... and not a floor / truncation: errors have both signs and a small mean
    err = (qb * step - vb)[np.broadcast_to(nz[:, :, :, None, :], qb.shape)]
    assert abs(err.mean()) < 0.02 * step.max()


def test_quantize_v_ties_to_even_and_non_finite():
    S, D = 32, 8
    v = np.zeros((1, 1, S, D), dtype=np.float32)
    v[0, 0, 0, :] = 127.0  # amax 127 * 2^0: inv = 1 exactly, so v * inv is exact
    v[0, 0, 1, :] = [0.0, 0.0, 2.5, 3.5, -2.5, -3.5, 126.5, 0.5]  # exact ties in columns 2..7
    v[0, 0, 2, 0] = np.inf  # non-finite columns 0 and 1
    v[0, 0, 3, 1] = np.nan
    qv, sv = orc.quantize_v(v)
    assert list(qv[0, 0, 1, 2:]) == [2, 4, -2, -4, 126, 0]
    assert np.isnan(sv[0, 0, 0, 0]) and np.isnan(sv[0, 0, 0, 1])
    assert np.all(qv[0, 0, :, 0] == 0) and np.all(qv[0, 0, :, 1] == 0)
    assert np.all(sv[0, 0, 0, 2:] == np.float32(1.0))


def test_lse_equals_binary32_forward():
    inp = make(2, 4, 2, 256, 64, seed=11)
    for window in (0, 64):
        _, lse8 = orc.attn_fwd_int8pv(inp["q"], inp["k"], inp["v"], window=window)
        _, lse = orc.attn_fwd(inp["q"], inp["k"], inp["v"], window=window, out_bf16=True)
        assert_bits_equal(lse8, lse, f"LSE window={window}")


@pytest.mark.parametrize("window", [0, 96])
def test_uniform_attention_on_exact_grid(window):
    rng = np.random.default_rng(5 + window)
    B, H, Hkv, S, D = 1, 2, 1, 256, 64
    q = np.zeros((B, H, S, D), np.float32)
    k = synthetic.round_to_bf16(rng.standard_normal((B, Hkv, S, D)).astype(np.float32))
    v = _grid_v(rng, B, Hkv, S, D)
    o, lse = orc.attn_fwd_int8pv(q, k, v, window=window, out_bf16=False)
    vs = v.astype(np.float64)
    for i in range(S):
        lo = max(0, i - window + 1) if window else 0
        mean = vs[0, 0, lo:i + 1].mean(axis=0)
        np.testing.assert_allclose(o[0, :, i], np.broadcast_to(mean, (H, D)), rtol=0, atol=2.0 ** -20 * 127 * 2.0 ** -6)
        assert lse[0, 0, i] == np.float32(math.log(i + 1 - lo))


def test_uniform_attention_error_within_half_step():
    rng = np.random.default_rng(8)
    B, H, Hkv, S, D = 1, 1, 1, 192, 64
    q = np.zeros((B, H, S, D), np.float32)
    k = np.zeros((B, Hkv, S, D), np.float32)
    v = synthetic.round_to_bf16(rng.standard_normal((B, Hkv, S, D)).astype(np.float32))
    o, _ = orc.attn_fwd_int8pv(q, k, v, out_bf16=False)
    vb = v.reshape(S // 32, 32, D).astype(np.float64)
    half = np.abs(vb).max(axis=1) / 127 / 2  # [block, D]
    err = np.abs(o[0, 0] - np.cumsum(v[0, 0].astype(np.float64), axis=0) / np.arange(1, S + 1)[:, None])
    bound = np.maximum.accumulate(half, axis=0).repeat(32, axis=0) * (1 + 2.0 ** -16) + 1e-6
    assert np.all(err <= bound)
    assert err.max() > 0.2 * half.min()  # V really is quantized


def _bound_and_ref(q, k, v, window):
    """float64 attention and a per-element bound on the int8-PV error."""
    B, H, S, D = q.shape
    G = H // k.shape[1]
    kk = np.repeat(k.astype(np.float64), G, axis=1)
    vv = np.repeat(v.astype(np.float64), G, axis=1)
    s = np.einsum("bhid,bhjd->bhij", q.astype(np.float64), kk) / math.sqrt(D)
    i = np.arange(S)[:, None]
    j = np.arange(S)[None, :]
    mask = (j > i) | ((j <= i - window) if window else False)
    s = np.where(mask, -np.inf, s)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    l = p.sum(axis=-1, keepdims=True)
    o = (p @ vv) / l
    nb = S // 32
    pb = p.reshape(B, H, S, nb, 32)
    pmax = pb.max(axis=-1)  # [B,H,S,nb] block maxima relative to the row max
    sv = np.abs(vv.reshape(B, H, nb, 32, D)).max(axis=3) / 127  # [B,H,nb,D]
    # sum_j sp/2 (|v| + sv/2) + p sv/2, with sp = pmax / 127
    absv = np.abs(vv).reshape(B, H, nb, 32, D).sum(axis=3)  # sum_j |v_j| per block
    t1 = np.einsum("bhin,bhnd->bhid", pmax / 254, absv + 16 * sv)
    t2 = np.einsum("bhinj,bhnd->bhid", pb, sv) / 2
    bound = (t1 + t2) / l * (1 + 2.0 ** -10) + 2.0 ** -20 * (np.abs(p) @ np.abs(vv)) / l + 1e-7
    return o, bound


@pytest.mark.parametrize("window", [0, 64])
def test_random_inputs_within_quantization_bound(window):
    inp = make(1, 4, 2, 256, 64, seed=21 + window)
    o8, _ = orc.attn_fwd_int8pv(inp["q"], inp["k"], inp["v"], window=window, out_bf16=False)
    ref, bound = _bound_and_ref(inp["q"], inp["k"], inp["v"], window)
    err = np.abs(o8 - ref)
    assert np.all(err <= bound), float((err / bound).max())
    assert (err / bound).max() > 0.05
    o, _ = orc.attn_fwd(inp["q"], inp["k"], inp["v"], window=window)
    assert not np.array_equal(o8, o)


def test_causality_and_window_match_binary32_visibility():
    """Changing a future key/value or one outside the window changes nothing."""
    inp = make(1, 2, 2, 128, 64, seed=4)
    o, lse = orc.attn_fwd_int8pv(inp["q"], inp["k"], inp["v"], window=64)
    k2, v2 = inp["k"].copy(), inp["v"].copy()
    k2[:, :, 100:] = -k2[:, :, 100:]
    v2[:, :, 100:] = 3 * v2[:, :, 100:]
    o2, lse2 = orc.attn_fwd_int8pv(inp["q"], k2, v2, window=64)
    assert_bits_equal(o2[:, :, :96], o[:, :, :96], "O before the changed block")
    assert_bits_equal(lse2[:, :, :100], lse[:, :, :100], "LSE before the changed keys")
    # keys 0..31 lie outside the window of queries >= 96 (window 64 with blocks of 32)
    k3 = inp["k"].copy()
    k3[:, :, :32] = 0
    o3, lse3 = orc.attn_fwd_int8pv(inp["q"], k3, inp["v"], window=64)
    assert_bits_equal(o3[:, :, 96:], o[:, :, 96:], "O outside the window")
    assert_bits_equal(lse3[:, :, 96:], lse[:, :, 96:], "LSE outside the window")
