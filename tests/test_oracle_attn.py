"""CPU pins of the attention oracle (oracle/attn_oracle.c).

The reference operator (repop's causal_flash_attention) is closed and absent,
and the reference's own tests hold no attention golden vectors, so every check
here is fixed by something other than the oracle's code:

  closed forms    q = 0 (uniform attention: O is the ascending running sum of
                  V divided by the key count, LSE = log(count)); the first
                  query row (O_0 = V_0, LSE_0 = s_00); one-hot V columns (O
                  equals the probabilities).
  order / fma     inputs chosen so that a reversed or pairwise dot product,
                  or a multiply-then-add in place of the fma, gives a
                  different LSE bit pattern than the serial ascending fma fold.
  mathematics     forward and gradients against a float64 torch autograd
                  implementation of softmax attention (tolerance 2e-5 relative
                  to the output scale): a dropped term, a wrong sign, a wrong
                  index or a transposed operand fails these.
  invariants      causality, batch-size and thread-count invariance, GQA with
                  duplicated K/V heads equal to MHA, sliding window equal to an
                  explicit mask.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from attn_util import assert_bits_equal, make, oracle_fwd_bwd
from oracle import oracle as orc


def _f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def _torch_ref(q, k, v, do, window):
    """float64 softmax attention and its autograd gradients (GQA by repeat)."""
    q64, k64, v64 = (torch.from_numpy(np.asarray(x, dtype=np.float64)).requires_grad_() for x in (q, k, v))
    B, H, S, D = q64.shape
    G = H // k64.shape[1]
    kk = k64.repeat_interleave(G, dim=1)
    vv = v64.repeat_interleave(G, dim=1)
    s = (q64 @ kk.transpose(-1, -2)) / math.sqrt(D)
    i = torch.arange(S)[:, None]
    j = torch.arange(S)[None, :]
    mask = j > i
    if window > 0:
        mask = mask | (j <= i - window)
    s = s.masked_fill(mask, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    o = torch.softmax(s, dim=-1) @ vv
    o.backward(torch.from_numpy(np.asarray(do, dtype=np.float64)))
    return (o.detach().numpy(), lse.detach().numpy(), q64.grad.numpy(), k64.grad.numpy(), v64.grad.numpy())


def test_q_zero_is_uniform_attention():
    B, H, S, D = 1, 2, 96, 64
    inp = make(B, H, H, S, D, dtype="f32", seed=21)
    q0 = np.zeros_like(inp["q"])
    o, lse = orc.attn_fwd(q0, inp["k"], inp["v"])
    # p = exp(0) = 1 exactly; acc = ascending float32 running sum; l = key count.
    run = np.add.accumulate(inp["v"], axis=2, dtype=np.float32)
    cnt = np.arange(1, S + 1, dtype=np.float64)[None, None, :, None]
    want_o = (run.astype(np.float64) / cnt).astype(np.float32)  # double rounding is exact for a quotient
    assert_bits_equal(o, want_o, "O (q = 0)")
    want_lse = np.array([orc.load().orc_logf_quad(float(n)) for n in range(1, S + 1)], dtype=np.float32)
    assert_bits_equal(lse, np.broadcast_to(want_lse, lse.shape), "LSE (q = 0)")


def test_first_row_closed_form():
    rng = np.random.default_rng(3)
    D = 64
    q = rng.integers(-4, 5, (1, 1, 64, D)).astype(np.float32)
    k = rng.integers(-4, 5, (1, 1, 64, D)).astype(np.float32)
    v = rng.standard_normal((1, 1, 64, D)).astype(np.float32)
    o, lse = orc.attn_fwd(q, k, v)
    assert_bits_equal(o[0, 0, 0], v[0, 0, 0], "O_0 = V_0")
    exact = float(np.dot(q[0, 0, 0].astype(np.float64), k[0, 0, 0].astype(np.float64))) * 0.125
    assert lse[0, 0, 0] == np.float32(exact)


def test_dot_is_serial_ascending_fma():
    """LSE_0 = RN(dot(q_0, k_0) * sigma) exposes the dot product's order and fma."""
    D = 64
    q = np.zeros((1, 1, 32, D), dtype=np.float32)
    k = np.zeros_like(q)
    v = np.zeros_like(q)
    # order: 1 + 2^24 rounds to 2^24 (tie to even), then - 2^24 gives 0;
    # a reversed or pairwise sum would keep the 1.
    q[0, 0, 0, :3] = [1.0, 2.0**24, -(2.0**24)]
    k[0, 0, 0, :3] = 1.0
    _, lse = orc.attn_fwd(q, k, v)
    assert lse[0, 0, 0] == 0.0
    # fma: -1 + (1 + 2^-12)^2 keeps the 2^-24 term only when fused.
    q[0, 0, 0, :3] = [1.0, 1.0 + 2.0**-12, 0.0]
    k[0, 0, 0, :3] = [-1.0, 1.0 + 2.0**-12, 0.0]
    _, lse = orc.attn_fwd(q, k, v)
    assert lse[0, 0, 0] == np.float32((2.0**-11 + 2.0**-24) * 0.125)


def test_one_hot_v_gives_probabilities():
    B, H, S, D = 1, 1, 64, 64
    inp = make(B, H, H, S, D, dtype="f32", seed=4)
    v = np.zeros((B, H, S, D), dtype=np.float32)
    v[0, 0, np.arange(D), np.arange(D)] = 1.0  # value of key j = e_j (keys 0..63)
    o, lse = orc.attn_fwd(inp["q"], inp["k"], v)
    s = (inp["q"][0, 0].astype(np.float64) @ inp["k"][0, 0].astype(np.float64).T) / 8.0
    s[np.triu_indices(S, 1)] = -np.inf
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    np.testing.assert_allclose(o[0, 0], p, rtol=0, atol=2e-6)


@pytest.mark.parametrize(
    "B,H,Hkv,S,D,window,seed",
    [(1, 2, 2, 64, 64, 0, 1), (2, 4, 2, 96, 64, 32, 2), (1, 3, 1, 128, 128, 64, 3), (1, 2, 2, 160, 128, 0, 4)],
)
def test_oracle_matches_float64_math(B, H, Hkv, S, D, window, seed):
    inp = make(B, H, Hkv, S, D, dtype="f32", seed=seed)
    got = oracle_fwd_bwd(inp, window, bf16=False)
    o, lse, dq, dk, dv = _torch_ref(inp["q"], inp["k"], inp["v"], inp["do"], window)
    for name, a, b in (("o", got["o"], o), ("lse", got["lse"], lse), ("dq", got["dq"], dq), ("dk", got["dk"], dk),
                       ("dv", got["dv"], dv)):
        scale = max(1.0, float(np.abs(b).max()))
        err = float(np.abs(a.astype(np.float64) - b).max())
        assert err <= 2e-5 * scale, f"{name}: max error {err} (scale {scale})"


def test_bf16_outputs_are_rounded_fp32_outputs():
    """bf16 mode returns the RNE bf16 value of the fp32 result (same arithmetic)."""
    inp = make(1, 2, 2, 64, 64, dtype="bf16", seed=8)
    o32, lse32 = orc.attn_fwd(inp["q"], inp["k"], inp["v"], out_bf16=False)
    o16, lse16 = orc.attn_fwd(inp["q"], inp["k"], inp["v"], out_bf16=True)
    from open_transformers_amd import synthetic

    assert_bits_equal(o16, synthetic.round_to_bf16(o32), "O bf16")
    assert_bits_equal(lse16, lse32, "LSE")


def test_causality():
    inp = make(1, 2, 2, 128, 64, dtype="bf16", seed=5)
    o, lse = orc.attn_fwd(inp["q"], inp["k"], inp["v"], out_bf16=True)
    k2, v2 = inp["k"].copy(), inp["v"].copy()
    k2[:, :, 70:] = -k2[:, :, 70:]
    v2[:, :, 70:] = 7.0
    o2, lse2 = orc.attn_fwd(inp["q"], k2, v2, out_bf16=True)
    assert_bits_equal(o2[:, :, :70], o[:, :, :70], "O rows before the change")
    assert_bits_equal(lse2[:, :, :70], lse[:, :, :70], "LSE rows before the change")
    assert not np.array_equal(o2[:, :, 70:], o[:, :, 70:])


def test_window_equals_explicit_mask_math():
    inp = make(1, 2, 2, 128, 64, dtype="f32", seed=6)
    got = oracle_fwd_bwd(inp, 64, bf16=False)
    ref = _torch_ref(inp["q"], inp["k"], inp["v"], inp["do"], 64)
    np.testing.assert_allclose(got["o"], ref[0], atol=2e-5)
    # rows whose window starts exactly at a block edge see 64 keys
    full = oracle_fwd_bwd(inp, 0, bf16=False)
    assert not np.array_equal(got["o"][:, :, 64:], full["o"][:, :, 64:])
    assert_bits_equal(got["o"][:, :, :64], full["o"][:, :, :64], "rows inside the window")


def test_batch_and_thread_invariance():
    big = make(3, 2, 2, 96, 64, dtype="bf16", seed=12)
    one = make(1, 2, 2, 96, 64, dtype="bf16", seed=12)
    for name in ("q", "k", "v", "do"):
        assert_bits_equal(big[name][0:1], one[name], f"input {name} of sequence 0")
    r_big = oracle_fwd_bwd(big, 0, True, nthreads=8)
    r_one = oracle_fwd_bwd(one, 0, True, nthreads=1)
    for name in ("o", "lse", "dq", "dk", "dv"):
        assert_bits_equal(r_big[name][0:1], r_one[name], f"{name}: B=3/8 threads vs B=1/1 thread")


def test_gqa_equals_mha_with_duplicated_kv():
    gqa = make(1, 4, 2, 64, 64, dtype="bf16", seed=13)
    mha = dict(gqa)
    mha["k"] = np.repeat(gqa["k"], 2, axis=1)
    mha["v"] = np.repeat(gqa["v"], 2, axis=1)
    rg = oracle_fwd_bwd(gqa, 0, True)
    rm = oracle_fwd_bwd(mha, 0, True)
    for name in ("o", "lse", "dq"):
        assert_bits_equal(rg[name], rm[name], f"{name}: GQA vs MHA")
    # dK/dV of a group = the group's heads folded in order; check the math
    np.testing.assert_allclose(rg["dv"][:, 0], rm["dv"][:, 0] + rm["dv"][:, 1], rtol=0, atol=3e-2)


def test_zero_upstream_gradient():
    inp = make(1, 2, 2, 64, 64, dtype="bf16", seed=14)
    inp["do"] = np.zeros_like(inp["do"])
    r = oracle_fwd_bwd(inp, 0, True)
    for name in ("dq", "dk", "dv"):
        assert not np.any(r[name]), name


def test_oracle_rejects_bad_shapes():
    x = np.zeros((1, 1, 33, 64), dtype=np.float32)
    with pytest.raises(ValueError):
        orc.attn_fwd(x, x, x)
    y = np.zeros((1, 1, 64, 64), dtype=np.float32)
    with pytest.raises(ValueError):
        orc.attn_fwd(y, y, y, window=48)
