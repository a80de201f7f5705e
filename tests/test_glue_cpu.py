"""CPU pins of the closed forms the fused layer kernels implement.

The decoder layer's RoPE + head layout (rope.py:103-125 followed by
attention_repop.py:143-149) and its SwiGLU product (ffn_repop.py:52-54) are
torch compositions in the reference, so their bytes are what torch's forward
and autograd backward give.  ``csrc/rope.hip`` and ``swiglu_*_kernel`` in
``csrc/norm_act.hip`` compute them from closed forms (stated in
include/otx_attn.h).  These tests restate those closed forms in numpy and check
them against torch's own composition on the CPU, bit for bit, on random,
signed-zero, subnormal, large and tie-prone inputs.  A mistake in the
derivation (a dropped per-branch rounding, the wrong sign branch, the -0 -> +0
rule of the slice-gradient sum) fails here without a GPU; the GPU tests then
compare the kernels with the same compositions.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from layer_ref import apply_rope, rope_heads_ref, swiglu_ref
from open_transformers_amd import synthetic
from open_transformers_amd.nn.layer import rope_tables
from oracle import oracle as orc


def rnd(x: np.ndarray, bf16: bool) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    return synthetic.round_to_bf16(x) if bf16 else x


def bits(a) -> np.ndarray:
    a = a.detach().float().numpy() if isinstance(a, torch.Tensor) else np.asarray(a, np.float32)
    return a.view(np.uint32)


def rope_closed_form(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, g: np.ndarray, bf16: bool):
    """Forward y [B, H, T, D] and backward dx [B, T, H, D] as the kernels compute them."""
    f = np.float32
    e, o = x[..., 0::2], x[..., 1::2]
    c, s = cos[None, :, None, :], sin[None, :, None, :]
    y = np.empty_like(x)
    y[..., 0::2] = rnd(f(e * c) - f(o * s), bf16)
    y[..., 1::2] = rnd(f(e * s) + f(o * c), bf16)
    gt = g.transpose(0, 2, 1, 3)  # [B, T, H, D]
    ge, go = gt[..., 0::2], gt[..., 1::2]
    dx = np.empty_like(x)
    dx[..., 0::2] = rnd(rnd(f(ge * c), bf16) + rnd(f(go * s), bf16), bf16) + f(0.0)
    dx[..., 1::2] = rnd(rnd(f(-ge * s), bf16) + rnd(f(go * c), bf16), bf16) + f(0.0)
    return y.transpose(0, 2, 1, 3), dx


def special_values(rng, shape, bf16: bool) -> np.ndarray:
    v = rng.standard_normal(shape).astype(np.float32)
    flat = v.reshape(-1)
    n = flat.size
    picks = rng.integers(0, n, n // 4)
    kinds = rng.integers(0, 6, picks.size)
    tiny = np.float32(2.0 ** -130 if not bf16 else 2.0 ** -128)
    table = np.array([0.0, -0.0, tiny, -tiny, 3.0e37, 1.0 + 2.0 ** -8], dtype=np.float32)
    flat[picks] = table[kinds]
    return rnd(v, bf16)


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("shape", [(2, 24, 3, 16), (1, 40, 2, 128)])
def test_rope_heads_closed_form_matches_torch(bf16, shape):
    B, T, H, D = shape
    rng = np.random.default_rng(11 + D + int(bf16))
    cos, sin = (t.numpy() for t in rope_tables(T, D, 500000.0))
    x = special_values(rng, shape, bf16)
    g = special_values(rng, (B, H, T, D), bf16)
    g.reshape(-1)[: D] = -0.0  # every pair of one row: both branches -0
    dt = torch.bfloat16 if bf16 else torch.float32
    xt = torch.from_numpy(x).to(dt).requires_grad_(True)
    y = rope_heads_ref(xt, torch.from_numpy(cos), torch.from_numpy(sin))
    y.backward(torch.from_numpy(g).to(dt))
    y_cf, dx_cf = rope_closed_form(x, cos, sin, g, bf16)
    assert np.array_equal(bits(y), bits(y_cf))
    assert np.array_equal(bits(xt.grad), bits(dx_cf))


def test_rope_gradient_zero_sign_rule():
    """The slice gradients are summed as full tensors holding +0 elsewhere, so a
    -0 branch sum is stored as +0 (the closed form's z()); without that rule the
    all -0 row would keep -0."""
    x = torch.zeros(1, 1, 1, 8, dtype=torch.bfloat16, requires_grad=True)
    cos = torch.ones(1, 4)
    sin = torch.full((1, 4), 0.5)
    y = apply_rope(x, cos, sin)
    y.backward(torch.full_like(y, -0.0))
    assert np.all(bits(x.grad) == 0)  # +0, not 0x80000000


@pytest.mark.parametrize("bf16", [True, False])
def test_swiglu_closed_form_matches_torch(bf16):
    rng = np.random.default_rng(5 + int(bf16))
    rows, F = 6, 32
    gu = special_values(rng, (rows, 2 * F), bf16)
    gu[:, :F] = np.clip(gu[:, :F], -80.0, 80.0)  # SiLU's input range of interest
    dh = special_values(rng, (rows, F), bf16)
    dt = torch.bfloat16 if bf16 else torch.float32
    gt = torch.from_numpy(gu).to(dt).requires_grad_(True)
    h = swiglu_ref(gt)
    h.backward(torch.from_numpy(dh).to(dt))
    gate, up = gu[:, :F], gu[:, F:]
    with np.errstate(over="ignore"):  # huge up or dh values overflow to inf, as in torch
        y = orc.silu_fwd(gate, out_bf16=bf16)
        h_cf = rnd(np.float32(y * up), bf16)
        gy = rnd(np.float32(dh * up), bf16)
        dgu_cf = np.concatenate([orc.silu_bwd(gate, gy, out_bf16=bf16), rnd(np.float32(dh * y), bf16)], axis=1)
    assert np.array_equal(bits(h), bits(h_cf))
    assert np.array_equal(bits(gt.grad), bits(dgu_cf))
