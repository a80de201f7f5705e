"""GPU parity of the int8-PV forward (int8pv_causal_flash_attention) and of its
straight-through backward, byte for byte against the CPU oracle.

  quantized V    the workspace the library fills (int8 V^T per key block and
                 one binary32 step per (key block, column)) equals the
                 oracle's quantizer, including zero and non-finite columns.
  forward        O and LSE for head dims 64 and 128, GQA / MQA, sliding
                 windows, odd block counts and every launch variant; LSE is
                 also bit-identical to the binary32 forward's.
  backward       autograd through the operator gives the binary32 flash
                 backward evaluated at the int8-PV forward's O and LSE.
  production     the OPEN-1B attention shape (H16, Hkv 4, D128, window 512,
                 S2048), all heads, against the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from attn_util import assert_bits_equal, make
from oracle import oracle as orc
from open_transformers_amd import _lib
from open_transformers_amd.nn import flash_attention as fa

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _gpu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).to(DEV)


def _host(t):
    return t.detach().float().cpu().numpy()


def test_quantized_v_workspace_matches_oracle():
    B, H, Hkv, S, D = 2, 2, 2, 96, 128
    inp = make(B, H, Hkv, S, D, seed=31)
    v = inp["v"].copy()
    v[0, 0, 32:64, 7] = 0.0  # a zero block column
    v[1, 1, 5, 9] = np.inf   # a non-finite block column
    q, k, vv = _gpu(inp["q"]), _gpu(inp["k"]), _gpu(v)
    o = torch.empty_like(q)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=DEV)
    n = fa.int8pv_workspace_bytes(B, H, Hkv, S, D)
    ws = torch.zeros(n, dtype=torch.uint8, device=DEV)
    lib = _lib.load()
    rc = lib.otx_attn_fwd_int8pv(q.data_ptr(), k.data_ptr(), vv.data_ptr(), o.data_ptr(), lse.data_ptr(), B, H, Hkv,
                                 S, D, 0, _lib.DTYPE_BF16, ws.data_ptr(), n, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "otx_attn_fwd_int8pv")
    torch.cuda.synchronize()
    raw = ws.cpu().numpy()
    nq = B * Hkv * S * D
    qvt = raw[:nq].view(np.int8).reshape(B, Hkv, S // 32, D, 32)
    off = (nq + 255) // 256 * 256
    step = raw[off:off + B * Hkv * (S // 32) * D * 4].view(np.float32).reshape(B, Hkv, S // 32, D)
    rq, rs = orc.quantize_v(v)
    want_qvt = rq.reshape(B, Hkv, S // 32, 32, D).transpose(0, 1, 2, 4, 3)
    assert np.array_equal(qvt, want_qvt)
    assert_bits_equal(step, rs, "V steps")


# (B, H, Hkv, S, D, window, seed)
CASES = [
    pytest.param(1, 2, 2, 128, 128, 0, 1, id="d128"),
    pytest.param(1, 2, 2, 128, 64, 0, 2, id="d64"),
    pytest.param(2, 4, 2, 160, 128, 64, 3, id="gqa2-win64-odd-blocks"),
    pytest.param(1, 4, 1, 96, 64, 32, 4, id="mqa-win32-d64"),
    pytest.param(1, 2, 1, 1024, 128, 128, 5, id="gqa-win128-s1024"),
    pytest.param(1, 1, 1, 32, 128, 0, 6, id="single-block"),
]


@pytest.mark.parametrize("B,H,Hkv,S,D,window,seed", CASES)
def test_int8pv_fwd_bwd_bitexact(B, H, Hkv, S, D, window, seed):
    print(f"int8pv case B={B} H={H} Hkv={Hkv} S={S} D={D} window={window} seed={seed}", flush=True)
    inp = make(B, H, Hkv, S, D, seed=seed)
    ro, rl = orc.attn_fwd_int8pv(inp["q"], inp["k"], inp["v"], window=window)
    q, k, v = (_gpu(inp[n]) for n in ("q", "k", "v"))
    for variant in (0, 1, 2):
        o, lse = fa.int8pv_flash_attention_forward(q, k, v, window=window, variant=variant)
        torch.cuda.synchronize()
        assert_bits_equal(_host(o), ro, f"O (variant {variant})")
        assert_bits_equal(_host(lse), rl, f"LSE (variant {variant})")
    _, lse32 = fa.flash_attention_forward(q, k, v, window=window)
    assert_bits_equal(_host(lse32), rl, "LSE of the binary32 forward")
    # the score cache of the int8-PV forward is the binary32 forward's (same scores)
    for variant in (0, 1, 2):
        o8, l8, sc8 = fa.int8pv_flash_attention_forward_sc(q, k, v, window=window, variant=variant)
        _, _, sc32 = fa.flash_attention_forward_sc(q, k, v, window=window, variant=variant)
        torch.cuda.synchronize()
        assert_bits_equal(_host(o8), ro, f"O with score cache (variant {variant})")
        assert_bits_equal(_host(l8), rl, f"LSE with score cache (variant {variant})")
        assert torch.equal(sc8.view(torch.int32), sc32.view(torch.int32)), f"score caches differ (variant {variant})"
    # straight-through backward through autograd
    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
    out = fa.int8pv_causal_flash_attention(qg, kg, vg, window=window)
    out.backward(_gpu(inp["do"]))
    torch.cuda.synchronize()
    assert_bits_equal(_host(out), ro, "autograd O")
    dq, dk, dv = orc.attn_bwd(inp["q"], inp["k"], inp["v"], ro, rl, inp["do"], window=window, out_bf16=True)
    assert_bits_equal(_host(qg.grad), dq, "dq")
    assert_bits_equal(_host(kg.grad), dk, "dk")
    assert_bits_equal(_host(vg.grad), dv, "dv")


def test_int8pv_subnormal_outputs():
    """V scaled into the bf16 subnormal range: O below the binary32 normal range,
    where the forward's reciprocal quotient takes the division; against the oracle."""
    from open_transformers_amd import synthetic

    inp = make(1, 2, 2, 128, 128, seed=22)
    inp["v"] = synthetic.round_to_bf16(inp["v"] * np.float32(2.0 ** -128))
    ro, rl = orc.attn_fwd_int8pv(inp["q"], inp["k"], inp["v"], window=0)
    assert (np.abs(ro) < np.float32(2.0 ** -126)).mean() > 0.9
    q, k, v = (_gpu(inp[n]) for n in ("q", "k", "v"))
    for variant in (0, 1, 2):
        o, lse = fa.int8pv_flash_attention_forward(q, k, v, window=0, variant=variant)
        torch.cuda.synchronize()
        assert_bits_equal(_host(o), ro, f"O (variant {variant})")
        assert_bits_equal(_host(lse), rl, f"LSE (variant {variant})")


def test_int8pv_tiny_block_maxima():
    """Q scaled by 60 (scores spread over hundreds): many (query, key block) pairs
    have a probability maximum below 127 / FLT_MAX, where 127/pmax overflows and
    the contract clamps the quantized probabilities (127, or 0 for p = 0); V is
    O(1), and the V of one block is scaled down as far for the V quantizer's own
    clamp.  O and LSE against the oracle."""
    from open_transformers_amd import synthetic

    inp = make(1, 2, 2, 256, 128, seed=23)
    inp["q"] = synthetic.round_to_bf16(inp["q"] * np.float32(60.0))
    inp["v"][:, :, 32:64, :] = synthetic.round_to_bf16(inp["v"][:, :, 32:64, :] * np.float32(2.0 ** -128))
    # reached: blocks whose maximum probability, exp(block max - running max), is below 127 / FLT_MAX
    sig = 1.0 / np.sqrt(128.0)
    s = np.einsum("bhqd,bhkd->bhqk", inp["q"].astype(np.float64), inp["k"].astype(np.float64)) * sig
    tiny = 0
    for qi in range(256):
        for kb in range(qi // 32 + 1):
            hi = min(32 * kb + 32, qi + 1)
            run = s[..., qi, :hi].max(axis=-1)
            tiny += int(np.sum(np.exp(s[..., qi, 32 * kb:hi].max(axis=-1) - run) < 127.0 / 3.4028234663852886e38))
    assert tiny > 50
    ro, rl = orc.attn_fwd_int8pv(inp["q"], inp["k"], inp["v"], window=0)
    q, k, v = (_gpu(inp[n]) for n in ("q", "k", "v"))
    for variant in (0, 1, 2):
        o, lse = fa.int8pv_flash_attention_forward(q, k, v, window=0, variant=variant)
        torch.cuda.synchronize()
        assert_bits_equal(_host(o), ro, f"O (variant {variant})")
        assert_bits_equal(_host(lse), rl, f"LSE (variant {variant})")


def test_int8pv_nan_in_k():
    """A NaN key: NaN exactly where the oracle has NaN in O and LSE (the rows that
    see the key), every other element bit for bit."""
    from attn_util import assert_bits_equal_nan_class

    inp = make(1, 2, 2, 128, 128, seed=24)
    inp["k"][0, 0, 40, 5] = np.nan
    ro, rl = orc.attn_fwd_int8pv(inp["q"], inp["k"], inp["v"], window=0)
    assert np.isnan(rl).sum() == 88
    q, k, v = (_gpu(inp[n]) for n in ("q", "k", "v"))
    o, lse = fa.int8pv_flash_attention_forward(q, k, v, window=0)
    torch.cuda.synchronize()
    assert_bits_equal_nan_class(_host(o), ro, "O")
    assert_bits_equal_nan_class(_host(lse), rl, "LSE")


def test_int8pv_open1b_shape_all_heads():
    """H16 Hkv4 D128 window 512 S2048 (configs/model/llama3_1b_proxy_repop.yaml),
    RoPE'd inputs, B=1: every head against the oracle."""
    print("int8pv OPEN-1B attention shape B1 H16 Hkv4 S2048 D128 window 512", flush=True)
    inp = make(1, 16, 4, 2048, 128, seed=41, rope_theta=500000.0)
    ro, rl = orc.attn_fwd_int8pv(inp["q"], inp["k"], inp["v"], window=512)
    o, lse = fa.int8pv_flash_attention_forward(*(_gpu(inp[n]) for n in ("q", "k", "v")), window=512)
    torch.cuda.synchronize()
    assert_bits_equal(_host(o), ro, "O")
    assert_bits_equal(_host(lse), rl, "LSE")


def test_int8pv_rejects_fp32():
    q = torch.zeros(1, 1, 32, 64, device=DEV)
    with pytest.raises(ValueError, match="bfloat16"):
        fa.int8pv_causal_flash_attention(q, q, q)
