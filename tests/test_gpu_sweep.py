"""Seeded sweep of small attention shapes on the GPU, each byte-compared with
the CPU oracle (forward O and LSE, backward dQ, dK and dV).

The cases are drawn once from a fixed generator, so the list is the same on
every run: batch 1-3, 1-8 query heads with every divisor of the head count as
KV heads (MHA, GQA, MQA), 1-16 key blocks, D 64 or 128, a sliding window or
full causal, bf16 or binary32 storage, the three launch variants, and for bf16
the score cache on or off.  The inputs are the package's seeded N(0, 1)
generator, some cases scaled so that the scores spread over tens of units
(large softmax ranges, many exps far below the maximum).  A second seeded list
covers the int8-PV forward and the binary32 backward on its outputs, a third
the decoder layer's GEMM in its three operand layouts.
"""
from __future__ import annotations

import random

import numpy as np
import pytest

from attn_util import assert_bits_equal, gpu_fwd_bwd, make, oracle_fwd_bwd

pytestmark = pytest.mark.gpu
NAMES = ("o", "lse", "dq", "dk", "dv")


def _cases(n=32, seed=20261202):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        H = rng.randint(1, 8)
        Hkv = rng.choice([d for d in range(1, H + 1) if H % d == 0])
        nb = rng.randint(1, 16)
        S = 32 * nb
        window = 0 if rng.random() < 0.5 else 32 * rng.randint(1, nb)
        bf16 = rng.random() < 0.75
        out.append(dict(B=rng.randint(1, 3), H=H, Hkv=Hkv, S=S, D=rng.choice([64, 128]), window=window, bf16=bf16,
                        variant=rng.randint(0, 2), cache=bf16 and rng.random() < 0.5,
                        qk_scale=rng.choice([None, None, 4.0]), seed=1000 + i))
    return out


CASES = _cases()


@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(len(CASES))])
def test_gpu_sweep_matches_oracle(case):
    c = case
    print(f"sweep: B{c['B']} H{c['H']} Hkv{c['Hkv']} S{c['S']} D{c['D']} window {c['window']} "
          f"{'bf16' if c['bf16'] else 'fp32'} variant {c['variant']} cache {c['cache']} scale {c['qk_scale']}",
          flush=True)
    inp = make(c["B"], c["H"], c["Hkv"], c["S"], c["D"], dtype="bf16" if c["bf16"] else "f32", seed=c["seed"],
               qk_scale=c["qk_scale"])
    got = gpu_fwd_bwd(inp, c["window"], c["bf16"], variant=c["variant"], score_cache=c["cache"])
    ref = oracle_fwd_bwd(inp, c["window"], c["bf16"])
    for n in NAMES:
        assert np.all(np.isfinite(ref[n]) | np.isneginf(ref[n])), n
        assert_bits_equal(got[n], ref[n], n)


def _int8_cases(n=16, seed=20261203):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        H = rng.randint(1, 8)
        Hkv = rng.choice([d for d in range(1, H + 1) if H % d == 0])
        nb = rng.randint(1, 16)
        window = 0 if rng.random() < 0.5 else 32 * rng.randint(1, nb)
        out.append(dict(B=rng.randint(1, 3), H=H, Hkv=Hkv, S=32 * nb, D=rng.choice([64, 128]), window=window,
                        variant=rng.randint(0, 2), cache=rng.random() < 0.5, seed=2000 + i))
    return out


INT8_CASES = _int8_cases()


@pytest.mark.parametrize("case", INT8_CASES, ids=[f"i{i}" for i in range(len(INT8_CASES))])
def test_gpu_sweep_int8pv_matches_oracle(case):
    """The int8-PV forward (bf16) and the binary32 straight-through backward on
    its O and LSE, against the int8-PV oracle and the backward oracle."""
    import torch

    from oracle import oracle as orc
    from open_transformers_amd.nn import flash_attention as fa

    c = case
    print(f"int8pv sweep: B{c['B']} H{c['H']} Hkv{c['Hkv']} S{c['S']} D{c['D']} window {c['window']} "
          f"variant {c['variant']} cache {c['cache']}", flush=True)
    inp = make(c["B"], c["H"], c["Hkv"], c["S"], c["D"], dtype="bf16", seed=c["seed"])
    t = {n: torch.from_numpy(np.ascontiguousarray(inp[n])).to(torch.bfloat16).to("cuda:0")
         for n in ("q", "k", "v", "do")}
    sc = None
    if c["cache"]:
        o, lse, sc = fa.int8pv_flash_attention_forward_sc(t["q"], t["k"], t["v"], window=c["window"],
                                                          variant=c["variant"])
    else:
        o, lse = fa.int8pv_flash_attention_forward(t["q"], t["k"], t["v"], window=c["window"], variant=c["variant"])
    dq, dk, dv = fa.flash_attention_backward(t["q"], t["k"], t["v"], o, lse, t["do"], window=c["window"],
                                             variant=c["variant"], score_cache=sc)
    torch.cuda.synchronize()
    ro, rl = orc.attn_fwd_int8pv(inp["q"], inp["k"], inp["v"], window=c["window"])
    rdq, rdk, rdv = orc.attn_bwd(inp["q"], inp["k"], inp["v"], ro, rl, inp["do"], window=c["window"], out_bf16=True)
    for name, g, r in (("o", o, ro), ("lse", lse, rl), ("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
        assert_bits_equal(g.float().cpu().numpy(), r, name)


def _gemm_cases(n=12, seed=20261204):
    rng = random.Random(seed)
    return [dict(M=128 * rng.randint(1, 4), N=128 * rng.randint(1, 4), R=32 * rng.randint(1, 32),
                 scale=rng.choice([1.0, 1.0, 30.0]), seed=3000 + i) for i in range(n)]


GEMM_CASES = _gemm_cases()


@pytest.mark.parametrize("case", GEMM_CASES, ids=[f"g{i}" for i in range(len(GEMM_CASES))])
def test_gpu_sweep_gemm_matches_oracle(case):
    """The decoder layer's GEMM in its three operand layouts (y = x w^T, dx = dy w,
    dw = dy^T x) and with a binary32 result, in every tile form, against the
    serial-fold oracle; R covers odd multiples of 32, and some inputs are scaled
    by 30 (large partial sums that cancel)."""
    import torch

    from oracle import oracle as orc
    from open_transformers_amd import synthetic
    from open_transformers_amd.nn import functional as F

    c = case
    M, N, R = c["M"], c["N"], c["R"]
    print(f"gemm sweep: M{M} N{N} R{R} scale {c['scale']}", flush=True)
    rng = np.random.default_rng(c["seed"])
    bf = lambda a: synthetic.round_to_bf16(np.asarray(a, dtype=np.float32))  # noqa: E731
    x = bf(c["scale"] * rng.standard_normal((M, R)))
    w = bf(c["scale"] * rng.standard_normal((N, R)))
    dy = bf(rng.standard_normal((M, N)))
    dev = torch.device("cuda:0")
    gx, gw, gdy = (torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).to(dev) for a in (x, w, dy))
    host = lambda t: t.detach().float().cpu().numpy()  # noqa: E731
    # every tile form (0: the library's choice, 1: 128 x 128, 2: 128 x 64, 3: 64 x 64) gives the oracle's bytes
    y, y32 = orc.gemm(x, w), orc.gemm(x, w, out_bf16=False)
    dx = orc.gemm(dy, w.T) if R % 128 == 0 else None
    dw = orc.gemm(dy.T, x.T) if R % 128 == 0 else None
    for v in (0, 1, 2, 3):
        assert_bits_equal(host(F.gemm_bf16(gx, (R, 1), gw, (R, 1), M, N, R, variant=v)), y, f"y = x w^T, form {v}")
        assert_bits_equal(host(F.gemm_bf16(gx, (R, 1), gw, (R, 1), M, N, R, out_dtype=torch.float32, variant=v)),
                          y32, f"y = x w^T (binary32), form {v}")
        if R % 128 == 0:  # dx and dw put R on an output axis, which must be a multiple of 128
            assert_bits_equal(host(F.gemm_bf16(gdy, (N, 1), gw, (1, R), M, R, N, variant=v)), dx,
                              f"dx = dy w, form {v}")
            assert_bits_equal(host(F.gemm_bf16(gdy, (1, N), gx, (1, R), N, R, M, variant=v)), dw,
                              f"dw = dy^T x, form {v}")
