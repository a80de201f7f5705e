"""A seeded sweep of small attention shapes with extreme input distributions against the
oracle: heavy tails (Cauchy, clipped to +-1e4), per-row scales over e^+-8, sparse spikes
of 60 among values of 0.01, tiny values (2^-60), a third of the values zero, and large
ones (2^40), drawn independently for q, k, v and dO; bf16 and binary32, every launch
variant, windows, GQA, the score cache, and the int8-PV forward on part of the cases.
Every element equal (NaN exactly where the oracle has NaN: huge inputs overflow)."""

from __future__ import annotations

import random

import numpy as np
import pytest

from attn_util import assert_bits_equal_nan_class as eq
from attn_util import gpu_fwd_bwd, make, oracle_fwd_bwd

pytestmark = pytest.mark.gpu
KINDS = ("normal", "cauchy", "rowscale", "spike", "tiny", "zeros", "huge")


def _shape_values(a, kind, nr):
    if kind == "normal":
        return a
    if kind == "cauchy":
        return np.clip(nr.standard_cauchy(a.shape), -1e4, 1e4).astype(np.float32)
    if kind == "rowscale":
        return a * np.exp(nr.uniform(-8, 8, a.shape[:-1] + (1,))).astype(np.float32)
    if kind == "spike":
        b = a * np.float32(0.01)
        idx = nr.integers(0, a.size, max(1, a.size // 500))
        b.reshape(-1)[idx] = nr.choice([-1.0, 1.0], idx.size) * 60.0
        return b
    if kind == "tiny":
        return a * np.float32(2.0 ** -60)
    if kind == "zeros":
        b = a.copy()
        b.reshape(-1)[nr.integers(0, a.size, a.size // 3)] = 0.0
        return b
    return a * np.float32(2.0 ** 40)  # huge


def _cases(n=96, seed=20261203):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        H = rng.randint(1, 6)
        out.append(dict(B=rng.randint(1, 2), H=H, Hkv=rng.choice([d for d in range(1, H + 1) if H % d == 0]),
                        S=32 * rng.randint(1, 8), D=rng.choice([64, 128]), bf16=rng.random() < 0.8,
                        variant=rng.randint(0, 2), window_frac=rng.random(), cache=rng.random() < 0.5,
                        kinds={nm: rng.choice(KINDS) for nm in ("q", "k", "v", "do")}, int8=rng.random() < 0.5,
                        seed=7000 + i))
    return out


CASES = _cases()


@pytest.mark.parametrize("case", CASES, ids=[f"x{i}" for i in range(len(CASES))])
def test_extreme_inputs_match_oracle(case):
    import torch

    from oracle import oracle as orc
    from open_transformers_amd import synthetic
    from open_transformers_amd.nn import flash_attention as fa

    c = case
    nb = c["S"] // 32
    window = 0 if c["window_frac"] < 0.5 else 32 * (1 + int(c["window_frac"] * nb) % nb)
    bf16 = c["bf16"]
    print(f"extremes B{c['B']} H{c['H']} Hkv{c['Hkv']} S{c['S']} D{c['D']} w{window} "
          f"{'bf16' if bf16 else 'fp32'} variant {c['variant']} {c['kinds']}", flush=True)
    inp = make(c["B"], c["H"], c["Hkv"], c["S"], c["D"], dtype="bf16" if bf16 else "f32", seed=c["seed"])
    nr = np.random.default_rng(c["seed"])
    for nm in ("q", "k", "v", "do"):
        x = _shape_values(inp[nm], c["kinds"][nm], nr).astype(np.float32)
        inp[nm] = synthetic.round_to_bf16(x) if bf16 else x
    with np.errstate(all="ignore"):
        ref = oracle_fwd_bwd(inp, window, bf16)
    got = gpu_fwd_bwd(inp, window, bf16, variant=c["variant"], score_cache=bf16 and c["cache"])
    for nm in ("o", "lse", "dq", "dk", "dv"):
        eq(got[nm], ref[nm], nm)
    if bf16 and c["D"] == 128 and c["int8"]:
        with np.errstate(all="ignore"):
            ro, rl = orc.attn_fwd_int8pv(inp["q"], inp["k"], inp["v"], window=window)
        t = {nm: torch.from_numpy(inp[nm]).to(torch.bfloat16).cuda() for nm in ("q", "k", "v")}
        o8, l8 = fa.int8pv_flash_attention_forward(t["q"], t["k"], t["v"], window=window, variant=c["variant"])
        torch.cuda.synchronize()
        eq(o8.float().cpu().numpy(), ro, "int8-PV O")
        eq(l8.cpu().numpy(), rl, "int8-PV LSE")
