"""GPU parity: every output byte of the gfx950 kernels equals the CPU oracle.

Forward O and LSE and backward dQ, dK, dV are compared bit for bit (no
tolerance) on seeded inputs, across dtypes, head dims, GQA groupings, sliding
windows, block counts that are not a multiple of the workgroup tile, and every
launch variant, with bf16 inputs both through the score-recomputing backward
and through the score cache.  BASELINE configuration 1 (B1 H4 S256 D64 fp32) runs at full
size; the larger configurations are checked on head slices here and through
size-independent properties in test_gpu_invariance.py.
"""

from __future__ import annotations

import numpy as np
import pytest

from attn_util import assert_bits_equal, assert_bits_equal_nan_class, gpu_fwd_bwd, make, oracle_fwd_bwd

pytestmark = pytest.mark.gpu

# (B, H, Hkv, S, D, window, dtype, seed, qk_scale)
CASES = [
    pytest.param(1, 4, 4, 256, 64, 0, "f32", 1, None, id="c1-fp32-d64"),
    pytest.param(1, 2, 2, 128, 128, 0, "bf16", 2, None, id="bf16-d128-small"),
    pytest.param(2, 4, 2, 160, 128, 64, "bf16", 3, None, id="bf16-gqa2-win64-odd-blocks"),
    pytest.param(1, 4, 1, 96, 64, 32, "bf16", 4, None, id="bf16-mqa-win32-d64"),
    pytest.param(1, 2, 2, 224, 128, 0, "f32", 5, None, id="fp32-d128"),
    pytest.param(1, 2, 2, 128, 64, 0, "bf16", 6, None, id="bf16-d64"),
    pytest.param(1, 2, 2, 512, 128, 0, "bf16", 7, 3.0, id="bf16-qk-x3"),
    pytest.param(1, 2, 1, 1024, 128, 128, "bf16", 8, None, id="bf16-gqa-win128-s1024"),
    pytest.param(1, 1, 1, 32, 128, 0, "bf16", 9, None, id="bf16-single-block"),
    pytest.param(1, 2, 2, 64, 64, 32, "f32", 10, 4.0, id="fp32-win32-qk-x4"),
]


@pytest.mark.parametrize("B,H,Hkv,S,D,window,dtype,seed,qk_scale", CASES)
def test_fwd_bwd_bitexact(B, H, Hkv, S, D, window, dtype, seed, qk_scale):
    print(f"case B={B} H={H} Hkv={Hkv} S={S} D={D} window={window} {dtype} seed={seed}", flush=True)
    inp = make(B, H, Hkv, S, D, dtype=dtype, seed=seed, qk_scale=qk_scale)
    bf16 = dtype == "bf16"
    ref = oracle_fwd_bwd(inp, window, bf16)
    for variant in (0, 1, 2):
        for sc in ((False, True) if bf16 else (False,)):
            got = gpu_fwd_bwd(inp, window, bf16, variant=variant, score_cache=sc)
            for name in ("o", "lse", "dq", "dk", "dv"):
                assert_bits_equal(got[name], ref[name], f"{name} (variant {variant}, score cache {sc})")


def test_c2_head_slice_bitexact():
    """BASELINE configuration 2 at full size on the GPU (RoPE'd bf16 inputs);
    the oracle recomputes two (batch, head) slices, which are independent."""
    inp = make(4, 16, 16, 2048, 128, dtype="bf16", seed=11, rope_theta=10000.0)
    got = gpu_fwd_bwd(inp, 0, True)
    cached = gpu_fwd_bwd(inp, 0, True, score_cache=True)
    for name in ("o", "lse", "dq", "dk", "dv"):
        assert_bits_equal(cached[name], got[name], f"c2 {name}: score cache vs recompute")
    for b, h in ((0, 0), (3, 15)):
        sl = {n: np.ascontiguousarray(a[b:b + 1, h:h + 1]) for n, a in inp.items()}
        ref = oracle_fwd_bwd(sl, 0, True)
        for name in ("o", "lse", "dq", "dk", "dv"):
            assert_bits_equal(got[name][b:b + 1, h:h + 1], ref[name], f"c2 {name} (b={b}, h={h})")


@pytest.mark.parametrize("S,window", [(16384, 0), (32768, 512)], ids=["s16k-full", "s32k-win512"])
def test_long_sequence_bitexact(S, window):
    """Long sequences with a GQA group of four (the head-grouped forward and dQ
    workgroups): tile indices, score-cache and dS-tile addresses and the 32-bit
    lane offsets at 16K (full causal, 131,328 tiles per head) and 32K tokens
    (window 512), launch variants 0 and 2, score cache off and on."""
    print(f"long sequence S={S} window={window}", flush=True)
    inp = make(1, 4, 1, S, 128, dtype="bf16", seed=21 + window)
    ref = oracle_fwd_bwd(inp, window, True)
    for variant in (0, 2):
        for sc in (False, True):
            got = gpu_fwd_bwd(inp, window, True, variant=variant, score_cache=sc)
            for name in ("o", "lse", "dq", "dk", "dv"):
                assert_bits_equal(got[name], ref[name], f"S{S} w{window} {name} (variant {variant}, score cache {sc})")


def test_subnormal_outputs_bitexact():
    """V scaled into the bf16 subnormal range, so that O = RN(acc / l) lies below
    the binary32 normal range: there a quotient can be a midpoint exactly, and
    the bf16 forward's reciprocal form takes the division instead (a
    wave-uniform branch).  Forward and backward, every launch variant, with and
    without the score cache, against the oracle."""
    from open_transformers_amd import synthetic

    inp = make(1, 2, 2, 128, 128, dtype="bf16", seed=21)
    inp["v"] = synthetic.round_to_bf16(inp["v"] * np.float32(2.0 ** -128))
    ref = oracle_fwd_bwd(inp, 0, True)
    tiny = np.abs(ref["o"]) < np.float32(2.0 ** -126)
    assert tiny.mean() > 0.9, "the case must put the outputs below the normal range"
    for variant in (0, 1, 2):
        for sc in (False, True):
            got = gpu_fwd_bwd(inp, 0, True, variant=variant, score_cache=sc)
            for name in ("o", "lse", "dq", "dk", "dv"):
                assert_bits_equal(got[name], ref[name], f"{name} (variant {variant}, score cache {sc})")


NONFINITE = [
    pytest.param("q", np.nan, id="nan-in-q"), pytest.param("k", np.nan, id="nan-in-k"),
    pytest.param("v", np.nan, id="nan-in-v"), pytest.param("do", np.nan, id="nan-in-do"),
    pytest.param("q", np.inf, id="inf-in-q"), pytest.param("k", -np.inf, id="minus-inf-in-k"),
]


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("what,val", NONFINITE)
def test_nonfinite_inputs_propagate_like_the_oracle(what, val, dtype):
    """One non-finite input element: NaN exactly where the oracle has NaN in O, LSE,
    dQ, dK and dV (a NaN score reaches the whole row's statistics, as the
    contract's exp carries it into l), and every other element bit for bit; the
    sign and payload of a NaN are not compared."""
    print(f"non-finite {what}={val} {dtype}", flush=True)
    inp = make(1, 2, 2, 128, 128, dtype=dtype, seed=31)
    inp[what][0, 0, 40, 5] = val
    bf16 = dtype == "bf16"
    ref = oracle_fwd_bwd(inp, 0, bf16)
    assert np.isnan(ref["o"]).any() or np.isnan(ref["dq"]).any()
    for sc in ((False, True) if bf16 else (False,)):
        got = gpu_fwd_bwd(inp, 0, bf16, score_cache=sc)
        for name in ("o", "lse", "dq", "dk", "dv"):
            assert_bits_equal_nan_class(got[name], ref[name], f"{name} (score cache {sc})")


def test_overflowing_accumulation_and_wide_windows():
    """V at +-3e38 (the P V and dV folds overflow), and windows of S and beyond (a
    window no smaller than the sequence is full causal)."""
    from open_transformers_amd import synthetic

    inp = make(1, 2, 2, 128, 128, dtype="bf16", seed=32)
    for w in (128, 160, 512):
        ref = oracle_fwd_bwd(inp, w, True)
        for sc in (False, True):
            got = gpu_fwd_bwd(inp, w, True, score_cache=sc)
            for name in ("o", "lse", "dq", "dk", "dv"):
                assert_bits_equal(got[name], ref[name], f"{name} (window {w}, score cache {sc})")
    inp["v"] = synthetic.round_to_bf16(np.sign(inp["v"]) * np.float32(3.0e38))
    ref = oracle_fwd_bwd(inp, 0, True)
    for sc in (False, True):
        got = gpu_fwd_bwd(inp, 0, True, score_cache=sc)
        for name in ("o", "lse", "dq", "dk", "dv"):
            assert_bits_equal_nan_class(got[name], ref[name], f"{name} (V +-3e38, score cache {sc})")

