"""Helpers shared by the attention tests (inputs, GPU calls, byte comparison)."""

from __future__ import annotations

import numpy as np

from oracle import oracle as orc
from open_transformers_amd import synthetic


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bits_equal(got: np.ndarray, ref: np.ndarray, what: str) -> None:
    g, r = bits(got), bits(ref)
    assert g.shape == r.shape, f"{what}: shape {g.shape} vs {r.shape}"
    if not np.array_equal(g, r):
        bad = np.flatnonzero(g.ravel() != r.ravel())
        idx = np.unravel_index(bad[0], g.shape)
        raise AssertionError(
            f"{what}: {bad.size} of {g.size} elements differ; first at {idx}: "
            f"got {np.asarray(got)[idx]!r} ({g[idx]:#010x}) want {np.asarray(ref)[idx]!r} ({r[idx]:#010x})"
        )


def assert_bits_equal_nan_class(got: np.ndarray, ref: np.ndarray, what: str) -> None:
    """Every non-NaN element bit for bit, and NaN exactly where the reference has NaN
    (the sign and payload of a NaN are not part of the contract)."""
    g, r = np.asarray(got, dtype=np.float32), np.asarray(ref, dtype=np.float32)
    assert g.shape == r.shape, f"{what}: shape {g.shape} vs {r.shape}"
    gn, rn = np.isnan(g), np.isnan(r)
    if not np.array_equal(gn, rn):
        bad = np.flatnonzero(gn.ravel() != rn.ravel())
        idx = np.unravel_index(bad[0], g.shape)
        raise AssertionError(f"{what}: NaN at {bad.size} differing positions; first at {idx}: got {g[idx]!r} "
                             f"want {r[idx]!r} ({int(gn.sum())} NaN against {int(rn.sum())})")
    keep = ~gn
    assert_bits_equal(np.where(keep, g, 0.0).astype(np.float32), np.where(keep, r, 0.0).astype(np.float32), what)


def oracle_fwd_bwd(inp: dict, window: int, bf16: bool, nthreads: int = 0):
    o, lse = orc.attn_fwd(inp["q"], inp["k"], inp["v"], window=window, out_bf16=bf16, nthreads=nthreads)
    dq, dk, dv = orc.attn_bwd(inp["q"], inp["k"], inp["v"], o, lse, inp["do"], window=window, out_bf16=bf16,
                              nthreads=nthreads)
    return {"o": o, "lse": lse, "dq": dq, "dk": dk, "dv": dv}


def gpu_fwd_bwd(inp: dict, window: int, bf16: bool, variant: int = 0, device: str = "cuda:0",
                score_cache: bool = False):
    """GPU forward + backward through the C ABI; with ``score_cache`` (bf16) the
    forward stores its scores and the backward reads them instead of
    recomputing Q K^T."""
    import torch
    from open_transformers_amd.nn.flash_attention import (flash_attention_backward, flash_attention_forward,
                                                          flash_attention_forward_sc)

    dt = torch.bfloat16 if bf16 else torch.float32
    t = {n: torch.from_numpy(np.ascontiguousarray(inp[n])).to(dt).to(device) for n in ("q", "k", "v", "do")}
    sc = None
    if score_cache:
        o, lse, sc = flash_attention_forward_sc(t["q"], t["k"], t["v"], window=window, variant=variant)
    else:
        o, lse = flash_attention_forward(t["q"], t["k"], t["v"], window=window, variant=variant)
    dq, dk, dv = flash_attention_backward(t["q"], t["k"], t["v"], o, lse, t["do"], window=window, variant=variant,
                                          score_cache=sc)
    torch.cuda.synchronize()
    out = {"o": o, "lse": lse, "dq": dq, "dk": dk, "dv": dv}
    return {n: x.float().cpu().numpy() for n, x in out.items()}


def make(B, H, Hkv, S, D, dtype="bf16", seed=0, rope_theta=None, qk_scale=None):
    return synthetic.make_inputs(B, H, Hkv, S, D, dtype=dtype, seed=seed, rope_theta=rope_theta, qk_scale=qk_scale)
