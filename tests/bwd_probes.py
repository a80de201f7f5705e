"""Closed-form probes of the backward's bit-level rules (oracle/attn_oracle.c,
contract lines "Backward: ...").

Each probe is a small input whose expected bits follow from the contract by
hand, and for which the plausible one-line deviations give different bits:

  gqa_order     dV folds over the query heads of a GQA group first, then the
                queries: with P = 1, dO = 1 (head 0, query 1), 2^24 (head 1,
                query 0), -2^24 (head 2, query 0), the serial fold gives
                1 + 2^24 = 2^24 (tie to even) - 2^24 = 0; queries-outer or a
                reversed head order keep the 1.
  query_order   dV folds query blocks ascending, then queries ascending:
                2^24 (query 1) + 1 (query 33) - 2^24 (query 65) = 0 across
                blocks (column d = 0) and 2^24 + 1 - 2^24 = 0 inside one block
                (queries 34, 35, 36; column d = 1); any other association
                keeps the 1.
  dsum_stored_o Dsum is the dot of dO with the O passed to the backward (the
                stored output): with dO_0 = e_0, V_0 = 3 e_0 and O_0 = 1.5 e_0
                row 0 (one key) gives dS = 3 - 1.5 and dQ_0 = 1.5 / 8; a Dsum
                recomputed from P V would give 0.
  sigma_once    dK = RN(sigma * fold), sigma = RN(1/sqrt(128)) applied once
                after the fold: dS = 2^20, 1, -2^20 fold to exactly 1, so
                dK = sigma; sigma applied per term (or to dS or q before the
                fold) leaves sigma on the binary32 grid of sigma 2^20.
  ds_rounding   dS = RN(P * RN(dP - Dsum)): (P, dP, Dsum) found so that it
                differs from RN(P (dP - Dsum)) (no intermediate rounding),
                RN(RN(P dP) - RN(P Dsum)) and fma(P, dP, -RN(P Dsum)); observed
                through dQ_0 = dS / 8 and, on the GPU, the workspace's dS tile.

Scores are steered exactly: q or k is zero where a score must be 0, and the
backward takes LSE as an input, so P = exp(RN(0 - LSE)) is 1 for LSE = 0.
All values are bf16-exact, so the same arrays serve the binary32 and the bf16
kernels.  The expected values below are hand-derived numbers or searches over
the deviations' formulas, not a second copy of the oracle.
"""

from __future__ import annotations

import math

import numpy as np

F32 = np.float32


def _zeros(B, H, Hkv, S, D):
    return {
        "q": np.zeros((B, H, S, D), F32), "k": np.zeros((B, Hkv, S, D), F32), "v": np.zeros((B, Hkv, S, D), F32),
        "o": np.zeros((B, H, S, D), F32), "lse": np.zeros((B, H, S), F32), "do": np.zeros((B, H, S, D), F32),
    }


def _bf16_exact(x) -> bool:
    u = np.asarray(x, F32).reshape(-1).view(np.uint32)
    return bool(np.all((u & 0xFFFF) == 0))


def gqa_order():
    p = _zeros(1, 3, 1, 32, 64)
    p["v"][0, 0, :, 0] = 1.0
    p["do"][0, 0, 1, :] = 1.0
    p["do"][0, 1, 0, :] = 2.0**24
    p["do"][0, 2, 0, :] = -(2.0**24)
    return p


def check_gqa_order(out):
    dv = out["dv"]
    assert np.all(dv[0, 0, 0, :] == 0.0), f"dV_0 = {dv[0, 0, 0, :4]} (heads then queries gives 0)"
    # sensitivity: queries outer (query 0 of heads 1, 2 first) or heads reversed keep the 1
    assert F32(F32(F32(0.0) + F32(2.0**24)) - F32(2.0**24)) + F32(1.0) == 1.0


def query_order():
    p = _zeros(1, 1, 1, 96, 64)
    p["do"][0, 0, 1, 0] = 2.0**24
    p["do"][0, 0, 33, 0] = 1.0
    p["do"][0, 0, 65, 0] = -(2.0**24)
    p["do"][0, 0, 34, 1] = 2.0**24
    p["do"][0, 0, 35, 1] = 1.0
    p["do"][0, 0, 36, 1] = -(2.0**24)
    return p


def check_query_order(out, bf16: bool):
    dv = out["dv"]
    assert dv[0, 0, 0, 0] == 0.0 and dv[0, 0, 0, 1] == 0.0, f"dV_0[:2] = {dv[0, 0, 0, :2]}"
    assert dv[0, 0, 32, 1] == 0.0, f"dV_32[1] = {dv[0, 0, 32, 1]}"
    # key 32 sees queries 32..95: 1 (query 33) - 2^24 (query 65) in column 0
    want = F32(1.0 - 2.0**24)
    assert dv[0, 0, 32, 0] == (_to_bf16(want) if bf16 else want)
    # sensitivity: (block 1 + block 2) first, or the in-block sum reversed, gives 1
    assert F32(F32(2.0**24) + F32(F32(1.0) - F32(2.0**24))) == 1.0


def dsum_stored_o():
    p = _zeros(1, 1, 1, 32, 64)
    p["k"][0, 0, 0, 0] = 1.0      # key 0 = e_0 (q = 0 keeps every score 0)
    p["v"][0, 0, 0, 0] = 3.0      # V_0 = 3 e_0
    p["do"][0, 0, 0, 0] = 1.0     # dO_0 = e_0: dP_00 = 3
    p["o"][0, 0, 0, 0] = 1.5      # stored O_0 = 1.5 e_0: Dsum_0 = 1.5
    return p


def check_dsum_stored_o(out):
    assert out["dq"][0, 0, 0, 0] == F32(0.1875), f"dQ_0[0] = {out['dq'][0, 0, 0, 0]!r} (want 1.5 / 8)"
    if "ds" in out:
        assert out["ds"][0, 0, 0] == F32(1.5)


def _sigma(D):
    return F32(1.0 / math.sqrt(D))


def sigma_once():
    """dS_i0 = 2^20, 1, -2^20 for queries 0, 1, 2 and q_i = e_0 there: the fold
    is RN(RN(2^20 + 1) - 2^20) = 1 exactly, so dK_0[0] = RN(sigma * 1) = sigma.
    With sigma applied per term (or to dS, or to q, before the fold) the sum
    RN(RN(sigma 2^20) + RN(sigma)) keeps sigma only to the binary32 grid at
    sigma 2^20 (steps of 2^-7), which the cancellation then exposes: an error
    of percents, visible in bf16 too."""
    s = _sigma(128)
    xs = (2.0**20, 1.0, -(2.0**20))
    p = _zeros(1, 1, 1, 32, 128)      # k = 0: every score 0, LSE = 0: P = 1
    p["v"][0, 0, 0, 0] = 1.0          # dP_i0 = dO_i[0]; O = 0: Dsum = 0; dS_i0 = dO_i[0]
    for i, x in enumerate(xs):
        p["do"][0, 0, i, 0] = x
        p["q"][0, 0, i, 0] = 1.0
    per = F32(0.0)
    for x in xs:
        per = F32(per + F32(s * F32(x)))
    p["_want"] = s
    p["_deviation"] = per
    return p


def check_sigma_once(out, p, bf16: bool):
    got = out["dk"][0, 0, 0, 0]
    want, dev = p["_want"], p["_deviation"]
    if bf16:
        want, dev = _to_bf16(want), _to_bf16(dev)
    assert want != dev
    assert got == want, f"dK_0[0] = {got!r}, want RN(sigma * fold) = {want!r} (sigma per term: {dev!r})"


def _to_bf16(x):
    u = np.asarray([x], F32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16).view(F32)[0]


def ds_rounding_case():
    """(L, a, b) with P = RN(exp(-L)) and dS = RN(P RN(a - b)) different from the
    three deviations; a, b bf16."""
    from oracle import oracle as orc

    for L in (0.5, 0.75, 1.25, 0.375, 2.5):
        P = F32(orc.expf(F32(-L)))
        assert P == F32(math.exp(-L))  # an argument far from a rounding boundary
        for ka in range(1, 128):
            a = F32(1.0 + ka * 2.0**-7)
            for eb in range(22, 27):  # a - b inexact in binary32, exact in binary64 with P (a - b)
                for mb in (1.0, 1.5, 1.25, 1.75):
                    b = F32(mb * 2.0**-eb)
                    want = F32(P * F32(a - b))
                    d1 = F32(float(P) * (float(a) - float(b)))          # no intermediate rounding (exact in binary64)
                    d2 = F32(F32(P * a) - F32(P * b))
                    d3 = F32(float(P) * float(a) - float(F32(P * b)))   # fma(P, a, -RN(P b)), exact in binary64
                    if want != d1 and want != d2 and want != d3:
                        return float(L), float(a), float(b), want, (d1, d2, d3)
    raise AssertionError("no probe case found")


def ds_rounding():
    L, a, b, want, devs = ds_rounding_case()
    p = _zeros(1, 1, 1, 32, 64)
    p["k"][0, 0, 0, 0] = 1.0          # q = 0: s_00 = 0; k_0 = e_0: dQ_0[0] = RN(sigma dS_00)
    p["v"][0, 0, 0, 0] = a            # dO_0 = e_0: dP_00 = a
    p["o"][0, 0, 0, 0] = b            # Dsum_0 = b
    p["do"][0, 0, 0, 0] = 1.0
    p["lse"][0, 0, :] = L             # P_00 = exp(RN(0 - L))
    p["_want"] = want
    p["_deviations"] = devs
    return p


def check_ds_rounding(out, p, bf16: bool):
    want = p["_want"]
    for d in p["_deviations"]:
        assert d != want
    if "ds" in out:
        assert out["ds"][0, 0, 0] == want, f"dS_00 = {out['ds'][0, 0, 0]!r}, want {want!r}"
    if not bf16:
        assert out["dq"][0, 0, 0, 0] == F32(want * F32(0.125)), f"dQ_0[0] = {out['dq'][0, 0, 0, 0]!r}"


def all_probes(bf16: bool):
    """[(name, inputs, check(out))] for one dtype."""
    sg = sigma_once()
    ds = ds_rounding()
    return [
        ("gqa_order", gqa_order(), lambda out: check_gqa_order(out)),
        ("query_order", query_order(), lambda out: check_query_order(out, bf16)),
        ("dsum_stored_o", dsum_stored_o(), lambda out: check_dsum_stored_o(out)),
        ("sigma_once", sg, lambda out: check_sigma_once(out, sg, bf16)),
        ("ds_rounding", ds, lambda out: check_ds_rounding(out, ds, bf16)),
    ]


def arrays(p):
    return {n: p[n] for n in ("q", "k", "v", "o", "lse", "do")}


def assert_inputs_bf16_exact(p):
    for n in ("q", "k", "v", "o", "do"):
        assert _bf16_exact(p[n]), n
