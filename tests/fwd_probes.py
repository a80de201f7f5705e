"""Closed-form probes of the forward's online-softmax bookkeeping
(oracle/attn_oracle.c, contract lines "Forward per row i: ...").

Scores are steered exactly: the probed query row is q = e_0 + e_1 + e_2 and
each key k_j = (x, y, z, 0, ...) with bf16 x, y, z chosen so that the serial
fma dot RN(RN(x + y) + z) equals a chosen binary32 value; the score is then
RN(dot * sigma) (sigma = 1/8 exactly at D = 64).  Keys switched off get a
score near -512, whose probability exp(RN(s - m)) is +0.  Every input value
is bf16-exact, so the same arrays serve the binary32 and the bf16 kernels.

Each probe's expected bits follow from the contract written as a few explicit
scalar steps on exact rationals (rn32 below) with the correctly rounded exp
and log (pinned against libquadmath by tests/test_oracle_math.py), and each
probe's inputs are searched so that the plausible deviations give different
bits:

  l_fold        l = RN(l alpha), then + p_j for j ascending, against
                  rowsum  RN(l alpha) + RN(sum of the block's p)
                  fma     fma(l, alpha, sum of the block's p)
                  reverse RN(l alpha), then + p_j for j descending
                block 1 holds 31 probabilities between half and one unit in
                the last place of RN(l alpha) and then the block maximum
                (p = 1); seen in LSE and O.
  acc_rescale   acc = RN(acc alpha), then fma(p_j, v_j, acc) ascending,
                against
                  fused   fma(acc, alpha, RN(p_0 v_0)), then the chain
                  partial RN(RN(acc alpha) + chain from +0)
                  partial_fma fma(acc, alpha, chain from +0)
                column 0 cancels RN(A alpha) down to three units in its last
                place (the unrounded product leaves a different residue);
                column 1 adds and subtracts T = 2^21 ulp(RN(B alpha)), which
                keeps only the top bits of the rescaled value unless the
                block's own sum (T - T = 0) is formed first; seen in O, bf16
                included.
  lse           LSE = RN(m + RN(log l)) with m != 0 and l != 1, against one
                rounding of the binary64 value m + log l.
  exp_argument  p = exp(RN(s - m')) against exp of the exact difference
                (what exp2(fma(s, log2 e, -m' log2 e)) style code computes);
                seen in O (binary32).
  uniform       q = 0: every p is 1, O = RN(serial sum / count), LSE =
                log(count); a multiply by RN(1 / count) in place of the
                division differs on some rows.
  window_edge   window 32, q = 0: rows 32..63 drop block 0's keys; row 63's
                block 0 is fully masked, so m' = m = -inf and alpha must be
                taken as 1 (exp(-inf - -inf) is NaN), and masked keys must be
                skipped rather than given exp(s - m').
"""

from __future__ import annotations

import functools
import math
from fractions import Fraction as Fr

import numpy as np

F32 = np.float32
NEG_DOT = -4096.0  # score about -512 (D 64) or -362 (D 128): exp(RN(s - m)) = +0


# ---------------------------------------------------------------- binary32 on exact rationals
def rn32(x) -> np.float32:
    """The binary32 value nearest to the rational x (ties to even, subnormals
    kept, +0 for an exact zero, infinity past the largest finite value)."""
    x = Fr(x)
    if x == 0:
        return F32(0.0)
    neg = x < 0
    a = -x if neg else x
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fr(2) ** e > a:
        e -= 1
    qexp = max(e - 23, -149)
    scaled = a / Fr(2) ** qexp
    n = scaled.numerator // scaled.denominator
    rem = scaled - n
    if rem > Fr(1, 2) or (rem == Fr(1, 2) and n % 2):
        n += 1
    val = Fr(n) * Fr(2) ** qexp
    r = F32(np.inf) if val >= Fr(2) ** 128 else F32(float(val))
    return F32(-r) if neg else r


def _fr(x) -> Fr:
    return Fr(float(F32(x)))


def fadd(a, b):
    return rn32(_fr(a) + _fr(b))


def fsub(a, b):
    return rn32(_fr(a) - _fr(b))


def fmul(a, b):
    return rn32(_fr(a) * _fr(b))


def ffma(a, b, c):
    return rn32(_fr(a) * _fr(b) + _fr(c))


def fdiv(a, b):
    return rn32(_fr(a) / _fr(b))


def fexp(x):
    from oracle import oracle as orc

    return F32(orc.expf(F32(x)))


def flog(x):
    from oracle import oracle as orc

    return F32(orc.logf(F32(x)))


def to_bf16(x):
    u = np.asarray([x], F32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16).view(F32)[0]


def ulp(x):
    x = abs(float(x))
    return 2.0 ** (math.frexp(x)[1] - 24)


def sigma(D: int):
    s = {64: F32(0.125), 128: F32(F32(np.sqrt(np.float64(2.0))) / F32(16.0))}[D]
    assert D != 128 or int(np.asarray([s], F32).view(np.uint32)[0]) == 0x3DB504F3  # RN(1/sqrt(128))
    return s


def score(dot, D):
    return fmul(dot, sigma(D))


def _bf16_exact(x) -> bool:
    u = np.asarray(x, F32).reshape(-1).view(np.uint32)
    return bool(np.all((u & 0xFFFF) == 0))


def split3(t):
    """bf16 (x, y, z) whose serial fma dot with (1, 1, 1) is exactly t."""
    t = F32(t)

    def trunc(a):
        return (np.asarray([a], F32).view(np.uint32) & np.uint32(0xFFFF0000)).view(F32)[0]

    x = trunc(t)
    r = F32(t - x)
    y = trunc(r)
    z = F32(r - y)
    assert _bf16_exact([x, y, z]) and fadd(fadd(x, y), z) == t, t
    return x, y, z


# ---------------------------------------------------------------- inputs
def build(D, S, row, dots, vals, window=0):
    """One head; query ``row`` = e_0 + e_1 + e_2, every other query 0.  ``dots``
    maps key -> the dot wanted with that row (keys up to ``row`` not listed
    get NEG_DOT); ``vals`` maps key -> {column: value}."""
    p = {n: np.zeros((1, 1, S, D), F32) for n in ("q", "k", "v", "do")}
    p["q"][0, 0, row, :3] = 1.0
    for j in range(row + 1):
        p["k"][0, 0, j, :3] = split3(dots.get(j, NEG_DOT))
    for j, cols in vals.items():
        for c, x in cols.items():
            p["v"][0, 0, j, c] = x
    for n in ("q", "k", "v"):
        assert _bf16_exact(p[n]), n
    p["_row"], p["_window"] = row, window
    return p


def arrays(p):
    return {n: p[n] for n in ("q", "k", "v", "do")}


# ---------------------------------------------------------------- l fold
def _l_fold_forms(l0, alpha, pt, n=31):
    x = fmul(l0, alpha)
    want = x
    for _ in range(n):
        want = fadd(want, pt)
    want = fadd(want, F32(1.0))
    rs = F32(0.0)
    for _ in range(n):
        rs = fadd(rs, pt)
    rs = fadd(rs, F32(1.0))
    rev = fadd(x, F32(1.0))
    for _ in range(n):
        rev = fadd(rev, pt)
    return want, {"rowsum": fadd(x, rs), "fma": ffma(l0, alpha, rs), "reverse": rev}


@functools.lru_cache(maxsize=None)
def l_fold_case(D):
    sg = float(sigma(D))
    for ka in range(1, 60):
        dot_a = F32(-0.0625 * ka / sg)         # block 0 maximum a in (-0.6, 0): alpha = exp(a)
        a = score(dot_a, D)
        for ku in range(1, 40):
            dot_u = F32((float(a) - 0.37 - 0.11 * ku) / sg)
            u = score(dot_u, D)
            pu = fexp(fsub(u, a))
            l0 = fadd(F32(1.0), pu)
            alpha = fexp(a)
            x = fmul(l0, alpha)
            if not (0.5 <= x < 1.0 - 40 * 2.0**-24):
                continue
            for kt in range(0, 24):
                dot_t = F32((-16.7 - 0.03 * kt) / sg)
                t = score(dot_t, D)
                pt = fexp(t)
                if not (0.5 * ulp(x) < pt < ulp(x)):
                    continue
                want, devs = _l_fold_forms(l0, alpha, pt)
                lse, o0 = flog(want), fdiv(alpha, want)
                if all(flog(d) != lse and fdiv(alpha, d) != o0 for d in devs.values()):
                    return dict(dot_a=dot_a, dot_u=dot_u, dot_t=dot_t, alpha=alpha, want_l=want, lse=lse, o0=o0,
                                dev_l=devs)
    raise AssertionError(f"no l_fold case at D={D}")


def l_fold(D):
    c = l_fold_case(D)
    dots = {0: c["dot_a"], 1: c["dot_u"], 63: F32(0.0)}
    dots.update({j: c["dot_t"] for j in range(32, 63)})
    p = build(D, 64, 63, dots, {0: {0: 1.0}})
    p["_want"] = {"lse": c["lse"], "o": {0: c["o0"]}}
    p["_dev"] = {k: {"lse": flog(l), "o": {0: fdiv(c["alpha"], l)}} for k, l in c["dev_l"].items()}
    return p


# ---------------------------------------------------------------- acc rescale
def _acc_forms(acc0, alpha, col):
    """contract and deviations for one column; ``col`` = the block-1 values
    (all with p = 1), in key order."""
    want = fmul(acc0, alpha)
    for x in col:
        want = ffma(F32(1.0), x, want)
    part = F32(0.0)
    for x in col:
        part = ffma(F32(1.0), x, part)
    fused = ffma(acc0, alpha, fmul(F32(1.0), col[0]))
    for x in col[1:]:
        fused = ffma(F32(1.0), x, fused)
    return want, {"fused": fused, "partial": fadd(fmul(acc0, alpha), part), "partial_fma": ffma(acc0, alpha, part)}


@functools.lru_cache(maxsize=None)
def acc_rescale_case(D):
    sg = float(sigma(D))
    rng = np.random.default_rng(11)
    for _ in range(400):
        A = to_bf16(F32(rng.uniform(1.0, 2.0)))
        B = to_bf16(F32(rng.uniform(1.0, 2.0)))
        dot_a = F32(-rng.uniform(0.05, 0.6) / sg)
        a = score(dot_a, D)
        alpha = fexp(a)
        x0, x1 = fmul(A, alpha), fmul(B, alpha)
        r0 = F32(3 * ulp(x0))
        w = fsub(x0, r0)
        hi, mid, lo = split3(w)
        T = F32(2.0 ** (math.frexp(float(x1))[1] - 1 + 21))
        col0 = [F32(-hi), F32(-mid), F32(-lo), F32(0.0), F32(0.0)]
        col1 = [F32(0.0), F32(0.0), F32(0.0), T, F32(-T)]
        w0, d0 = _acc_forms(A, alpha, col0)
        w1, d1 = _acc_forms(B, alpha, col1)
        if w0 != r0:
            continue
        l = fmul(F32(1.0), alpha)
        for _ in range(5):
            l = fadd(l, F32(1.0))
        o = (fdiv(w0, l), fdiv(w1, l))
        devs = {k: (fdiv(d0[k], l), fdiv(d1[k], l)) for k in d0}
        if all(to_bf16(dv[0]) != to_bf16(o[0]) or to_bf16(dv[1]) != to_bf16(o[1]) for dv in devs.values()):
            return dict(A=A, B=B, dot_a=dot_a, hi=hi, mid=mid, lo=lo, T=T, o=o, dev=devs, l=l)
    raise AssertionError(f"no acc_rescale case at D={D}")


def acc_rescale(D):
    c = acc_rescale_case(D)
    dots = {0: c["dot_a"]}
    dots.update({j: F32(0.0) for j in range(32, 37)})
    vals = {0: {0: c["A"], 1: c["B"]}, 32: {0: -c["hi"]}, 33: {0: -c["mid"]}, 34: {0: -c["lo"]}, 35: {1: c["T"]},
            36: {1: -c["T"]}}
    p = build(D, 64, 63, dots, vals)
    p["_want"] = {"lse": flog(c["l"]), "o": {0: c["o"][0], 1: c["o"][1]}}
    p["_dev"] = {k: {"o": {0: o[0], 1: o[1]}} for k, o in c["dev"].items()}
    return p


# ---------------------------------------------------------------- LSE composition
@functools.lru_cache(maxsize=None)
def lse_case(D):
    sg = float(sigma(D))
    for km in range(1, 400):
        dot_m = F32((1.0 + 0.0173 * km) / sg)
        m = score(dot_m, D)
        for kb in range(1, 30):
            dot_b = F32((float(m) - 0.05 * kb) / sg)
            b = score(dot_b, D)
            l = fadd(F32(1.0), fexp(fsub(b, m)))
            want = fadd(m, flog(l))
            dev = F32(float(m) + math.log(float(l)))
            if m != 0 and l != 1 and dev != want:
                return dict(dot_m=dot_m, dot_b=dot_b, m=m, l=l, lse=want, dev=dev)
    raise AssertionError(f"no lse case at D={D}")


def lse(D):
    c = lse_case(D)
    p = build(D, 32, 1, {0: c["dot_m"], 1: c["dot_b"]}, {})
    p["_want"] = {"lse": c["lse"], "o": {0: F32(0.0)}}
    p["_dev"] = {"binary64": {"lse": c["dev"]}}
    return p


# ---------------------------------------------------------------- exp argument
@functools.lru_cache(maxsize=None)
def exp_argument_case(D):
    sg = float(sigma(D))
    for km in range(1, 200):
        dot_m = F32((5.0 + 0.0371 * km) / sg)
        m = score(dot_m, D)
        for kb in range(1, 60):
            dot_b = F32((-0.001 - 0.000731 * kb * km) / sg)
            b = score(dot_b, D)
            d = fsub(b, m)
            if _fr(b) - _fr(m) == _fr(d):
                continue  # exact difference: nothing to see
            exact = float(b) - float(m)  # exact in binary64
            lo, hi = F32(math.exp(exact) * (1 - 2.0**-50)), F32(math.exp(exact) * (1 + 2.0**-50))
            if lo != hi:
                continue
            p, pdev = fexp(d), lo
            l, ldev = fadd(F32(1.0), p), fadd(F32(1.0), pdev)
            o, odev = fdiv(p, l), fdiv(pdev, ldev)
            if o != odev:
                return dict(dot_m=dot_m, dot_b=dot_b, o=o, odev=odev, lse=fadd(m, flog(l)))
    raise AssertionError(f"no exp_argument case at D={D}")


def exp_argument(D):
    c = exp_argument_case(D)
    p = build(D, 32, 1, {0: c["dot_m"], 1: c["dot_b"]}, {1: {0: 1.0}})
    p["_want"] = {"lse": c["lse"], "o": {0: c["o"]}}
    p["_dev"] = {"unrounded": {"o": {0: c["odev"]}}}
    return p


# ---------------------------------------------------------------- uniform and window edge (q = 0)
def _bf16_values(shape, seed):
    x = np.random.default_rng(seed).standard_normal(shape).astype(F32)
    return (x.view(np.uint32) & np.uint32(0xFFFF0000)).view(F32)


def uniform(D):
    S = 96
    p = {n: np.zeros((1, 1, S, D), F32) for n in ("q", "k", "do")}
    p["k"][...] = _bf16_values((1, 1, S, D), 5)
    p["v"] = _bf16_values((1, 1, S, D), 6)
    run = np.add.accumulate(p["v"][0, 0], axis=0, dtype=F32)  # serial binary32 sums, keys ascending
    cnt = np.arange(1, S + 1, dtype=np.float64)[:, None]
    want = (run.astype(np.float64) / cnt).astype(F32)  # a binary64 quotient of binary32 operands rounds once
    recip = (run * (1.0 / cnt).astype(F32)).astype(F32)
    p["_rows"] = {"o": want, "lse": np.array([flog(F32(n)) for n in range(1, S + 1)], F32)}
    p["_rows_dev"] = {"reciprocal": recip}
    p["_window"] = 0
    return p


def window_edge(D):
    S, w = 64, 32
    p = {n: np.zeros((1, 1, S, D), F32) for n in ("q", "k", "do")}
    p["k"][...] = _bf16_values((1, 1, S, D), 7)
    p["v"] = _bf16_values((1, 1, S, D), 8)
    want = np.zeros((S, D), F32)
    for i in range(S):
        run = np.zeros(D, F32)
        for j in range(max(0, i - w + 1), i + 1):
            run = (run + p["v"][0, 0, j]).astype(F32)
        want[i] = (run.astype(np.float64) / min(i + 1, w)).astype(F32)
    p["_rows"] = {"o": want, "lse": np.array([flog(F32(min(i + 1, w))) for i in range(S)], F32)}
    p["_window"] = w
    return p


# ---------------------------------------------------------------- checks
def check_row(out, p, bf16: bool, name: str):
    """The probed row's LSE and listed O columns equal the contract's bits; the
    deviations' bits are asserted to differ (where the output dtype shows them)."""
    row = p["_row"]
    w = p["_want"]
    got_lse = out["lse"][0, 0, row]
    assert got_lse == w["lse"], f"{name}: LSE_{row} = {got_lse!r}, want {w['lse']!r}"
    for c, x in w["o"].items():
        want = to_bf16(x) if bf16 else x
        got = out["o"][0, 0, row, c]
        assert np.asarray([got], F32).view(np.uint32)[0] == np.asarray([want], F32).view(np.uint32)[0], (
            f"{name}: O_{row}[{c}] = {got!r}, want {want!r}")
    for dn, dv in p["_dev"].items():
        seen = False
        if "lse" in dv and dv["lse"] != w["lse"]:
            seen = True
        for c, x in dv.get("o", {}).items():
            a, b = (to_bf16(x), to_bf16(w["o"][c])) if bf16 else (x, w["o"][c])
            seen = seen or a != b
        if not bf16:
            assert seen, f"{name}: deviation {dn} gives the contract's bits"


def check_rows(out, p, bf16: bool, name: str):
    want_o = p["_rows"]["o"]
    if bf16:
        want_o = np.vectorize(to_bf16, otypes=[F32])(want_o)
    got = np.ascontiguousarray(out["o"][0, 0], F32)
    bad = np.flatnonzero(got.view(np.uint32).ravel() != np.ascontiguousarray(want_o).view(np.uint32).ravel())
    assert bad.size == 0, f"{name}: {bad.size} O elements differ from the closed form, first {np.unravel_index(bad[0], got.shape)}"
    lse = np.ascontiguousarray(out["lse"][0, 0], F32)
    assert np.array_equal(lse.view(np.uint32), p["_rows"]["lse"].view(np.uint32)), f"{name}: LSE differs"
    for dn, dev in p.get("_rows_dev", {}).items():
        assert not np.array_equal(dev.view(np.uint32), p["_rows"]["o"].view(np.uint32)), dn


ROW_PROBES = ("l_fold", "acc_rescale", "lse", "exp_argument")
CLOSED_PROBES = ("uniform", "window_edge")


def all_probes(D: int):
    """[(name, inputs, window)] for one head dimension."""
    out = [(n, globals()[n](D)) for n in ROW_PROBES + CLOSED_PROBES]
    return [(n, p, p["_window"]) for n, p in out]


def check(name, out, p, bf16: bool):
    if name in ROW_PROBES:
        check_row(out, p, bf16, name)
    else:
        check_rows(out, p, bf16, name)
