"""CPU pins of the forward's online-softmax bookkeeping (tests/fwd_probes.py).

Each closed-form probe runs on the oracle at D 64 and 128, with binary32 and
bf16 outputs.  Then each probe runs against copies of oracle/attn_oracle.c
with one planted deviation from the contract (compiled here, in a temporary
directory, never shipped), to show that the probe catches it:

  l_rowsum        l = RN(l alpha) + RN(sum of the block's p) (SURVEY's C5 form)
  l_fma           l = fma(l, alpha, sum of the block's p)
  l_reversed      the block's p added to l in descending key order
  acc_fused       acc = fma(acc, alpha, RN(p_0 v_0)), then the chain from key 1
  acc_partial     acc = RN(RN(acc alpha) + block chain from +0)
  acc_partial_fma acc = fma(acc, alpha, block chain from +0)
  lse_binary64    LSE = one rounding of the binary64 m + log(l)
  exp_unrounded   p = exp of the exact s - m' instead of exp(RN(s - m'))
  o_reciprocal    O = RN(acc RN(1 / l)) instead of RN(acc / l)
  alpha_always    alpha = exp(m - m') even when m' == m (NaN for -inf)
  masked_exp      masked keys given exp(s - m') instead of +0
"""

from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np
import pytest

import fwd_probes as fp
from oracle import oracle as orc

ORACLE_C = pathlib.Path(__file__).resolve().parents[1] / "oracle" / "attn_oracle.c"


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("bf16", [False, True], ids=["binary32", "bf16"])
def test_forward_probes_on_oracle(D, bf16):
    for name, p, window in fp.all_probes(D):
        o, lse = orc.attn_fwd(p["q"], p["k"], p["v"], window=window, out_bf16=bf16)
        fp.check(name, {"o": o, "lse": lse}, p, bf16)


def test_int8pv_lse_equals_binary32_lse_on_probes():
    """The int8-PV forward sums the unquantized p into l, so its LSE is the
    binary32 forward's on every probe (the O differs by quantization)."""
    for name, p, window in fp.all_probes(128):
        _, lse = orc.attn_fwd(p["q"], p["k"], p["v"], window=window, out_bf16=True)
        _, lse8 = orc.attn_fwd_int8pv(p["q"], p["k"], p["v"], window=window, out_bf16=True)
        assert np.array_equal(np.asarray(lse, np.float32).view(np.uint32),
                              np.asarray(lse8, np.float32).view(np.uint32)), name


_L_BLOCK = """        l = l * alpha;
        for (int jj = 0; jj < 32; jj++) {
          p[jj] = masked(i, 32 * J + jj, window) ? 0.0f : orc_expf(s[jj] - mn);
          l = l + p[jj];
        }
"""
_ACC_BLOCK = """          float a = acc[d] * alpha;
          for (int jj = 0; jj < 32; jj++) a = fmaf(p[jj], vb[(long)(32 * J + jj) * D + d], a);
          acc[d] = a;
"""
_P_LINE = "          p[jj] = masked(i, 32 * J + jj, window) ? 0.0f : orc_expf(s[jj] - mn);\n"


def _l_sum(combine):
    return (_L_BLOCK, "        float rs = 0.0f;\n        for (int jj = 0; jj < 32; jj++) {\n" + _P_LINE +
            "          rs = rs + p[jj];\n        }\n        " + combine + "\n")


def _acc_partial(combine):
    return (_ACC_BLOCK, "          float part = 0.0f;\n"
            "          for (int jj = 0; jj < 32; jj++) part = fmaf(p[jj], vb[(long)(32 * J + jj) * D + d], part);\n"
            "          acc[d] = " + combine + ";\n")


MUTANTS = {
    "l_rowsum": [_l_sum("l = l * alpha;\n        l = l + rs;")],
    "l_fma": [_l_sum("l = fmaf(l, alpha, rs);")],
    "l_reversed": [(_L_BLOCK, "        l = l * alpha;\n        for (int jj = 0; jj < 32; jj++)\n  " + _P_LINE +
                    "        for (int jj = 31; jj >= 0; jj--) l = l + p[jj];\n")],
    "acc_fused": [(_ACC_BLOCK, "          float a = fmaf(acc[d], alpha, p[0] * vb[(long)(32 * J) * D + d]);\n"
                   "          for (int jj = 1; jj < 32; jj++) a = fmaf(p[jj], vb[(long)(32 * J + jj) * D + d], a);\n"
                   "          acc[d] = a;\n")],
    "acc_partial": [_acc_partial("acc[d] * alpha + part")],
    "acc_partial_fma": [_acc_partial("fmaf(acc[d], alpha, part)")],
    "lse_binary64": [("      lse[row] = m + orc_logf(l);", "      lse[row] = (float)((double)m + log((double)l));")],
    "exp_unrounded": [(_P_LINE, "          p[jj] = masked(i, 32 * J + jj, window) ? 0.0f : "
                       "(float)expq((__float128)s[jj] - (__float128)mn);\n")],
    "o_reciprocal": [("        float x = (float)((double)acc[d] / (double)l);",
                      "        float x = acc[d] * (1.0f / l);")],
    "alpha_always": [("        const float alpha = (mn == m) ? 1.0f : orc_expf(m - mn);",
                      "        const float alpha = orc_expf(m - mn);")],
    "masked_exp": [(_P_LINE, "          p[jj] = orc_expf(s[jj] - mn);\n")],
}
# the probe each deviation must fail (the others may or may not notice)
CAUGHT_BY = {"l_rowsum": "l_fold", "l_fma": "l_fold", "l_reversed": "l_fold", "acc_fused": "acc_rescale",
             "acc_partial": "acc_rescale", "acc_partial_fma": "acc_rescale", "lse_binary64": "lse",
             "exp_unrounded": "exp_argument", "o_reciprocal": "uniform", "alpha_always": "window_edge",
             "masked_exp": "window_edge"}
# deviations whose only trace is below bf16 resolution in O and absent from LSE
BINARY32_ONLY = {"exp_unrounded", "o_reciprocal"}


def _build_mutant(name, tmp):
    src = ORACLE_C.read_text()
    for old, new in MUTANTS[name]:
        assert src.count(old) == 1, (name, old)
        src = src.replace(old, new)
    c = tmp / f"{name}.c"
    c.write_text(src)
    so = tmp / f"{name}.so"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-fopenmp", "-shared", str(c),
                    "-o", str(so), "-lquadmath", "-lm"], check=True, capture_output=True)
    lib = ctypes.CDLL(str(so))
    lib.orc_attn_fwd.restype = ctypes.c_int
    lib.orc_attn_fwd.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 8
    return lib


def _mutant_fwd(lib, p, window, bf16):
    f = {n: np.ascontiguousarray(p[n], dtype=np.float32) for n in ("q", "k", "v")}
    B, H, S, D = f["q"].shape
    Hkv = f["k"].shape[1]
    o, lse = np.empty_like(f["q"]), np.empty((B, H, S), np.float32)
    ptr = lambda a: a.ctypes.data  # noqa: E731
    assert lib.orc_attn_fwd(ptr(f["q"]), ptr(f["k"]), ptr(f["v"]), ptr(o), ptr(lse), B, H, Hkv, S, D, window,
                            int(bf16), 1) == 0
    return {"o": o, "lse": lse}


def test_mutant_sources_compile_unchanged(tmp_path):
    """The planting helper on an empty list reproduces the oracle's results
    (so a failure below is the deviation's, not the copy's)."""
    MUTANTS["_none"] = []
    try:
        lib = _build_mutant("_none", tmp_path)
    finally:
        del MUTANTS["_none"]
    for name, p, window in fp.all_probes(128):
        fp.check(name, _mutant_fwd(lib, p, window, False), p, False)


@pytest.mark.parametrize("mutant", sorted(MUTANTS))
def test_each_probe_catches_its_planted_deviation(mutant, tmp_path):
    lib = _build_mutant(mutant, tmp_path)
    for D in (64, 128):
        for bf16 in (False, True):
            if bf16 and mutant in BINARY32_ONLY:
                continue
            probes = {name: (p, w) for name, p, w in fp.all_probes(D)}
            p, window = probes[CAUGHT_BY[mutant]]
            with pytest.raises(AssertionError):
                fp.check(CAUGHT_BY[mutant], _mutant_fwd(lib, p, window, bf16), p, bf16)
