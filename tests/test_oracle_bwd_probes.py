"""CPU pins of the backward's bit-level rules (tests/bwd_probes.py).

Each closed-form probe is run on the oracle in binary32 and in bf16 output
mode.  Then every probe is run against copies of oracle/attn_oracle.c, each
with one planted deviation from the contract (compiled here, in a temporary
directory, never shipped), to show that the probe catches it:

  heads_reversed   the GQA head loop of the dK/dV fold runs backwards
  queries_reversed the query loop of the dK/dV fold runs backwards
  dsum_dropped     Dsum taken as 0 instead of the dot with the stored O
  sigma_per_term   sigma applied to dS inside the dK fold instead of once after it
  ds_fused         dS = fma(P, dP, -RN(P Dsum)) instead of RN(P RN(dP - Dsum))
  ds_unrounded     dS = RN(P (dP - Dsum)) with the difference kept in binary64
"""

from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np
import pytest

import bwd_probes as bp
from attn_util import bits
from oracle import oracle as orc

ORACLE_C = pathlib.Path(__file__).resolve().parents[1] / "oracle" / "attn_oracle.c"


@pytest.mark.parametrize("bf16", [False, True], ids=["binary32", "bf16"])
def test_backward_probes_on_oracle(bf16):
    for name, p, check in bp.all_probes(bf16):
        bp.assert_inputs_bf16_exact(p)
        dq, dk, dv = orc.attn_bwd(p["q"], p["k"], p["v"], p["o"], p["lse"], p["do"], window=0, out_bf16=bf16)
        check({"dq": dq, "dk": dk, "dv": dv})


def test_stored_bf16_o_changes_dq():
    """The operator's backward sees the O it returned (bf16 for bf16 inputs).
    For these inputs a backward fed the binary32 O instead gives different dQ
    bits, so the GPU parity tests (which feed the stored bf16 O to both sides)
    would see a kernel that used the binary32 O."""
    from attn_util import make

    inp = make(1, 2, 2, 64, 64, dtype="bf16", seed=12)
    o16, lse = orc.attn_fwd(inp["q"], inp["k"], inp["v"], out_bf16=True)
    o32, lse32 = orc.attn_fwd(inp["q"], inp["k"], inp["v"], out_bf16=False)
    assert np.array_equal(bits(lse), bits(lse32))
    assert not np.array_equal(bits(o16), bits(o32))
    dq16, _, _ = orc.attn_bwd(inp["q"], inp["k"], inp["v"], o16, lse, inp["do"])
    dq32, _, _ = orc.attn_bwd(inp["q"], inp["k"], inp["v"], o32, lse, inp["do"])
    assert not np.array_equal(bits(dq16), bits(dq32))


MUTANTS = {
    "heads_reversed": [("        for (int r = 0; r < G; r++) {\n          const int h = g * G + r;\n          const long base = ((long)b * H + h) * S;\n          const float* Pr",
                        "        for (int r = G - 1; r >= 0; r--) {\n          const int h = g * G + r;\n          const long base = ((long)b * H + h) * S;\n          const float* Pr")],
    "queries_reversed": [("          for (int i = 32 * J; i < ihi; i++) {", "          for (int i = ihi - 1; i >= 32 * J; i--) {")],
    "dsum_dropped": [("        const float Di = dotf(doi, o + (base + i) * D, D);", "        const float Di = 0.0f;")],
    "sigma_per_term": [("              acck[d] = fmaf(dsij, qi[d], acck[d]);", "              acck[d] = fmaf(dsij * sigma, qi[d], acck[d]);"),
                       ("          const float x = acck[d] * sigma;\n          dvj[d]", "          const float x = acck[d];\n          dvj[d]")],
    "ds_fused": [("          dSr[(size_t)i * S + j] = pij * (dp - Di);", "          dSr[(size_t)i * S + j] = fmaf(pij, dp, -(pij * Di));")],
    "ds_unrounded": [("          dSr[(size_t)i * S + j] = pij * (dp - Di);",
                      "          dSr[(size_t)i * S + j] = (float)((double)pij * ((double)dp - (double)Di));")],
}
# the probe each deviation must fail (every other probe may or may not notice)
CAUGHT_BY = {"heads_reversed": "gqa_order", "queries_reversed": "query_order", "dsum_dropped": "dsum_stored_o",
             "sigma_per_term": "sigma_once", "ds_fused": "ds_rounding", "ds_unrounded": "ds_rounding"}


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
    lib.orc_attn_bwd.restype = ctypes.c_int
    lib.orc_attn_bwd.argtypes = [ctypes.c_void_p] * 9 + [ctypes.c_int] * 8
    return lib


def _mutant_bwd(lib, p, bf16):
    f = {n: np.ascontiguousarray(p[n], dtype=np.float32) for n in ("q", "k", "v", "o", "lse", "do")}
    B, H, S, D = f["q"].shape
    Hkv = f["k"].shape[1]
    dq, dk, dv = np.empty_like(f["q"]), np.empty_like(f["k"]), np.empty_like(f["v"])
    ptr = lambda a: a.ctypes.data  # noqa: E731
    rc = lib.orc_attn_bwd(ptr(f["q"]), ptr(f["k"]), ptr(f["v"]), ptr(f["o"]), ptr(f["lse"]), ptr(f["do"]), ptr(dq),
                          ptr(dk), ptr(dv), B, H, Hkv, S, D, 0, int(bf16), 1)
    assert rc == 0
    return {"dq": dq, "dk": dk, "dv": dv}


@pytest.mark.parametrize("mutant", sorted(MUTANTS))
def test_each_probe_catches_its_planted_deviation(mutant, tmp_path):
    lib = _build_mutant(mutant, tmp_path)
    for bf16 in (False, True):
        probes = {name: (p, check) for name, p, check in bp.all_probes(bf16)}
        p, check = probes[CAUGHT_BY[mutant]]
        if mutant == "ds_unrounded" or mutant == "ds_fused":
            if bf16:
                continue  # dS is seen through binary32 dQ (the GPU test also reads the workspace's dS tile)
        with pytest.raises(AssertionError):
            check(_mutant_bwd(lib, p, bf16))
