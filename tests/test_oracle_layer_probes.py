"""CPU pins of the decoder-layer and int8-PV oracles' bit rules
(tests/layer_probes.py).

Every probe runs on the oracle with binary32 and bf16 outputs.  Then each
probe runs against copies of oracle/layer_oracle.c or oracle/int8pv_oracle.c
with one planted deviation from the contract (compiled here with
oracle/attn_oracle.c, in a temporary directory, never shipped), to show that
the probe catches it:

  RMSNorm  ss_serial         fold32 as one serial fold (forward ss and backward c)
           fold_reversed     fold32's chunk partials added in descending order
           mean_reciprocal   mean = RN(ss RN(1/D))
           y_rstd_w          y = RN(x RN(rstd w))
           c_reciprocal      c = RN(fold RN(1/D))
           dx_fma            dx = RN(rstd fma(-xh, c, g))
           dx_distributed    dx = RN(RN(rstd g) - RN(rstd RN(xh c)))
           dw_serial         dw folded over all rows serially
           dw_reversed       dw's row-chunk partials added in descending order
  SiLU     silu_reciprocal   y = RN(x RN(1/d))
           silu_dy_first     dx = RN(RN(dy s) RN(1 + x (1 - s)))
           silu_distributed  g = s + x s (1 - s)
           silu_expanded     g = s ((1 + x) - x s)
  int8-PV  i8_step_product   acc = RN(a RN(sv sp)) + RN(acc alpha)
           i8_rescale_unrounded acc = fma(acc, alpha, RN(RN(a sv) sp))
           i8_dequant_order  acc = fma(RN(a sp), sv, RN(acc alpha))
           i8_qv_by_step     qv = rint(RN(v / sv))
           i8_qp_by_step     qp = rint(RN(p / sp))
"""

from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np
import pytest

import fwd_probes as fp
import layer_probes as lp
from oracle import oracle as orc

ORACLE = pathlib.Path(__file__).resolve().parents[1] / "oracle"
_fp = ctypes.POINTER(ctypes.c_float)
_i, _l = ctypes.c_int, ctypes.c_long


class _Lib:
    """The oracle entry points these probes call, on liborc or on a mutant build."""

    def __init__(self, lib):
        self.lib = lib
        lib.orc_rmsnorm_fwd.argtypes = [_fp, _fp, _fp, _fp, _l, _i, ctypes.c_float, _i, _i]
        lib.orc_rmsnorm_bwd.argtypes = [_fp, _fp, _fp, _fp, _fp, _fp, _l, _i, _i, _i]
        lib.orc_silu_fwd.argtypes = [_fp, _fp, _l, _i]
        lib.orc_silu_bwd.argtypes = [_fp, _fp, _fp, _l, _i]
        lib.orc_quantize_v.argtypes = [_fp, ctypes.c_void_p, _fp, _i, _i, _i, _i]
        lib.orc_attn_fwd_int8pv.argtypes = [_fp] * 5 + [_i] * 8
        for f in ("orc_rmsnorm_fwd", "orc_rmsnorm_bwd", "orc_silu_fwd", "orc_silu_bwd", "orc_quantize_v",
                  "orc_attn_fwd_int8pv"):
            getattr(lib, f).restype = _i

    @staticmethod
    def _p(a):
        return a.ctypes.data_as(_fp)

    def rms_fwd(self, x, w, bf16):
        x, w = np.ascontiguousarray(x, np.float32), np.ascontiguousarray(w, np.float32)
        rows, D = x.shape
        y, rstd = np.empty_like(x), np.empty(rows, np.float32)
        assert self.lib.orc_rmsnorm_fwd(self._p(x), self._p(w), self._p(y), self._p(rstd), rows, D, lp.EPS,
                                        int(bf16), 1) == 0
        return y, rstd

    def rms_bwd(self, x, w, rstd, dy, bf16):
        x, w, rstd, dy = (np.ascontiguousarray(a, np.float32) for a in (x, w, rstd, dy))
        rows, D = x.shape
        dx, dw = np.empty_like(x), np.empty(D, np.float32)
        assert self.lib.orc_rmsnorm_bwd(self._p(x), self._p(w), self._p(rstd), self._p(dy), self._p(dx),
                                        self._p(dw), rows, D, int(bf16), 1) == 0
        return dx, dw

    def silu_fwd(self, x, bf16):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        self.lib.orc_silu_fwd(self._p(x), self._p(y), x.size, int(bf16))
        return y

    def silu_bwd(self, x, dy, bf16):
        x, dy = np.ascontiguousarray(x, np.float32), np.ascontiguousarray(dy, np.float32)
        dx = np.empty_like(x)
        self.lib.orc_silu_bwd(self._p(x), self._p(dy), self._p(dx), x.size, int(bf16))
        return dx

    def quantize_v(self, v):
        v = np.ascontiguousarray(v, np.float32)
        B, Hkv, S, D = v.shape
        qv, sv = np.empty(v.shape, np.int8), np.empty((B, Hkv, S // 32, D), np.float32)
        assert self.lib.orc_quantize_v(self._p(v), qv.ctypes.data, self._p(sv), B, Hkv, S, D) == 0
        return qv, sv

    def int8pv_fwd(self, p, bf16):
        q, k, v = (np.ascontiguousarray(p[n], np.float32) for n in ("q", "k", "v"))
        B, H, S, D = q.shape
        o, lse = np.empty_like(q), np.empty((B, H, S), np.float32)
        assert self.lib.orc_attn_fwd_int8pv(self._p(q), self._p(k), self._p(v), self._p(o), self._p(lse), B, H,
                                            k.shape[1], S, D, p["_window"], int(bf16), 1) == 0
        return {"o": o, "lse": lse}


def run_probe(lib: _Lib, name: str, bf16: bool):
    """Run the named probe (every D for the int8-PV ones) and check it."""
    if name.startswith("rms_bwd"):
        p = dict(lp.rms_bwd_probes())[name]
        dx, dw = lib.rms_bwd(p["x"], p["w"], p["rstd"], p["dy"], bf16)
        lp.check_rms_bwd(name, p, dx, dw, bf16)
    elif name.startswith("rms"):
        p = dict(lp.rms_fwd_probes())[name]
        y, rstd = lib.rms_fwd(p["x"], p["w"], bf16)
        lp.check_rms_fwd(name, p, y, rstd, bf16)
    elif name == "silu_fwd":
        p = lp.silu_fwd()
        lp.check_silu(name, p, lib.silu_fwd(p["x"], bf16), bf16, "y")
    elif name == "silu_bwd":
        p = lp.silu_bwd()
        lp.check_silu(name, p, lib.silu_bwd(p["x"], p["dy"], bf16), bf16, "dx")
    else:
        for D in (64, 128):
            p = dict(lp.int8pv_probes(D))[name]
            fp.check_row(lib.int8pv_fwd(p, bf16), p, bf16, name)
            if name == "i8_qv":
                qv, _ = lib.quantize_v(p["v"])
                assert int(qv[0, 0, 1, 0]) == p["_qv"][0], f"i8_qv: qv = {qv[0, 0, 1, 0]}, want {p['_qv'][0]}"


ALL = ["rms_fold", "rms_mean", "rms_y", "rms_bwd_fold", "rms_bwd_c", "rms_bwd_dx", "rms_bwd_dw", "silu_fwd",
       "silu_bwd", "i8_acc", "i8_qv", "i8_qp"]


@pytest.mark.parametrize("bf16", [False, True], ids=["binary32", "bf16"])
@pytest.mark.parametrize("name", ALL)
def test_probe_on_oracle(name, bf16):
    run_probe(_Lib(orc.load()), name, bf16)


def test_probe_inputs_are_bf16_values():
    """The GPU runs the same probes with bf16 inputs, so every input value must
    be a bf16 value."""
    for _, p in lp.rms_fwd_probes() + lp.rms_bwd_probes():
        for n in ("x", "w", "dy"):
            if n in p:
                assert np.array_equal(p[n], lp.fp_bf16(p[n])), n
    assert lp.silu_inputs_bf16_exact(lp.silu_fwd()) and lp.silu_inputs_bf16_exact(lp.silu_bwd())
    for D in (64, 128):
        for _, p in lp.int8pv_probes(D):
            for n in ("q", "k", "v"):
                assert np.array_equal(p[n], lp.fp_bf16(p[n])), n


_FOLD = """  for (int c = 0; c < n / 32; c++) {
    float p = 0.0f;
    for (int i = 32 * c; i < 32 * c + 32; i++) p = fmaf(a[i], b[i], p);
    acc = acc + p;
  }"""
_DW = """    for (long c = 0; c < rows / 32; c++) {
      float p = 0.0f;
      for (long r = 32 * c; r < 32 * c + 32; r++) p = fmaf(dy[r * D + d], xh[r * D + d], p);
      acc = acc + p;
    }"""
_SILU_G = "    const float g = s * (1.0f + x[i] * (1.0f - s));\n    dx[i] = out_round(dy[i] * g, out_bf16);"
_I8_ACC = "          acc[d] = fmaf((float)a * svb[d], sp, acc[d] * alpha);"

LAYER_MUTANTS = {
    "ss_serial": [(_FOLD, "  for (int i = 0; i < n; i++) acc = fmaf(a[i], b[i], acc);")],
    "fold_reversed": [(_FOLD, _FOLD.replace("for (int c = 0; c < n / 32; c++)", "for (int c = n / 32 - 1; c >= 0; c--)"))],
    "mean_reciprocal": [("    const float mean = (float)((double)ss / (double)D);",
                         "    const float mean = ss * (1.0f / (float)D);")],
    "y_rstd_w": [("      y[r * D + d] = out_round(xh * w[d], out_bf16);",
                  "      y[r * D + d] = out_round(xr[d] * (rs * w[d]), out_bf16);\n      (void)xh;")],
    "c_reciprocal": [("      const float cc = (float)((double)dot / (double)D);",
                      "      const float cc = dot * (1.0f / (float)D);")],
    "dx_fma": [("dx[r * D + d] = out_round(rs * (g[d] - xh[r * D + d] * cc), out_bf16);",
                "dx[r * D + d] = out_round(rs * fmaf(-xh[r * D + d], cc, g[d]), out_bf16);")],
    "dx_distributed": [("dx[r * D + d] = out_round(rs * (g[d] - xh[r * D + d] * cc), out_bf16);",
                        "dx[r * D + d] = out_round(rs * g[d] - rs * (xh[r * D + d] * cc), out_bf16);")],
    "dw_serial": [(_DW, "    for (long r = 0; r < rows; r++) acc = fmaf(dy[r * D + d], xh[r * D + d], acc);")],
    "dw_reversed": [(_DW, _DW.replace("for (long c = 0; c < rows / 32; c++)", "for (long c = rows / 32 - 1; c >= 0; c--)"))],
    "silu_reciprocal": [("    y[i] = out_round((float)((double)x[i] / (double)d), out_bf16);",
                         "    y[i] = out_round(x[i] * (1.0f / d), out_bf16);")],
    "silu_dy_first": [(_SILU_G, "    dx[i] = out_round((dy[i] * s) * (1.0f + x[i] * (1.0f - s)), out_bf16);")],
    "silu_distributed": [(_SILU_G, "    const float g = s + (x[i] * s) * (1.0f - s);\n    dx[i] = out_round(dy[i] * g, out_bf16);")],
    "silu_expanded": [(_SILU_G, "    const float g = s * ((1.0f + x[i]) - x[i] * s);\n    dx[i] = out_round(dy[i] * g, out_bf16);")],
}
INT8_MUTANTS = {
    "i8_step_product": [(_I8_ACC, "          acc[d] = (float)a * (svb[d] * sp) + acc[d] * alpha;")],
    "i8_rescale_unrounded": [(_I8_ACC, "          acc[d] = fmaf(acc[d], alpha, ((float)a * svb[d]) * sp);")],
    "i8_dequant_order": [(_I8_ACC, "          acc[d] = fmaf((float)a * sp, svb[d], acc[d] * alpha);")],
    "i8_qv_by_step": [("      for (int j = 0; j < 32; j++) qb[(long)j * D + d] = inv == 0.0f ? 0 : quant(vb[(long)j * D + d], inv);",
                       "      for (int j = 0; j < 32; j++) qb[(long)j * D + d] = inv == 0.0f ? 0 : quant(vb[(long)j * D + d] / s, 1.0f);")],
    "i8_qp_by_step": [("        for (int jj = 0; jj < 32; jj++) qp[jj] = inv == 0.0f ? 0 : quant(p[jj], inv);",
                       "        for (int jj = 0; jj < 32; jj++) qp[jj] = inv == 0.0f ? 0 : quant(p[jj] / sp, 1.0f);")],
}
CAUGHT_BY = {"ss_serial": "rms_fold", "fold_reversed": "rms_fold", "mean_reciprocal": "rms_mean", "y_rstd_w": "rms_y",
             "c_reciprocal": "rms_bwd_c", "dx_fma": "rms_bwd_dx", "dx_distributed": "rms_bwd_dx",
             "dw_serial": "rms_bwd_dw", "dw_reversed": "rms_bwd_dw", "silu_reciprocal": "silu_fwd",
             "silu_dy_first": "silu_bwd", "silu_distributed": "silu_bwd", "silu_expanded": "silu_bwd",
             "i8_step_product": "i8_acc", "i8_rescale_unrounded": "i8_acc", "i8_dequant_order": "i8_acc",
             "i8_qv_by_step": "i8_qv", "i8_qp_by_step": "i8_qp"}
# deviations that only a binary32 output shows: results one binary32 unit apart
# round to the same bf16 value unless one of them is exactly a bf16 midpoint
BINARY32_ONLY = {"y_rstd_w", "silu_reciprocal", "c_reciprocal", "dx_fma", "dx_distributed", "silu_dy_first", "silu_distributed",
                 "silu_expanded"}


def _build(srcs: dict, tmp: pathlib.Path) -> _Lib:
    paths = []
    for name, text in srcs.items():
        f = tmp / name
        f.write_text(text)
        paths.append(str(f))
    so = tmp / "mutant.so"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-fopenmp", "-shared", *paths, "-o",
                    str(so), "-lquadmath", "-lm"], check=True, capture_output=True)
    return _Lib(ctypes.CDLL(str(so)))


def _mutant(name: str, tmp: pathlib.Path) -> _Lib:
    srcs = {f: (ORACLE / f).read_text() for f in ("attn_oracle.c", "layer_oracle.c", "int8pv_oracle.c")}
    target, edits = ("layer_oracle.c", LAYER_MUTANTS[name]) if name in LAYER_MUTANTS else \
        ("int8pv_oracle.c", INT8_MUTANTS[name])
    for old, new in edits:
        assert srcs[target].count(old) == 1, (name, old)
        srcs[target] = srcs[target].replace(old, new)
    return _build(srcs, tmp)


def test_unmutated_copy_passes_every_probe(tmp_path):
    srcs = {f: (ORACLE / f).read_text() for f in ("attn_oracle.c", "layer_oracle.c", "int8pv_oracle.c")}
    lib = _build(srcs, tmp_path)
    for name in ALL:
        for bf16 in (False, True):
            run_probe(lib, name, bf16)


@pytest.mark.parametrize("mutant", sorted(CAUGHT_BY))
def test_each_probe_catches_its_planted_deviation(mutant, tmp_path):
    lib = _mutant(mutant, tmp_path)
    for bf16 in (False, True):
        if bf16 and mutant in BINARY32_ONLY:
            continue
        with pytest.raises(AssertionError):
            run_probe(lib, CAUGHT_BY[mutant], bf16)
