"""CPU pins of the scalar pieces of the contract: exp, log, scale, bf16 rounding.

What fixes each value independently of the code under test:
  exp / log   correct rounding is a definition.  The oracle's fast path
              (binary64 libm + boundary test) and the kernels' own source
              (otx_math.h built for the host) are both compared with
              RN32(expq / logq) from libquadmath on dense ranges, on the
              special values, and on the exception-table inputs.
  scale       RN(1/sqrt(D)) is exact for D = 64 (0.125) and is compared with
              the binary64 value rounded once for D = 128.
  bf16        RNE rounding is compared with a tie/overflow/NaN table worked out
              by hand.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

from oracle import oracle as orc


def f2u(x: float) -> int:
    return int(np.array([x], dtype=np.float32).view(np.uint32)[0])


def u2f(u: int) -> float:
    return float(np.array([u], dtype=np.uint32).view(np.float32)[0])


def _host_math():
    from open_transformers_amd import build

    path = build.PKG_DIR / build.HOST_MATH_LIB
    if not path.exists():
        build.build_host_math()
    lib = ctypes.CDLL(str(path))
    for n in ("otx_host_expf", "otx_host_logf"):
        getattr(lib, n).restype = ctypes.c_float
        getattr(lib, n).argtypes = [ctypes.c_float]
    lib.otx_host_div_rn.restype = ctypes.c_float
    lib.otx_host_div_rn.argtypes = [ctypes.c_float, ctypes.c_float]
    lib.otx_host_f32_to_bf16.restype = ctypes.c_uint16
    lib.otx_host_f32_to_bf16.argtypes = [ctypes.c_float]
    return lib


# Ranges of binary32 bit patterns: softmax arguments (x <= 0, down through the
# subnormal results to the +0 threshold), tiny |x| (results next to 1), and
# LSE's log arguments l >= 1.
EXP_RANGES = [
    (0x80000000, 1 << 20),
    (f2u(-1e-3), 1 << 20),
    (f2u(-0.5), 1 << 20),
    (f2u(-10.0), 1 << 20),
    (f2u(-87.0), 1 << 20),
    (f2u(-103.5), 1 << 18),
    (f2u(0.25), 1 << 18),
]
LOG_RANGES = [(f2u(1.0), 1 << 21), (f2u(1000.0), 1 << 20), (f2u(0.3), 1 << 19)]


@pytest.mark.parametrize("lo,count", EXP_RANGES)
def test_oracle_exp_correctly_rounded(lo, count):
    lib = orc.load()
    assert lib.orc_verify_math(lo, lo + count, 0) == 0


@pytest.mark.parametrize("lo,count", LOG_RANGES)
def test_oracle_log_correctly_rounded(lo, count):
    lib = orc.load()
    assert lib.orc_verify_math(lo, lo + count, 1) == 0


def test_exp_log_special_values():
    assert orc.expf(0.0) == 1.0
    assert orc.expf(-0.0) == 1.0
    assert orc.expf(float("-inf")) == 0.0 and math.copysign(1.0, orc.expf(float("-inf"))) == 1.0
    assert orc.expf(-104.0) == 0.0
    assert orc.expf(-103.0) == u2f(1)  # exp(-103) ~ 1.4e-45: rounds to the smallest subnormal
    assert orc.expf(1.0) == u2f(0x402DF854)  # e to binary32
    assert orc.logf(1.0) == 0.0
    assert orc.logf(2.0) == u2f(0x3F317218)  # ln 2 to binary32
    assert orc.logf(0.0) == float("-inf")


def test_kernel_math_source_matches_oracle():
    """The device exp/log/division source, compiled for the host, equals the
    oracle on every input of the sampled ranges and on its exception tables."""
    host = _host_math()
    rng = np.random.default_rng(5)
    xs = np.concatenate([
        rng.uniform(-104.0, 0.0, 20000).astype(np.float32),
        -np.exp(rng.uniform(-40, 4, 20000)).astype(np.float32),
        np.array([0.0, -0.0, -103.97, -87.33655, -87.33654, -1e-30, 88.7], dtype=np.float32),
    ])
    for x in xs:
        assert f2u(host.otx_host_expf(float(x))) == f2u(orc.expf(float(x))), x
    ls = np.concatenate([np.exp(rng.uniform(0, 20, 20000)).astype(np.float32), np.float32([1.0, 2.0, 3.0])])
    for x in ls:
        assert f2u(host.otx_host_logf(float(x))) == f2u(orc.logf(float(x))), x


def test_exception_tables_are_correct():
    """Every exception-table entry is the libquadmath correctly rounded value."""
    import re

    from open_transformers_amd import build

    text = (build.CSRC / "otx_math_tables.h").read_text()
    for fn, name in ((orc.load().orc_expf_quad, "exp"), (orc.load().orc_logf_quad, "log")):
        keys = [int(x, 16) for x in re.findall(r"0x([0-9a-f]+)u", text.split(f"otx_{name}_exc_keys")[1].split(";")[0])]
        vals = [int(x, 16) for x in re.findall(r"0x([0-9a-f]+)u", text.split(f"otx_{name}_exc_vals")[1].split(";")[0])]
        assert len(keys) == len(vals) > 0
        assert keys == sorted(keys)
        for kk, vv in zip(keys, vals):
            assert f2u(fn(u2f(kk))) == vv


def test_division_correctly_rounded():
    host = _host_math()
    rng = np.random.default_rng(9)
    a = rng.standard_normal(5000).astype(np.float32)
    b = rng.uniform(1.0, 3000.0, 5000).astype(np.float32)
    from fractions import Fraction

    for x, y in zip(a[:500], b[:500]):
        got = host.otx_host_div_rn(float(x), float(y))
        exact = Fraction(float(x)) / Fraction(float(y))
        # neighbours of the result bracket the exact quotient within half an ulp
        u = f2u(got)
        lo_n, hi_n = u2f(u - 1) if got != 0 else 0.0, u2f(u + 1)
        err = abs(Fraction(got) - exact)
        assert err <= abs(Fraction(hi_n) - Fraction(got)) / 2 and err <= abs(Fraction(got) - Fraction(lo_n)) / 2


def test_scale():
    assert orc.scale(64) == 0.125
    assert orc.scale(128) == float(np.float32(1.0 / math.sqrt(128.0)))
    from open_transformers_amd import _lib

    if _lib.lib_path().exists():
        lib = _lib.load()
        assert lib.otx_softmax_scale(64) == orc.scale(64)
        assert lib.otx_softmax_scale(128) == orc.scale(128)


@pytest.mark.parametrize(
    "x,want",
    [
        (0x3F808000, 0x3F80),  # exact tie, even below: stays
        (0x3F818000, 0x3F82),  # exact tie, odd below: rounds up to even
        (0x3F808001, 0x3F81),  # just above the tie
        (0x3F807FFF, 0x3F80),  # just below the tie
        (0x7F7FFFFF, 0x7F80),  # overflow to +inf
        (0x80000001, 0x8000),  # negative subnormal to -0
        (0x7FC00001, 0x7FC0),  # NaN stays NaN
    ],
)
def test_bf16_rounding(x, want):
    host = _host_math()
    assert host.otx_host_f32_to_bf16(u2f(x)) == want
    assert f2u(orc.load().orc_round_bf16(u2f(x))) >> 16 == want
    from open_transformers_amd import synthetic

    assert int(synthetic.round_to_bf16(np.array([x], dtype=np.uint32).view(np.float32)).view(np.uint32)[0]) >> 16 == want


def test_exp2_table256_entries():
    """Every entry of the softmax path's table (otx_exp2_tab256) is 2^(j/256)
    correctly rounded to binary64, against a 60-digit decimal evaluation."""
    import decimal
    host = _host_math()
    host.otx_host_exp2_tab256.restype = ctypes.c_double
    host.otx_host_exp2_tab256.argtypes = [ctypes.c_int]
    ctx = decimal.Context(prec=60)
    for j in range(256):
        ref = float(ctx.power(decimal.Decimal(2), ctx.divide(decimal.Decimal(j), decimal.Decimal(256))))
        assert host.otx_host_exp2_tab256(j) == ref, j


def test_kernel_exp_paths_exhaustive():
    """Both table-driven exp paths of the kernels equal the correctly rounded
    exp on every binary32 input they decide, checked on every input of their
    domains in one pass (reference: glibc's binary64 exp rounded once where
    that is unambiguous, otx_expf elsewhere).
      otx_expf_fast (x <= 88: all negative bit patterns and [+0, 88]) defers
      only NaN, x > 88 and the eight inputs whose exp lies within 2^-50 of a
      rounding boundary (four of them negative).
      otx_expf_fast_le0 (softmax arguments: x <= 0 or -inf; 256-entry table,
      degree-4 polynomial) has no rounding test and defers nothing: it is
      correct on all 2^31 + 1 inputs, the four hard-to-round negative ones
      included."""
    host = _host_math()
    host.otx_host_exp_paths_check.restype = None
    host.otx_host_exp_paths_check.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)]
    out = (ctypes.c_uint64 * 4)()
    host.otx_host_exp_paths_check(0x80000000, 1 << 31, out)
    bad_f, slow_f, bad_l, n_l = list(out)
    assert bad_f == 0 and bad_l == 0
    assert slow_f == (1 << 23) - 1 + 4  # negative NaNs + four hard-to-round inputs
    assert n_l == (1 << 31) - ((1 << 23) - 1)  # every negative pattern but the NaNs, -0 and -inf included
    host.otx_host_exp_paths_check(0, f2u(88.0) + 1, out)
    bad_f, slow_f, bad_l, n_l = list(out)
    assert bad_f == 0 and slow_f == 4
    assert bad_l == 0 and n_l == 1  # +0 (exp(0) = 1)


def test_log_rsqrt_tables_complete_exhaustive():
    """otx_logf (LSE) and otx_rsqrtf (RMSNorm's rstd) on every finite positive
    binary32 input: wherever the binary64 evaluation leaves the binary32
    rounding undecided (the Ziv test), the input is in the function's exception
    table, so the "unreachable" fall-through is never taken; and every table
    value that is used equals libquadmath's logq / 1/sqrtq rounded once."""
    host = _host_math()
    host.otx_host_log_rsqrt_tables_check.restype = None
    host.otx_host_log_rsqrt_tables_check.argtypes = [ctypes.POINTER(ctypes.c_uint64), ctypes.c_void_p,
                                                      ctypes.c_void_p, ctypes.c_int]
    out = (ctypes.c_uint64 * 4)()
    cap = 4096
    hits_log = np.zeros(cap, np.uint32)
    hits_rsqrt = np.zeros(cap, np.uint32)
    host.otx_host_log_rsqrt_tables_check(out, hits_log.ctypes.data, hits_rsqrt.ctypes.data, cap)
    miss_l, miss_r, n_l, n_r = list(out)
    assert miss_l == 0 and miss_r == 0
    assert 0 < n_l <= cap and 0 < n_r <= cap
    host.otx_host_rsqrtf.restype = ctypes.c_float
    host.otx_host_rsqrtf.argtypes = [ctypes.c_float]
    lib = orc.load()
    for u in hits_log[:n_l]:
        x = u2f(int(u))
        assert f2u(host.otx_host_logf(x)) == f2u(lib.orc_logf_quad(x)), hex(int(u))
    for u in hits_rsqrt[:n_r]:
        x = u2f(int(u))
        assert f2u(host.otx_host_rsqrtf(x)) == f2u(orc.rsqrtf(x)), hex(int(u))


def test_division_by_127_through_its_reciprocal():
    """The int8 forward's step RN(pmax / 127) as RN32(RN64(pmax * RN64(1/127))):
    equal to the correctly rounded quotient for every finite binary32 pmax >= 0."""
    host = _host_math()
    host.otx_host_div_127_check.restype = ctypes.c_uint64
    host.otx_host_div_127_check.argtypes = []
    assert host.otx_host_div_127_check() == 0


def test_division_through_one_reciprocal_below_the_normal_range():
    """Below the normal range a quotient can be a binary32 midpoint exactly
    (a = 294 * 2^-149, b = 196: 1.5 * 2^-149), and the plain reciprocal form
    rounds some of those the wrong way; otx_div_by_recip_checked (the bf16
    forward's O = RN(acc / l) and the loss backward's RN(e / Z)) takes the
    division there, and equals the correctly rounded quotient on 2^24 pairs
    whose quotients lie below or near the normal range and on the directed
    midpoint cases, against exact rational rounding."""
    from fractions import Fraction

    host = _host_math()
    for name in ("otx_host_div_by_recip", "otx_host_div_by_recip_checked"):
        getattr(host, name).restype = ctypes.c_float
        getattr(host, name).argtypes = [ctypes.c_float, ctypes.c_float]
    host.otx_host_div_recip_subnormal_check.restype = ctypes.c_uint64
    host.otx_host_div_recip_subnormal_check.argtypes = [ctypes.c_uint64, ctypes.c_uint64,
                                                        ctypes.POINTER(ctypes.c_uint64)]
    unchecked = ctypes.c_uint64(0)
    assert host.otx_host_div_recip_subnormal_check(1 << 24, 777, ctypes.byref(unchecked)) == 0
    assert unchecked.value > 0  # the check is needed: the plain form misrounds some of these

    def rn32_exact(fr):  # correctly rounded binary32 of a rational below 2^-126 (the fixed-point grid)
        q = abs(fr) / Fraction(2) ** -149
        n = q.numerator // q.denominator
        r = q - n
        if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2):
            n += 1
        return math.copysign(n * 2.0 ** -149, fr)

    for B in range(3, 2048, 2):  # a = (2k + 1) B 2^-149, b = 4 B: quotients (2k + 1) / 4 * 2^-149
        for k in range(0, 16):
            A = (2 * k + 1) * B
            if A >= 1 << 23:
                break
            a, b = u2f(A), float(4 * B)  # a = A * 2^-149 (subnormal), a / b = (2k + 1) / 4 * 2^-149
            exact = rn32_exact(Fraction(a) / Fraction(b))
            assert host.otx_host_div_by_recip_checked(a, b) == exact, (A, B)
    assert host.otx_host_div_by_recip_checked(u2f(294), 196.0) == u2f(2)  # 1.5 * 2^-149 -> 2 * 2^-149 (even)
    assert host.otx_host_div_by_recip(u2f(294), 196.0) == u2f(1)  # the plain form rounds it down


def test_division_through_one_reciprocal():
    """otx_div_by_recip (one binary64 reciprocal per row, then RN32(RN64(a * 1/l))
    per element) equals the correctly rounded quotient: on 2^26 pseudo-random
    pairs against otx_div_rn (a over every binade, l in the row-sum range and
    beyond), and on directed cases whose quotients lie next to binary32
    midpoints or are subnormal (not midpoints), against exact rational rounding.
    Exact subnormal midpoints are the next test's."""
    from fractions import Fraction

    host = _host_math()
    host.otx_host_div_recip_check.restype = ctypes.c_uint64
    host.otx_host_div_recip_check.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
    assert host.otx_host_div_recip_check(1 << 26, 12345) == 0
    host.otx_host_div_by_recip.restype = ctypes.c_float
    host.otx_host_div_by_recip.argtypes = [ctypes.c_float, ctypes.c_float]
    cases = [(u2f(0x3f800000 + k), float(d)) for k in range(1, 8192, 2) for d in (3, 5, 7, 2049, 4097, 8388607)]
    cases += [(u2f(k), 3.0) for k in range(1, 256)] + [(u2f(0x7f7fffff), 1.5), (-u2f(0x00800001), 3.0)]
    for x, y in cases:
        got = host.otx_host_div_by_recip(x, y)
        exact = Fraction(x) / Fraction(y)
        g = Fraction(got)
        u = f2u(got)
        nxt = Fraction(u2f(u + 1)) if (u & 0x7FFFFFFF) != 0x7F7FFFFF else g * 2
        prv = Fraction(u2f(u - 1)) if (u & 0x7FFFFFFF) else -Fraction(u2f(1))
        assert abs(g - exact) <= abs(nxt - g) / 2 and abs(g - exact) <= abs(g - prv) / 2, (x, y, got)
    assert host.otx_host_div_by_recip(-0.0, 3.0) == 0.0 and math.copysign(1.0, host.otx_host_div_by_recip(-0.0, 3.0)) < 0
