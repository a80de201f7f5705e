"""GPU checks of the two hardware facts the kernels rest on.

1. v_mfma_f32_32x32x1_2b_f32 and v_mfma_f32_16x16x1_4b_f32 compute exactly
   fmaf(a, b, c) per output (adversarial inputs: random binary32, bf16
   products, cancellation, subnormal inputs/products/results, signed zeros,
   ties), with the documented lane layouts.
2. The kernels' exp and log are the oracle's correctly rounded exp and log:
   order-independent checksums over whole ranges of binary32 inputs agree.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _row(r: int, h: int) -> int:
    return 8 * ((r & 15) >> 2) + 4 * h + (r & 3)


def _gen(cat: int, rng: np.random.Generator, n: int) -> np.ndarray:
    sign = rng.integers(0, 2, n).astype(np.uint32) << 31
    mant = rng.integers(0, 1 << 23, n).astype(np.uint32)

    def fl(elo, ehi, m=mant):
        e = rng.integers(elo + 127, ehi + 128, n).astype(np.uint32)
        return (sign | (e << 23) | m).view(np.float32)

    if cat == 0:
        return fl(-20, 20)
    if cat == 1:
        return fl(-10, 10, mant & np.uint32(0x7F0000))
    if cat == 2:
        return fl(-70, -60)
    if cat == 3:
        return (sign | mant).view(np.float32)  # subnormals
    if cat == 4:
        z = np.array([0.0, -0.0, 1.0, -1.0, 1e-30, -1e-30], dtype=np.float32)
        return z[rng.integers(0, 6, n)]
    return fl(-80, -40)


@pytest.mark.parametrize("cat", range(6))
def test_mfma_is_fmaf(cat):
    import torch
    from open_transformers_amd import _lib

    rng = np.random.default_rng(100 + cat)
    G = 64
    a = _gen(cat, rng, G * 64).reshape(G, 64)
    b = _gen(cat if cat != 3 else 0, rng, G * 64).reshape(G, 64)
    c = _gen(cat, rng, G * 32 * 64).reshape(G, 32, 64)
    if cat == 2:  # exact cancellation targets
        c[:, ::2, :] = -c[:, ::2, :]
    dev = torch.device("cuda:0")
    ta, tb, tc = (torch.from_numpy(x.copy()).to(dev) for x in (a, b, c))
    out = torch.empty_like(tc)
    lib = _lib.load()
    rc = lib.otx_selftest_mfma(ta.data_ptr(), tb.data_ptr(), tc.data_ptr(), out.data_ptr(), G,
                               torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "otx_selftest_mfma")
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    r = np.arange(32)[:, None]
    lane = np.arange(64)[None, :]
    h = lane >> 5
    blk = r >> 4
    arow = 32 * blk + (8 * ((r & 15) >> 2) + 4 * h + (r & 3))
    bcol = 32 * blk + (lane & 31)
    A = a[:, arow]
    Bv = b[:, bcol]
    want = orc.fmaf(A, Bv, c)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (
        f"{int(np.count_nonzero(got.view(np.uint32) != want.view(np.uint32)))} MFMA results differ from fmaf")


def _mfma16(a, b, c):
    import torch
    from open_transformers_amd import _lib

    dev = torch.device("cuda:0")
    ta, tb, tc = (torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dev) for x in (a, b, c))
    out = torch.empty_like(tc)
    rc = _lib.load().otx_selftest_mfma16(ta.data_ptr(), tb.data_ptr(), tc.data_ptr(), out.data_ptr(), a.shape[0],
                                         torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "otx_selftest_mfma16")
    torch.cuda.synchronize()
    return out.cpu().numpy()


# v_mfma_f32_16x16x1_4b_f32, as the dK/dV kernel assumes: result register r of
# lane L is block r // 4, row 4 (L // 16) + r % 4, column L % 16; A of block k,
# row i comes from lane 16 k + i, B of block k, column j from lane 16 k + j.
_R16 = np.arange(16)[:, None]
_L16 = np.arange(64)[None, :]
A_LANE16 = 16 * (_R16 >> 2) + 4 * (_L16 >> 4) + (_R16 & 3)
B_LANE16 = 16 * (_R16 >> 2) + (_L16 & 15) + 0 * _R16


def test_mfma16_lane_layout():
    # small integers (every result exact): which lane's A and B feed each output
    idx = np.arange(1, 65, dtype=np.float32)[None, :]
    one = np.ones((1, 64), np.float32)
    zero = np.zeros((1, 16, 64), np.float32)
    got_a = _mfma16(idx, one, zero)[0]
    got_b = _mfma16(one, idx, zero)[0]
    assert np.array_equal(got_a, (A_LANE16 + 1).astype(np.float32))
    assert np.array_equal(got_b, (B_LANE16 + 1).astype(np.float32))


@pytest.mark.parametrize("cat", range(6))
def test_mfma16_is_fmaf(cat):
    rng = np.random.default_rng(300 + cat)
    G = 64
    a = _gen(cat, rng, G * 64).reshape(G, 64)
    b = _gen(cat if cat != 3 else 0, rng, G * 64).reshape(G, 64)
    c = _gen(cat, rng, G * 16 * 64).reshape(G, 16, 64)
    if cat == 2:  # exact cancellation targets
        c[:, ::2, :] = -c[:, ::2, :]
    got = _mfma16(a, b, c)
    want = orc.fmaf(a[:, A_LANE16], b[:, B_LANE16], c)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (
        f"{int(np.count_nonzero(got.view(np.uint32) != want.view(np.uint32)))} MFMA results differ from fmaf")


def _f2u(x: float) -> int:
    return int(np.array([x], dtype=np.float32).view(np.uint32)[0])


EXP_RANGES = [
    (_f2u(-88.0), 1 << 22),      # exp(x) crosses into the subnormal range
    (_f2u(-103.0), 1 << 21),     # deep subnormal results down to +0
    (0x80000000, 1 << 22),       # tiny negative x: results just below 1
    (_f2u(-0.5), 1 << 22),
    (_f2u(-10.0), 1 << 22),
    (_f2u(0.25), 1 << 22),
    (0xB3000000 - 4096, 8192),   # around the exception -2^-25
]
LOG_RANGES = [
    (_f2u(1.0), 1 << 23),        # [1, 2)
    (_f2u(2048.0), 1 << 22),
    (_f2u(0.7), 1 << 21),
]


def _gpu_checksum(which: int, lo: int, count: int) -> int:
    import torch
    from open_transformers_amd import _lib

    nblk = 1024
    part = torch.zeros(nblk, dtype=torch.int64, device="cuda:0")
    lib = _lib.load()
    rc = lib.otx_selftest_math(which, lo, count, part.data_ptr(), nblk, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "otx_selftest_math")
    torch.cuda.synchronize()
    return int(part.cpu().numpy().view(np.uint64).sum(dtype=np.uint64))


@pytest.mark.parametrize("lo,count", EXP_RANGES)
def test_gpu_exp_matches_oracle(lo, count):
    assert _gpu_checksum(0, lo, count) == orc.math_checksum(0, lo, count)


# The kernels' batched exp (two passes per chunk, wave-wide fallback to otx_expf):
# ranges around every negative hard-to-round input (the fallback runs), plus, for
# the checked variant, positive inputs (which must take the fallback) and the
# most negative values up to -inf.
BATCH_RANGES = [
    (0xB3000000 - 4096, 8192),   # -2^-25
    (0xBAE0E25C - 2048, 4096),
    (0xBBF0EDF1 - 2048, 4096),
    (0xC16912CD - 2048, 4096),
    (0x80000000, 1 << 22),
    (_f2u(-10.0), 1 << 22),
    (_f2u(-90.0), 1 << 20),      # subnormal results
]
CHECKED_ONLY = [
    (_f2u(0.25), 1 << 20),
    (_f2u(80.0), 1 << 20),       # up to overflow to +inf
    (0xFF800000 - 4095, 4096),   # the most negative finite values, then -inf
]


@pytest.mark.parametrize("lo,count", BATCH_RANGES + CHECKED_ONLY)
def test_gpu_batched_exp_checked_matches_oracle(lo, count):
    assert _gpu_checksum(2, lo, count) == orc.math_checksum(0, lo, count)


@pytest.mark.parametrize("lo,count", BATCH_RANGES)
def test_gpu_batched_exp_le0_matches_oracle(lo, count):
    assert _gpu_checksum(3, lo, count) == orc.math_checksum(0, lo, count)


@pytest.mark.parametrize("lo,count", LOG_RANGES)
def test_gpu_log_matches_oracle(lo, count):
    assert _gpu_checksum(1, lo, count) == orc.math_checksum(1, lo, count)


# The kernels' binary32 -> bf16 rounding (the conversion instruction on the device)
# against the oracle's round-to-nearest-even with quiet NaNs, over every bit pattern.
@pytest.mark.parametrize("lo", [0, 1 << 30, 2 << 30, 3 << 30])
def test_gpu_bf16_rounding_matches_oracle_everywhere(lo):
    count = 1 << 30
    assert _gpu_checksum(4, lo, count) == orc.math_checksum(4, lo, count)


# The int8-PV quantizer's rounding (v_cvt_pk_u8_f32, byte insert) against rint over
# every bit pattern of [+0, 128), the range p * 127/pmax lies in.
@pytest.mark.parametrize("lo,count", [(0, 1 << 30), (1 << 30, 0x43000000 - (1 << 30))])
def test_gpu_int8_quantizer_rounding_matches_rint(lo, count):
    assert _gpu_checksum(5, lo, count) == orc.math_checksum(5, lo, count)
