"""Why the kernels multiply bf16 tensors with the K=1 fp32 matrix instruction.

The bf16 matrix instructions of gfx950 take several products per output per
instruction.  They could replace the QK^T and dO V^T chains only if each
instruction accumulated exactly like the serial fma chain the contract
prescribes.  This test runs one instruction of each shape on raw operand
registers (tests of the lane layout use small integers, where every
summation order is exact) and then compares random inputs with the serial
ascending chain: the layout matches, the rounding does not, so the bf16
instructions stay out of the contract's arithmetic.  Even with exactly one
non-zero product per output (no order question at all) the instruction does
not round like fmaf (test_bf16_mfma_single_product_is_not_fmaf).
"""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

AW = {0: 4, 1: 4, 2: 8, 3: 4, 4: 8}   # bf16 values per lane
CR = {0: 32, 1: 16, 2: 16, 3: 4, 4: 4}  # result registers per lane
KK = {0: 4, 1: 8, 2: 16, 3: 16, 4: 32}  # products per output
NAMES = {0: "32x32x4_2b", 1: "32x32x8", 2: "32x32x16", 3: "16x16x16", 4: "16x16x32"}


def _layout(kind):
    """(lane, reg) of each output and the (lane, element) of A and B for each k."""
    outs, a_idx, b_idx = [], [], []
    for L in range(64):
        for r in range(CR[kind]):
            if kind == 0:
                blk, j, i = r // 16, L % 32, 8 * ((r % 16) // 4) + 4 * (L // 32) + r % 4
                ak = [(i + 32 * blk, k) for k in range(4)]
                bk = [(j + 32 * blk, k) for k in range(4)]
            elif kind in (1, 2):
                j, i, per = L % 32, 8 * (r // 4) + 4 * (L // 32) + r % 4, AW[kind]
                ak = [(i + 32 * (k // per), k % per) for k in range(KK[kind])]
                bk = [(j + 32 * (k // per), k % per) for k in range(KK[kind])]
            else:
                j, i, per = L % 16, 4 * (L // 16) + r, AW[kind]
                ak = [(i + 16 * (k // per), k % per) for k in range(KK[kind])]
                bk = [(j + 16 * (k // per), k % per) for k in range(KK[kind])]
            outs.append((L, r))
            a_idx.append(ak)
            b_idx.append(bk)
    return np.array(outs), np.array(a_idx), np.array(b_idx)


def _run(kind, a_bits, b_bits, c):
    import torch

    from open_transformers_amd import _lib

    dev = torch.device("cuda:0")
    G = a_bits.shape[0]
    ta = torch.from_numpy(a_bits.view(np.int16).copy()).to(dev)
    tb = torch.from_numpy(b_bits.view(np.int16).copy()).to(dev)
    tc = torch.from_numpy(c.copy()).to(dev)
    to = torch.empty_like(tc)
    rc = _lib.load().otx_selftest_mfma_bf16(kind, ta.data_ptr(), tb.data_ptr(), tc.data_ptr(), to.data_ptr(), G,
                                            torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "otx_selftest_mfma_bf16")
    torch.cuda.synchronize()
    return to.cpu().numpy()


def _bits(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _serial(kind, a_bits, b_bits, c):
    outs, ai, bi = _layout(kind)
    a = (a_bits.astype(np.uint32) << 16).view(np.float32)
    b = (b_bits.astype(np.uint32) << 16).view(np.float32)
    acc = c[:, outs[:, 0], outs[:, 1]].copy()
    for k in range(KK[kind]):
        # bf16 x bf16 is exact in binary32, so fma == one rounded addition
        prod = a[:, ai[:, k, 0], ai[:, k, 1]] * b[:, bi[:, k, 0], bi[:, k, 1]]
        acc = (acc + prod).astype(np.float32)
    return acc, outs


@pytest.mark.parametrize("kind", sorted(NAMES), ids=[NAMES[k] for k in sorted(NAMES)])
def test_bf16_mfma_layout_exact_but_not_serial_fma(kind):
    print(f"bf16 matrix instruction {NAMES[kind]}", flush=True)
    rng = np.random.default_rng(40 + kind)
    G = 64
    shape_ab = (G, 64, AW[kind])
    # 1. small integers: every order is exact, so this pins the lane layout
    a = _bits(rng.integers(-8, 9, shape_ab).astype(np.float32))
    b = _bits(rng.integers(-8, 9, shape_ab).astype(np.float32))
    c = rng.integers(-64, 65, (G, 64, CR[kind])).astype(np.float32)
    got = _run(kind, a, b, c)
    want, outs = _serial(kind, a, b, c)
    assert np.array_equal(got[:, outs[:, 0], outs[:, 1]], want)
    # 2. random normal values: the serial fma chain is not what the hardware computes
    a = _bits(rng.standard_normal(shape_ab).astype(np.float32))
    b = _bits(rng.standard_normal(shape_ab).astype(np.float32))
    c = rng.standard_normal((G, 64, CR[kind])).astype(np.float32)
    got = _run(kind, a, b, c)
    want, outs = _serial(kind, a, b, c)
    differ = np.count_nonzero(got[:, outs[:, 0], outs[:, 1]].view(np.uint32) != want.view(np.uint32))
    print(f"  {differ} of {want.size} outputs differ from the serial fma chain", flush=True)
    assert differ > 0


def test_i8_mfma_32x32x32_layout():
    """The int8-PV forward multiplies with v_mfma_i32_32x32x32_i8: integer
    products accumulate exactly in int32 (no rounding, so no order question).
    This pins the lane layout the kernel assumes: A[i][k] in lane i + 32*(k//16),
    byte k % 16; B[k][j] in lane j + 32*(k//16); result register r of lane L
    holds row 8*(r//4) + 4*(L//32) + r%4, column L % 32."""
    import torch

    from open_transformers_amd import _lib

    rng = np.random.default_rng(77)
    G = 32
    a = rng.integers(-128, 128, (G, 64, 16)).astype(np.int8)
    b = rng.integers(-128, 128, (G, 64, 16)).astype(np.int8)
    c = rng.integers(-10**6, 10**6, (G, 64, 16)).astype(np.int32)
    dev = torch.device("cuda:0")
    ta, tb, tc = (torch.from_numpy(x.copy()).to(dev) for x in (a, b, c))
    to = torch.empty_like(tc)
    rc = _lib.load().otx_selftest_mfma_i8(ta.data_ptr(), tb.data_ptr(), tc.data_ptr(), to.data_ptr(), G,
                                          torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "otx_selftest_mfma_i8")
    torch.cuda.synchronize()
    got = to.cpu().numpy()
    A = np.zeros((G, 32, 32), np.int64)
    Bm = np.zeros((G, 32, 32), np.int64)
    for k in range(32):
        A[:, :, k] = a[:, np.arange(32) + 32 * (k // 16), k % 16]
        Bm[:, k, :] = b[:, np.arange(32) + 32 * (k // 16), k % 16]
    prod = A @ Bm
    want = np.empty_like(c)
    for L in range(64):
        for r in range(16):
            i = 8 * (r // 4) + 4 * (L // 32) + r % 4
            want[:, L, r] = c[:, L, r] + prod[:, i, L % 32]
    assert np.array_equal(got, want)


def _single_product(kind, k0, a_vals, b_vals, c):
    """Operands with exactly one non-zero product per output (slot k0 of A and
    B; every other A slot or B slot zero), so no summation order is involved."""
    outs, ai, bi = _layout(kind)
    G = c.shape[0]
    a = np.zeros((G, 64, AW[kind]), np.uint16)
    b = np.zeros((G, 64, AW[kind]), np.uint16)
    a[:, :, k0 % AW[kind]] = a_vals
    for o in range(outs.shape[0]):
        ln, el = bi[o, k0]
        b[:, ln, el] = b_vals[:, ln]
    A = (a.astype(np.uint32) << 16).view(np.float32)
    Bf = (b.astype(np.uint32) << 16).view(np.float32)
    av = A[:, ai[:, k0, 0], ai[:, k0, 1]]
    bv = Bf[:, bi[:, k0, 0], bi[:, k0, 1]]
    return a, b, av, bv, outs


def test_bf16_mfma_single_product_is_not_fmaf():
    """With one non-zero product per output the bf16 instruction has no order
    question left, yet it still does not round like fmaf: c + a*b with
    c = -1e-30, a = b = 1 gives 0.99999994 (fmaf: 1.0, round to nearest even),
    and (+0)*(-0) + (-0) gives +0 (fmaf: -0).  So a serial chain of bf16
    instructions with one useful product each is not the contract's fold, and
    the QK^T / dO V^T chains stay on the binary32 K=1 instruction."""
    from oracle import oracle as orc

    kind, k0, G = 2, 0, 4
    one, zero, negz = np.uint16(0x3F80), np.uint16(0x0000), np.uint16(0x8000)
    c = np.zeros((G, 64, CR[kind]), np.float32)
    av_bits = np.full((G, 64), one, np.uint16)
    bv_bits = np.full((G, 64), one, np.uint16)
    c[0] = np.float32(-1e-30)            # ties-to-even case: fmaf keeps 1.0
    av_bits[1], bv_bits[1] = zero, negz  # signed zero: fmaf gives -0
    c[1] = np.float32(-0.0)
    c[2] = np.float32(2.0 ** -24)        # exact: 1 + 2^-24 rounds to 1 (tie to even) either way
    c[3] = np.float32(0.5)               # exact sum
    a, b, av, bv, outs = _single_product(kind, k0, av_bits, bv_bits, c)
    got = _run(kind, a, b, c)[:, outs[:, 0], outs[:, 1]]
    want = orc.fmaf(av, bv, c[:, outs[:, 0], outs[:, 1]])
    print(f"group 0: got {got[0, 0]!r} want {want[0, 0]!r}; group 1: got {got[1, 0]!r} want {want[1, 0]!r}", flush=True)
    assert want[0, 0] == np.float32(1.0) and got[0, 0] == np.nextafter(np.float32(1.0), np.float32(0.0))
    assert np.signbit(want[1, 0]) and not np.signbit(got[1, 0])
    assert np.array_equal(got[2:].view(np.uint32), want[2:].view(np.uint32))
