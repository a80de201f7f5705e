"""GPU parity of the decoder-layer operators and of the whole layer
against the CPU oracle, byte for byte.

  GEMM      the three products of a linear layer (y = x w^T, dx = dy w,
            dw = dy^T x) on odd-sized multiples of the tile, bf16 and binary32
            outputs, and on views with padded row pitches in every tile form.
  RMSNorm   forward (y, rstd) and backward (dx, dw) for widths 128, 256, 2048.
  SiLU      forward and backward on random values and on the edges of the
            exp range.
  layer     RMSNorm -> QKV -> RoPE -> attention -> out proj -> residual ->
            RMSNorm -> SwiGLU -> residual, forward output and the gradients of
            the input and of every weight: a small GQA shape with a window, and
            configuration 5 itself (B4 S2048 d2048, 16 x 128 heads, d_ff 5632).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from attn_util import assert_bits_equal
from layer_ref import ORACLE_OPS
from oracle import oracle as orc
from open_transformers_amd import synthetic
from open_transformers_amd.nn import functional as F

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def bf(x):
    return synthetic.round_to_bf16(np.asarray(x, dtype=np.float32))


def gpu(a, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(DEV)


def host(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("M,N,R", [(128, 128, 128), (256, 384, 640), (384, 256, 1024)])
def test_gemm_three_forms(M, N, R):
    print(f"gemm M={M} N={N} R={R}", flush=True)
    rng = np.random.default_rng(M + N + R)
    x = bf(rng.standard_normal((M, R)))
    w = bf(rng.standard_normal((N, R)))
    dy = bf(rng.standard_normal((M, N)))
    gx, gw, gdy = gpu(x), gpu(w), gpu(dy)
    # y = x w^T
    y = F.gemm_bf16(gx, (R, 1), gw, (R, 1), M, N, R)
    assert_bits_equal(host(y), orc.gemm(x, w), "y = x w^T")
    y32 = F.gemm_bf16(gx, (R, 1), gw, (R, 1), M, N, R, out_dtype=torch.float32)
    assert_bits_equal(host(y32), orc.gemm(x, w, out_bf16=False), "y = x w^T (binary32 out)")
    # dx = dy w: dx[m][k] = sum_n dy[m][n] w[n][k]
    dx = F.gemm_bf16(gdy, (N, 1), gw, (1, R), M, R, N)
    assert_bits_equal(host(dx), orc.gemm(dy, w.T), "dx = dy w")
    # dw = dy^T x: dw[n][k] = sum_m dy[m][n] x[m][k]
    dw = F.gemm_bf16(gdy, (1, N), gx, (1, R), N, R, M)
    assert_bits_equal(host(dw), orc.gemm(dy.T, x.T), "dw = dy^T x")


@pytest.mark.parametrize("variant", [0, 1, 2, 3])
def test_gemm_padded_strides(variant):
    """Operands that are views into larger buffers: a row pitch past the logical
    width (still a multiple of 8 elements) and a start 8 elements into the buffer,
    for the three layouts.  The copies into LDS (straight from global memory for an
    i-contiguous operand, through registers for an r-contiguous one) address rows
    by the stride, not by the logical width."""
    M, N, R, PAD = 256, 384, 256, 40
    print(f"gemm padded strides variant {variant}", flush=True)
    rng = np.random.default_rng(77 + variant)
    x = bf(rng.standard_normal((M, R)))
    w = bf(rng.standard_normal((N, R)))
    dy = bf(rng.standard_normal((M, N)))

    def padded(a):  # a [rows, cols] placed at element offset 8 of a buffer with row pitch cols + PAD
        rows, cols = a.shape
        buf = torch.zeros(8 + rows * (cols + PAD), dtype=torch.bfloat16, device=DEV)
        view = buf[8:].view(rows, cols + PAD)
        view[:, :cols] = gpu(a)
        return view, cols + PAD

    px, lx = padded(x)
    pw, lw = padded(w)
    pdy, ldy = padded(dy)
    y = F.gemm_bf16(px, (lx, 1), pw, (lw, 1), M, N, R, variant=variant)
    assert_bits_equal(host(y), orc.gemm(x, w), "y = x w^T")
    dx = F.gemm_bf16(pdy, (ldy, 1), pw, (1, lw), M, R, N, variant=variant)
    assert_bits_equal(host(dx), orc.gemm(dy, w.T), "dx = dy w")
    dw = F.gemm_bf16(pdy, (1, ldy), px, (1, lx), N, R, M, variant=variant)
    assert_bits_equal(host(dw), orc.gemm(dy.T, x.T), "dw = dy^T x")


@pytest.mark.parametrize("rows,D", [(64, 128), (256, 256), (96, 2048)])
def test_rmsnorm_fwd_bwd(rows, D):
    print(f"rmsnorm rows={rows} D={D}", flush=True)
    rng = np.random.default_rng(rows + D)
    x = bf(rng.standard_normal((rows, D)) * 2)
    w = bf(1 + 0.2 * rng.standard_normal(D))
    dy = bf(rng.standard_normal((rows, D)))
    gx, gw = gpu(x).requires_grad_(), gpu(w).requires_grad_()
    y = F.rms_norm(gx, gw, 1e-5)
    y.backward(gpu(dy))
    torch.cuda.synchronize()
    ry, rstd = orc.rmsnorm_fwd(x, w, 1e-5)
    rdx, rdw = orc.rmsnorm_bwd(x, w, rstd, dy)
    assert_bits_equal(host(y), ry, "y")
    assert_bits_equal(host(gx.grad), rdx, "dx")
    assert_bits_equal(host(gw.grad), bf(rdw), "dw (bf16 weight)")


@pytest.mark.parametrize("rows,D,bf16,offset", [
    (131072, 128, True, 0),      # the OPEN-1B q-norm rows (16 heads x 8192 tokens): 4096 partial rows in the dw fold
    (32 * 4100, 128, True, 0),   # more than one 4096-row block of partials
    (8192, 2048, True, 0),       # the residual-stream norm
    (4160, 32, True, 0), (2080, 64, False, 0), (96, 1024, False, 0),
    (64, 96, True, 0), (64, 4096, True, 0),  # widths outside the row-group kernels
    (256, 128, True, 1),         # rows not 16-byte aligned: the general kernels
])
def test_rmsnorm_widths_and_layouts(rows, D, bf16, offset):
    """Every RMSNorm path (row-group kernels for D = 32 G, G a power of two up to 64,
    the general kernels otherwise or for unaligned rows) against the oracle."""
    print(f"rmsnorm rows={rows} D={D} bf16={bf16} offset={offset}", flush=True)
    rng = np.random.default_rng(rows + D + offset)
    dt = torch.bfloat16 if bf16 else torch.float32
    rnd = bf if bf16 else (lambda a: np.asarray(a, dtype=np.float32))
    x = rnd(rng.standard_normal((rows, D)) * 2)
    w = rnd(1 + 0.2 * rng.standard_normal(D))
    dy = rnd(rng.standard_normal((rows, D)))
    buf = torch.empty(rows * D + offset, dtype=dt, device="cuda:0")
    gx = buf[offset:].view(rows, D)
    gx.copy_(torch.from_numpy(x).to(dt))
    gx.requires_grad_()
    gw = torch.from_numpy(w).to(dt).to("cuda:0").requires_grad_()
    y = F.rms_norm(gx, gw, 1e-5)
    y.backward(torch.from_numpy(dy).to(dt).to("cuda:0"))
    torch.cuda.synchronize()
    ry, rstd = orc.rmsnorm_fwd(x, w, 1e-5, out_bf16=bf16)
    rdx, rdw = orc.rmsnorm_bwd(x, w, rstd, dy, out_bf16=bf16)
    assert_bits_equal(host(y), ry, "y")
    assert_bits_equal(host(gx.grad), rdx, "dx")
    assert_bits_equal(host(gw.grad), rnd(rdw), "dw (weight dtype)")


def test_silu_fwd_bwd():
    rng = np.random.default_rng(9)
    x = bf(np.concatenate([rng.standard_normal(50000) * 4, np.linspace(-120, 120, 4097),
                           [0.0, -0.0, 88.5, -88.5, 104.0, -104.0]]))
    dy = bf(rng.standard_normal(x.size))
    gx = gpu(x).requires_grad_()
    y = F.silu(gx)
    y.backward(gpu(dy))
    torch.cuda.synchronize()
    assert_bits_equal(host(y), orc.silu_fwd(x), "silu")
    assert_bits_equal(host(gx.grad), orc.silu_bwd(x, dy), "silu backward")


def _make_layer(B, T, d, H, Hkv, hd, dff, window, seed):
    from open_transformers_amd.nn.layer import DecoderLayer, rope_tables

    rng = np.random.default_rng(seed)
    params = {}
    layer_cpu = DecoderLayer(d, H, Hkv, hd, dff, window=window, ops=ORACLE_OPS)
    with torch.no_grad():
        for n, p in layer_cpu.named_parameters():
            if n.startswith("norm"):
                v = bf(1 + 0.1 * rng.standard_normal(tuple(p.shape)))
            else:
                v = bf(rng.standard_normal(tuple(p.shape)) * 0.02)
            params[n] = v
            p.copy_(torch.from_numpy(v))
    layer_gpu = DecoderLayer(d, H, Hkv, hd, dff, window=window, device=DEV)
    with torch.no_grad():
        for n, p in layer_gpu.named_parameters():
            p.copy_(gpu(params[n]))
    x = bf(rng.standard_normal((B, T, d)))
    dy = bf(rng.standard_normal((B, T, d)))
    cos, sin = rope_tables(T, hd, 10000.0)
    return layer_cpu, layer_gpu, x, dy, cos, sin


def _compare_layer(layer_cpu, layer_gpu, x, dy, cos, sin):
    xc = torch.from_numpy(x).to(torch.bfloat16).requires_grad_()
    yc = layer_cpu(xc, cos, sin)
    yc.backward(torch.from_numpy(dy).to(torch.bfloat16))
    xg = gpu(x).requires_grad_()
    yg = layer_gpu(xg, cos.to(DEV), sin.to(DEV))
    yg.backward(gpu(dy))
    torch.cuda.synchronize()
    assert_bits_equal(host(yg), yc.detach().float().numpy(), "layer output")
    assert_bits_equal(host(xg.grad), xc.grad.float().numpy(), "d input")
    pc = dict(layer_cpu.named_parameters())
    for n, p in layer_gpu.named_parameters():
        assert_bits_equal(host(p.grad), pc[n].grad.float().numpy(), f"d {n}")


def test_layer_small_gqa_window():
    print("layer B2 T128 d256 H4 Hkv2 hd64 dff512 window 64", flush=True)
    _compare_layer(*_make_layer(2, 128, 256, 4, 2, 64, 512, 64, seed=21))


def test_layer_config5():
    print("layer config 5: B4 S2048 d2048 16x128 dff5632", flush=True)
    _compare_layer(*_make_layer(4, 2048, 2048, 16, 16, 128, 5632, 0, seed=55))
