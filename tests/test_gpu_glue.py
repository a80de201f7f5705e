"""The fused layer kernels against the reference's torch compositions, bit for bit.

``rope_heads`` replaces apply_rope (rope.py:103-125) + transpose(1, 2).contiguous()
(attention_repop.py:143-149), ``heads`` / ``merge_heads`` the other layout changes
(attention_repop.py:150,155) and ``swiglu`` the product silu(gate) * up over
gu.chunk(2, -1) (ffn_repop.py:52-54).  The checker runs those compositions with
torch on the CPU (SiLU from the C oracle), forward and autograd backward, and
the GPU results must equal them byte for byte: the outputs and the gradients,
bf16 and binary32, at the OPEN-1B shapes and on inputs with signed zeros,
subnormals, huge values and near-ties.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from layer_ref import heads_ref, merge_heads_ref, rope_heads_ref, swiglu_ref
from open_transformers_amd.nn import functional as F
from open_transformers_amd.nn.layer import rope_tables

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def special(shape, seed, dtype, clip=None):
    g = torch.Generator().manual_seed(seed)
    v = torch.randn(shape, generator=g)
    flat = v.view(-1)
    n = flat.numel()
    idx = torch.randint(0, n, (n // 8,), generator=g)
    kinds = torch.randint(0, 6, (idx.numel(),), generator=g)
    table = torch.tensor([0.0, -0.0, 2.0 ** -128, -(2.0 ** -128), 3.0e37, 1.0 + 2.0 ** -8])
    flat[idx] = table[kinds]
    if clip is not None:
        v.clamp_(-clip, clip)
    return v.to(dtype)


def same_bits(a: torch.Tensor, b: torch.Tensor) -> bool:
    a, b = a.detach().cpu(), b.detach().cpu()
    if a.dtype != b.dtype or a.shape != b.shape:
        return False
    iv = torch.int16 if a.dtype == torch.bfloat16 else torch.int32
    return torch.equal(a.contiguous().view(iv), b.contiguous().view(iv))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,T,H,D", [(4, 2048, 16, 128), (4, 2048, 4, 128), (2, 96, 3, 64), (1, 32, 1, 8)])
def test_rope_heads_matches_reference(dtype, B, T, H, D):
    print(f"rope_heads {dtype} B{B} T{T} H{H} D{D}", flush=True)
    cos, sin = rope_tables(T, D, 500000.0)
    x = special((B, T, H, D), 1 + H, dtype)
    g = special((B, H, T, D), 2 + H, dtype)
    g.view(-1)[:D] = -0.0
    xc = x.clone().requires_grad_(True)
    yc = rope_heads_ref(xc, cos, sin)
    yc.backward(g)
    xg = x.to(DEV).requires_grad_(True)
    yg = F.rope_heads(xg, cos.to(DEV), sin.to(DEV))
    yg.backward(g.to(DEV))
    torch.cuda.synchronize()
    assert yg.is_contiguous() and yg.shape == (B, H, T, D)
    assert same_bits(yg, yc), "forward"
    assert same_bits(xg.grad, xc.grad), "backward"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_head_layout_swaps_match_reference(dtype):
    print(f"heads / merge_heads {dtype}", flush=True)
    B, T, H, D = 2, 160, 4, 128
    v = special((B, T, H, D), 3, dtype)
    o = special((B, H, T, D), 4, dtype)
    dv = special((B, H, T, D), 5, dtype)
    do = special((B, T, H * D), 6, dtype)
    vc, oc = v.clone().requires_grad_(True), o.clone().requires_grad_(True)
    ref_v, ref_o = heads_ref(vc), merge_heads_ref(oc)
    ref_v.backward(dv)
    ref_o.backward(do)
    vg, og = v.to(DEV).requires_grad_(True), o.to(DEV).requires_grad_(True)
    hv, mo = F.heads(vg), F.merge_heads(og)
    hv.backward(dv.to(DEV))
    mo.backward(do.to(DEV))
    torch.cuda.synchronize()
    assert same_bits(hv, ref_v) and same_bits(mo, ref_o)
    assert same_bits(vg.grad, vc.grad) and same_bits(og.grad, oc.grad)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,Fw", [(1024, 5632), (64, 8), (33, 136)])
def test_swiglu_matches_reference(dtype, rows, Fw):
    print(f"swiglu {dtype} rows{rows} F{Fw}", flush=True)
    # gate within SiLU's range of interest; up and dh below 1e18 so that no product
    # overflows (an inf times a zero derivative would make NaNs, whose payloads
    # are not part of the contract)
    gu = special((rows, 2 * Fw), 7 + Fw, dtype, clip=1e18)
    gu[:, :Fw] = gu[:, :Fw].float().clamp(-100.0, 100.0).to(dtype)
    dh = special((rows, Fw), 8 + Fw, dtype, clip=1e18)
    guc = gu.clone().requires_grad_(True)
    hc = swiglu_ref(guc)
    hc.backward(dh)
    gug = gu.to(DEV).requires_grad_(True)
    hg = F.swiglu(gug)
    hg.backward(dh.to(DEV))
    torch.cuda.synchronize()
    assert same_bits(hg, hc), "forward"
    assert same_bits(gug.grad, guc.grad), "backward"


def test_swiglu_batched_shape_and_noncontiguous_grad():
    """[B, T, 2F] input (the layer's shape) and a non-contiguous incoming gradient."""
    print("swiglu batched", flush=True)
    B, T, Fw = 2, 64, 256
    gu = special((B, T, 2 * Fw), 9, torch.bfloat16, clip=50.0)
    dh_big = special((B, T, 2 * Fw), 10, torch.bfloat16, clip=1e18)
    dh = dh_big[..., ::2]
    guc = gu.clone().requires_grad_(True)
    swiglu_ref(guc).backward(dh)
    gug = gu.to(DEV).requires_grad_(True)
    hg = F.swiglu(gug)
    assert hg.shape == (B, T, Fw)
    hg.backward(dh_big.to(DEV)[..., ::2])
    torch.cuda.synchronize()
    assert same_bits(gug.grad, guc.grad)
    assert np.array_equal(hg.detach().cpu().float().numpy(), swiglu_ref(gu).float().numpy())
