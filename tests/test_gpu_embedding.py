"""GPU parity of the token embedding (csrc/embedding.hip) against the CPU
oracle, byte for byte: the forward gather (including NaN rows for ids outside
the vocabulary) and the position-ordered per-id fold of the backward, for bf16
and binary32 weights, heavy id repetition (few distinct ids: long segments),
and the OPEN-1B shape (vocabulary 128256, width 2048, 4 x 2048 positions)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from attn_util import assert_bits_equal
from oracle import oracle as orc
from open_transformers_amd import synthetic
from open_transformers_amd.nn import embedding as E

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.mark.parametrize("npos,V,D,dtype,distinct", [
    (4096, 64, 256, torch.bfloat16, 64),
    (1000, 5000, 128, torch.float32, 5000),
    (777, 300, 64, torch.bfloat16, 3),
    (8192, 128256, 2048, torch.bfloat16, 128256),
])
def test_embedding_fwd_bwd_bitexact(npos, V, D, dtype, distinct):
    print(f"embedding npos={npos} V={V} D={D} {dtype} distinct={distinct}", flush=True)
    rng = np.random.default_rng(npos + V)
    ids = rng.integers(0, distinct, npos).astype(np.int64)
    g = rng.standard_normal((npos, D)).astype(np.float32)
    if dtype == torch.bfloat16:
        g = synthetic.round_to_bf16(g)
    gen = torch.Generator(device=DEV).manual_seed(npos)
    wt = torch.randn(V, D, device=DEV, generator=gen).to(dtype).requires_grad_()
    it = torch.from_numpy(ids).to(DEV)
    out = E.embedding(it.view(1, -1), wt)
    out.backward(torch.from_numpy(g).to(dtype).to(DEV).view(1, npos, D))
    torch.cuda.synchronize()
    # the forward is a row gather: compare raw bits with torch's own indexing on the device
    ibits = torch.int16 if dtype == torch.bfloat16 else torch.int32
    assert torch.equal(out.detach()[0].view(ibits), wt.detach()[it].view(ibits)), "forward rows"
    ref = orc.embedding_bwd(ids, g, V, out_bf16=dtype == torch.bfloat16)
    assert_bits_equal(wt.grad.float().cpu().numpy(), ref, "weight gradient")


def test_embedding_out_of_range_ids():
    w = torch.randn(16, 64, device=DEV).to(torch.bfloat16).requires_grad_()
    ids = torch.tensor([[3, 16, -1, 3]], device=DEV)
    out = E.embedding(ids, w)
    out.backward(torch.ones_like(out))
    torch.cuda.synchronize()
    o = out.float().cpu()
    assert torch.isnan(o[0, 1]).all() and torch.isnan(o[0, 2]).all() and not torch.isnan(o[0, 0]).any()
    gw = w.grad.float().cpu()
    assert (gw[3] == 2.0).all() and (gw[torch.arange(16) != 3] == 0).all()
