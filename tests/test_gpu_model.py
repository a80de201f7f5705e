"""A tiny model's training step end to end on the GPU, byte for byte against
the same module code on the CPU oracle.

The model is ``nn.model.Llama3`` with the OPEN-1B module set
(configs/model/llama3_1b_proxy_repop.yaml): untied embedding, q/k RMSNorm,
sliding-window layers with a full-causal layer every second layer and at the
end, int8-PV or binary32 attention, SwiGLU, final RMSNorm, output projection
and the fused CE + z-loss.  One step = forward, loss, backward; compared: both
loss scalars and the gradient of every parameter.

Activation checkpointing (parallelize_llama3_repop.py:107-130 of the
reference) wraps every block with ``checkpoint_wrapper``: the recompute must
repeat the forward's bytes, and with ``attention_checkpoint_contexts`` as the
``context_fn`` the recompute reuses the recorded attention results instead.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from attn_util import assert_bits_equal
from layer_ref import ORACLE_OPS
from open_transformers_amd import synthetic
from open_transformers_amd.nn import flash_attention as fa
from open_transformers_amd.nn.model import Llama3

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

CFG = dict(vocab_size=1024, d_model=256, n_layers=3, n_heads=4, n_kv_heads=2, head_dim=64, d_ff=512,
           rope_theta=500000.0, swa_window=64, swa_full_every=2, qk_norm=True)
B, T, COEFF = 2, 128, 1e-4


def _models(int8_pv, seed=3):
    cpu = Llama3(**CFG, attn_int8_pv=int8_pv, ops=ORACLE_OPS)
    gpu = Llama3(**CFG, attn_int8_pv=int8_pv, device=DEV)
    rng = np.random.default_rng(seed)
    with torch.no_grad():
        for (n, pc), (_, pg) in zip(cpu.named_parameters(), gpu.named_parameters()):
            v = (1 + 0.1 * rng.standard_normal(tuple(pc.shape))) if "norm" in n else rng.standard_normal(
                tuple(pc.shape)) * 0.05
            v = torch.from_numpy(synthetic.round_to_bf16(v.astype(np.float32)))
            pc.copy_(v)
            pg.copy_(v.to(DEV))
    ids = rng.integers(0, CFG["vocab_size"], (B, T))
    labels = rng.integers(0, CFG["vocab_size"], (B, T))
    return cpu, gpu, torch.from_numpy(ids), torch.from_numpy(labels)


def _step(model, ids, labels):
    for p in model.parameters():
        p.grad = None
    ce, z = model.loss(ids, labels, COEFF)
    (ce + z).backward()
    out = {"ce": ce.detach().float().cpu().numpy().reshape(1), "z": z.detach().float().cpu().numpy().reshape(1)}
    for n, p in model.named_parameters():
        out[n.replace("._checkpoint_wrapped_module", "")] = p.grad.detach().float().cpu().numpy()
    return out


@pytest.mark.parametrize("int8_pv", [False, True], ids=["bf16-attention", "int8pv-attention"])
def test_tiny_model_step_bitexact(int8_pv):
    print(f"model step int8_pv={int8_pv}", flush=True)
    cpu, gpu, ids, labels = _models(int8_pv)
    ref = _step(cpu, ids, labels)
    got = _step(gpu, ids.to(DEV), labels.to(DEV))
    torch.cuda.synchronize()
    for n in ref:
        assert_bits_equal(got[n], ref[n], n)


def test_activation_checkpointing_repeats_bytes():
    from torch.distributed.algorithms._checkpoint.checkpoint_wrapper import checkpoint_wrapper

    print("model step under activation checkpointing", flush=True)
    _, gpu, ids, labels = _models(True, seed=4)
    ids, labels = ids.to(DEV), labels.to(DEV)
    plain = _step(gpu, ids, labels)
    blocks = list(gpu.blocks)
    for i, blk in enumerate(blocks):
        gpu.blocks[i] = checkpoint_wrapper(blk, preserve_rng_state=False)
    recomputed = _step(gpu, ids, labels)
    for i, blk in enumerate(blocks):
        gpu.blocks[i] = checkpoint_wrapper(blk, preserve_rng_state=False,
                                           context_fn=fa.attention_checkpoint_contexts)
    cached = _step(gpu, ids, labels)
    torch.cuda.synchronize()
    for n in plain:
        assert_bits_equal(recomputed[n].reshape(-1), plain[n].reshape(-1), f"recompute {n}")
        assert_bits_equal(cached[n].reshape(-1), plain[n].reshape(-1), f"cached attention {n}")


@pytest.mark.parametrize("int8_pv", [False, True], ids=["bf16-attention", "int8pv-attention"])
def test_checkpointed_first_forward_writes_no_score_cache(int8_pv, monkeypatch):
    """checkpoint_wrapper without a context_fn (the reference's GPU default,
    parallelize_llama3_repop.py:107-130) drops the first forward's saved
    tensors: that forward must allocate no score cache; the recompute in the
    backward writes one per attention call, and the step's bytes equal the
    unwrapped model's."""
    from torch.distributed.algorithms._checkpoint.checkpoint_wrapper import checkpoint_wrapper

    print(f"checkpointed model step, score-cache allocations, int8_pv={int8_pv}", flush=True)
    _, gpu, ids, labels = _models(int8_pv, seed=6)
    ids, labels = ids.to(DEV), labels.to(DEV)
    plain = _step(gpu, ids, labels)
    for i, blk in enumerate(list(gpu.blocks)):
        gpu.blocks[i] = checkpoint_wrapper(blk, preserve_rng_state=False)
    calls = []
    orig = fa._new_score_cache

    def counting(*a, **kw):
        calls.append(a)
        return orig(*a, **kw)

    monkeypatch.setattr(fa, "_new_score_cache", counting)
    params = list(gpu.parameters())
    for p in params:
        p.grad = None
    ce, z = gpu.loss(ids, labels, COEFF)
    torch.cuda.synchronize()
    assert calls == [], f"the first checkpointed forward allocated {len(calls)} score caches"
    (ce + z).backward()
    torch.cuda.synchronize()
    assert len(calls) == len(gpu.blocks), f"{len(calls)} score caches in the recompute, {len(gpu.blocks)} blocks"
    got = {"ce": ce.detach().float().cpu().numpy().reshape(1), "z": z.detach().float().cpu().numpy().reshape(1)}
    for n, p in gpu.named_parameters():
        got[n.replace("._checkpoint_wrapped_module", "")] = p.grad.detach().float().cpu().numpy()
    for n in plain:
        assert_bits_equal(got[n].reshape(-1), plain[n].reshape(-1), f"checkpointed {n}")
