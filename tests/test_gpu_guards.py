"""GPU checks of the operators' host-side guards: a tensor on the wrong device
is refused before any pointer reaches the C ABI (a host pointer handed to a
kernel would fault the GPU instead of raising, unlike torch.nn.Embedding's
device-mismatch error), and a call that cannot run a backward keeps no score
cache.  In the device tests the library loader is replaced by a stub that
fails if called, so no kernel can launch even if a guard regresses."""

from __future__ import annotations

import pytest

from attn_util import make

pytestmark = pytest.mark.gpu


def _no_library(*args, **kwargs):
    raise AssertionError("the C ABI was reached although an argument is on the wrong device")


def test_embedding_refuses_ids_on_another_device(monkeypatch):
    import torch

    from open_transformers_amd import _lib
    from open_transformers_amd.nn.embedding import embedding

    print("guard: embedding ids on the CPU, weight on cuda:0", flush=True)
    weight = torch.zeros(64, 32, dtype=torch.bfloat16, device="cuda:0")
    ids = torch.arange(8)  # CPU
    monkeypatch.setattr(_lib, "load", _no_library)
    with pytest.raises(RuntimeError, match="same device"):
        embedding(ids, weight)


def test_backward_refuses_saved_tensors_on_another_device(monkeypatch):
    import torch

    from open_transformers_amd import _lib
    from open_transformers_amd.nn import flash_attention as fa

    print("guard: flash_attention_backward with o / lse on the CPU", flush=True)
    dev = torch.device("cuda:0")
    q = torch.zeros(1, 2, 64, 64, dtype=torch.bfloat16, device=dev)
    k = torch.zeros(1, 1, 64, 64, dtype=torch.bfloat16, device=dev)
    lse = torch.zeros(1, 2, 64, dtype=torch.float32, device=dev)
    monkeypatch.setattr(_lib, "load", _no_library)
    with pytest.raises(ValueError, match="device"):
        fa.flash_attention_backward(q, k, k, q.cpu(), lse, q, 0)
    with pytest.raises(ValueError, match="device"):
        fa.flash_attention_backward(q, k, k, q, lse.cpu(), q, 0)


def test_no_grad_call_keeps_no_score_cache(monkeypatch):
    import torch

    from open_transformers_amd.nn import flash_attention as fa

    print("no_grad: B1 H4 Hkv2 S128 D128 bf16, both operators", flush=True)
    inp = make(1, 4, 2, 128, 128, dtype="bf16", seed=31)
    q, k, v = (torch.from_numpy(inp[n]).to(torch.bfloat16).to("cuda:0") for n in ("q", "k", "v"))
    prev = fa.set_score_cache(True)
    try:
        for op in (fa.causal_flash_attention, fa.int8pv_causal_flash_attention):
            kw = {"dropout": 0.0} if op is fa.causal_flash_attention else {}
            with_grad = op(q, k.clone().requires_grad_(), v, window=64, **kw).detach()
            calls = []

            def refuse(*a, **kw2):
                calls.append(a)
                raise AssertionError("score-cache forward called under no_grad")

            with monkeypatch.context() as m:
                m.setattr(fa, "flash_attention_forward_sc", refuse)
                m.setattr(fa, "int8pv_flash_attention_forward_sc", refuse)
                with torch.no_grad():
                    plain = op(q, k.clone().requires_grad_(), v, window=64, **kw)
                nograd_inputs = op(q, k, v, window=64, **kw)
            torch.cuda.synchronize()
            assert not calls
            assert torch.equal(plain.view(torch.int16), with_grad.view(torch.int16))
            assert torch.equal(nograd_inputs.view(torch.int16), with_grad.view(torch.int16))
    finally:
        fa.set_score_cache(prev)
