"""GPU check of the allocation-free int8-PV forward (otx_attn_fwd_int8pv_noalloc):
through the C ABI it gives the same O and LSE bytes as otx_attn_fwd_int8pv_ex
with a caller workspace, on two calls in a row that share the library's fixed
device scratch, the first near its 32 MiB limit and the second smaller (so the
second reads nothing the first left behind)."""

from __future__ import annotations

import pytest

from attn_util import make

pytestmark = pytest.mark.gpu

CASES = [
    # (B, H, Hkv, S, D, window, variant): 31.5 MiB of scratch, then 0.1 MiB
    (4, 16, 8, 7168, 128, 0, 0),
    (1, 4, 1, 256, 64, 64, 1),
]


def test_noalloc_int8pv_matches_workspace_entry_point():
    import torch

    from open_transformers_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda:0")
    sid = torch.cuda.current_stream(dev).cuda_stream
    for B, H, Hkv, S, D, window, variant in CASES:
        need = int(lib.otx_attn_fwd_int8pv_workspace_bytes(B, H, Hkv, S, D))
        print(f"noalloc int8-PV: B{B} H{H} Hkv{Hkv} S{S} D{D} window {window} variant {variant} "
              f"scratch {need} bytes", flush=True)
        assert 0 < need <= _lib.NOALLOC_SCRATCH_BYTES
        inp = make(B, H, Hkv, S, D, dtype="bf16", seed=S + window)
        q, k, v = (torch.from_numpy(inp[n]).to(torch.bfloat16).to(dev) for n in ("q", "k", "v"))
        outs = []
        for noalloc in (False, True):
            o = torch.full_like(q, float("nan"))
            lse = torch.full((B, H, S), float("nan"), dtype=torch.float32, device=dev)
            if noalloc:
                rc = lib.otx_attn_fwd_int8pv_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                                     lse.data_ptr(), B, H, Hkv, S, D, window, _lib.DTYPE_BF16,
                                                     variant, sid)
            else:
                ws = torch.empty(need, dtype=torch.uint8, device=dev)
                rc = lib.otx_attn_fwd_int8pv_ex(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                                lse.data_ptr(), B, H, Hkv, S, D, window, _lib.DTYPE_BF16,
                                                ws.data_ptr(), need, variant, sid)
            _lib.check(rc, "int8-PV forward")
            torch.cuda.synchronize()
            outs.append((o, lse))
        (o_ws, lse_ws), (o_na, lse_na) = outs
        assert torch.equal(o_na.view(torch.int16), o_ws.view(torch.int16)), "O differs"
        assert torch.equal(lse_na.view(torch.int32), lse_ws.view(torch.int32)), "LSE differs"
        assert not torch.isnan(lse_na).any()
        del q, k, v, outs, o_ws, lse_ws, o_na, lse_na


def test_noalloc_int8pv_under_graph_capture():
    """The use the header names: a caller that captures the call in a HIP graph.
    One call outside capture first (it resolves the scratch array's device
    address on this device), then the call is captured once and replayed on
    three different inputs copied into the captured tensors; each replay must
    give the workspace entry point's bytes, with eager work and
    synchronizations between the replays."""
    import torch

    from open_transformers_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda:0")
    B, H, Hkv, S, D, window, variant = 2, 8, 2, 1024, 128, 256, 0
    need = int(lib.otx_attn_fwd_int8pv_workspace_bytes(B, H, Hkv, S, D))
    print(f"noalloc int8-PV under graph capture: B{B} H{H} Hkv{Hkv} S{S} D{D} window {window}", flush=True)
    q = torch.empty((B, H, S, D), dtype=torch.bfloat16, device=dev)
    k = torch.empty((B, Hkv, S, D), dtype=torch.bfloat16, device=dev)
    v = torch.empty_like(k)
    o = torch.empty_like(q)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=dev)

    def noalloc(stream):
        rc = lib.otx_attn_fwd_int8pv_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                                             B, H, Hkv, S, D, window, _lib.DTYPE_BF16, variant, stream.cuda_stream)
        _lib.check(rc, "otx_attn_fwd_int8pv_noalloc")

    def load(seed):
        inp = make(B, H, Hkv, S, D, dtype="bf16", seed=seed)
        for t, n in ((q, "q"), (k, "k"), (v, "v")):
            t.copy_(torch.from_numpy(inp[n]).to(torch.bfloat16))

    load(1)
    noalloc(torch.cuda.current_stream(dev))  # outside capture: resolves the array's address
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        noalloc(torch.cuda.current_stream(dev))
    torch.cuda.synchronize()
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    for seed in (2, 3, 4):
        print(f"replay on inputs of seed {seed}", flush=True)
        load(seed)
        o.fill_(float("nan"))
        lse.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        o_ws, lse_ws = torch.full_like(o, float("nan")), torch.full_like(lse, float("nan"))
        rc = lib.otx_attn_fwd_int8pv_ex(q.data_ptr(), k.data_ptr(), v.data_ptr(), o_ws.data_ptr(), lse_ws.data_ptr(),
                                        B, H, Hkv, S, D, window, _lib.DTYPE_BF16, ws.data_ptr(), need, variant,
                                        torch.cuda.current_stream(dev).cuda_stream)
        _lib.check(rc, "otx_attn_fwd_int8pv_ex")
        torch.cuda.synchronize()
        assert torch.equal(o.view(torch.int16), o_ws.view(torch.int16)), f"O differs (replay, seed {seed})"
        assert torch.equal(lse.view(torch.int32), lse_ws.view(torch.int32)), f"LSE differs (replay, seed {seed})"
        assert not torch.isnan(lse).any()
    del g
