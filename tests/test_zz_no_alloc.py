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
