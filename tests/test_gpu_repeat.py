"""Run-to-run determinism of the backward on the GPU.

The same workspace and output buffers are reused for many calls whose inputs
alternate between two seeds, so that anything a call might pick up from the
one before it (LDS or cache contents left by the previous workgroup on a CU,
workspace bytes a kernel failed to write) holds the other input's values, and
every other call starts from buffers filled with NaN.  Every call's dq, dk and
dv bytes must equal the oracle's for its input.
"""

from __future__ import annotations

import numpy as np
import pytest

from attn_util import make, oracle_fwd_bwd

pytestmark = pytest.mark.gpu

REPS = 120

CASES = [
    # B, H, Hkv, S, D, window, seed, variant, score cache
    pytest.param(1, 2, 2, 128, 64, 0, 6, 0, False, id="d64-two-kb"),
    pytest.param(1, 2, 2, 128, 64, 0, 6, 2, False, id="d64-four-kb"),
    pytest.param(1, 2, 2, 128, 64, 0, 6, 0, True, id="d64-two-kb-cache"),
    pytest.param(1, 2, 2, 128, 128, 0, 2, 0, False, id="d128-two-kb"),
    pytest.param(2, 4, 2, 160, 128, 64, 3, 0, True, id="gqa-win64-cache"),
    pytest.param(1, 4, 1, 96, 64, 32, 4, 1, False, id="mqa-win32-two-waves"),
]


def _inputs(dev, B, H, Hkv, S, D, window, seed, variant, sc):
    import torch

    from open_transformers_amd.nn.flash_attention import flash_attention_forward, flash_attention_forward_sc

    inp = make(B, H, Hkv, S, D, dtype="bf16", seed=seed)
    ref = oracle_fwd_bwd(inp, window, True)
    t = {n: torch.from_numpy(np.ascontiguousarray(inp[n])).to(torch.bfloat16).to(dev) for n in ("q", "k", "v", "do")}
    if sc:
        o, lse, cache = flash_attention_forward_sc(t["q"], t["k"], t["v"], window=window, variant=variant)
    else:
        (o, lse), cache = flash_attention_forward(t["q"], t["k"], t["v"], window=window, variant=variant), None
    refs = {n: torch.from_numpy(np.ascontiguousarray(ref[n])).to(torch.bfloat16).to(dev) for n in ("dq", "dk", "dv")}
    return t, o, lse, cache, refs


@pytest.mark.parametrize("B,H,Hkv,S,D,window,seed,variant,sc", CASES)
def test_backward_repeats_bytes(B, H, Hkv, S, D, window, seed, variant, sc):
    import torch

    from open_transformers_amd import _lib

    print(f"case B={B} H={H} Hkv={Hkv} S={S} D={D} window={window} seeds {seed},{seed + 100} variant {variant} "
          f"score cache {sc}", flush=True)
    dev = torch.device("cuda:0")
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    sets = [_inputs(dev, B, H, Hkv, S, D, window, s, variant, sc) for s in (seed, seed + 100)]
    nbytes = int(lib.otx_attn_bwd_workspace_bytes(B, H, Hkv, S, D, window))
    ws = torch.empty(nbytes // 4 + 64, dtype=torch.float32, device=dev)
    base = ws.data_ptr()
    aligned = (base + 255) & ~255
    q0 = sets[0][0]
    dq, dk, dv = torch.empty_like(q0["q"]), torch.empty_like(q0["k"]), torch.empty_like(q0["v"])
    for rep in range(REPS):
        t, o, lse, cache, refs = sets[rep & 1]
        if rep % 4 >= 2:
            for x in (ws, dq, dk, dv):
                x.fill_(float("nan"))
        ptrs = (t["q"].data_ptr(), t["k"].data_ptr(), t["v"].data_ptr(), o.data_ptr(), lse.data_ptr(),
                t["do"].data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr())
        if cache is None:
            rc = lib.otx_attn_bwd_ex(*ptrs, B, H, Hkv, S, D, window, _lib.DTYPE_BF16, aligned, nbytes, variant, stream)
        else:
            rc = lib.otx_attn_bwd_sc(*ptrs, cache.data_ptr(), cache.numel() * 4, B, H, Hkv, S, D, window,
                                     _lib.DTYPE_BF16, aligned, nbytes, variant, 7, stream)
        _lib.check(rc, "otx_attn_bwd")
        for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
            ne = got.view(torch.int16) != refs[name].view(torch.int16)
            if bool(ne.any()):
                rows = ne.any(dim=-1).nonzero().cpu().numpy().tolist()
                raise AssertionError(f"rep {rep}: {name} has {int(ne.sum())} differing elements in "
                                     f"{len(rows)} rows (b, h, s), first {rows[:3]}, last {rows[-1]}")
