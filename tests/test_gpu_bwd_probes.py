"""The backward's closed-form probes (tests/bwd_probes.py) on the GPU.

Each probe runs through the C ABI with bf16 and binary32 inputs, in launch
variants 0 and 2 (for bf16 these take the two dK/dV kernel forms), with and
without the score cache (bf16).  The closed-form bits must hold, dS_00 read
back from the backward workspace must equal the contract's, and every output
byte must equal the oracle's.
"""

from __future__ import annotations

import numpy as np
import pytest

import bwd_probes as bp
from attn_util import assert_bits_equal
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _gpu_bwd(p, bf16, variant, score_cache):
    import torch

    from open_transformers_amd import _lib
    from open_transformers_amd.nn.flash_attention import flash_attention_forward_sc

    dev = torch.device("cuda:0")
    dt = torch.bfloat16 if bf16 else torch.float32
    t = {n: torch.from_numpy(np.ascontiguousarray(p[n])).to(dt).to(dev) for n in ("q", "k", "v", "o", "do")}
    lse = torch.from_numpy(np.ascontiguousarray(p["lse"])).to(dev)
    B, H, S, D = t["q"].shape
    Hkv = t["k"].shape[1]
    lib = _lib.load()
    sc = None
    if score_cache:
        _, _, sc = flash_attention_forward_sc(t["q"], t["k"], t["v"], window=0, variant=variant)
    nbytes = int(lib.otx_attn_bwd_workspace_bytes(B, H, Hkv, S, D, 0))
    ws = torch.zeros(nbytes // 4 + 64, dtype=torch.float32, device=dev)
    base = ws.data_ptr()
    off = ((base + 255) & ~255) - base
    dq, dk, dv = torch.empty_like(t["q"]), torch.empty_like(t["k"]), torch.empty_like(t["v"])
    ptrs = (t["q"].data_ptr(), t["k"].data_ptr(), t["v"].data_ptr(), t["o"].data_ptr(), lse.data_ptr(),
            t["do"].data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr())
    stream = torch.cuda.current_stream().cuda_stream
    dtc = _lib.DTYPE_BF16 if bf16 else _lib.DTYPE_F32
    if sc is None:
        rc = lib.otx_attn_bwd_ex(*ptrs, B, H, Hkv, S, D, 0, dtc, base + off, nbytes, variant, stream)
    else:
        rc = lib.otx_attn_bwd_sc(*ptrs, sc.data_ptr(), sc.numel() * 4, B, H, Hkv, S, D, 0, dtc, base + off, nbytes,
                                 variant, 7, stream)
    _lib.check(rc, "otx_attn_bwd")
    torch.cuda.synchronize()
    dsum_floats = ((B * H * S * 4 + 255) // 256 * 256) // 4
    w = ws.cpu().numpy()[off // 4:]
    tile0 = w[dsum_floats:dsum_floats + 1024].reshape(1, 32, 32)
    return {"dq": dq.float().cpu().numpy(), "dk": dk.float().cpu().numpy(), "dv": dv.float().cpu().numpy(),
            "ds": tile0}


@pytest.mark.parametrize("bf16", [True, False], ids=["bf16", "binary32"])
def test_backward_probes_on_gpu(bf16):
    for name, p, check in bp.all_probes(bf16):
        ref = dict(zip(("dq", "dk", "dv"),
                       orc.attn_bwd(p["q"], p["k"], p["v"], p["o"], p["lse"], p["do"], window=0, out_bf16=bf16)))
        for variant in (0, 2):
            for sc in ((False, True) if bf16 else (False,)):
                print(f"probe {name} {'bf16' if bf16 else 'binary32'} variant {variant} score cache {sc}", flush=True)
                got = _gpu_bwd(p, bf16, variant, sc)
                check(got)
                for n in ("dq", "dk", "dv"):
                    assert_bits_equal(got[n], ref[n], f"probe {name} {n} (variant {variant}, cache {sc})")


@pytest.mark.parametrize("bf16", [True, False], ids=["bf16", "binary32"])
def test_backward_with_lse_below_the_scores(bf16):
    """A caller-supplied LSE below a row's scores makes exp arguments positive.
    The dK/dV kernels' checked exp then evaluates the whole wave's array with
    otx_expf instead of the table-driven path, and every output byte must still
    equal the oracle's for the same LSE.  Every third query row has its LSE
    lowered by 2 (arguments up to about +2), the others keep the forward's; GQA
    (H 4, Hkv 2), both dK/dV forms (variants 0 and 2), score cache on and off."""
    rng = np.random.default_rng(7)
    B, H, Hkv, S, D = 1, 4, 2, 128, 128

    def bf16_exact(shape):
        x = rng.standard_normal(shape).astype(np.float32)
        return (x.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)

    p = {"q": bf16_exact((B, H, S, D)), "k": bf16_exact((B, Hkv, S, D)), "v": bf16_exact((B, Hkv, S, D)),
         "do": bf16_exact((B, H, S, D))}
    o, lse = orc.attn_fwd(p["q"], p["k"], p["v"], window=0, out_bf16=bf16)
    p["o"] = np.ascontiguousarray(o, dtype=np.float32)
    lse = np.array(lse, dtype=np.float32)
    lse[:, :, ::3] -= np.float32(2.0)
    p["lse"] = lse
    ref = dict(zip(("dq", "dk", "dv"),
                   orc.attn_bwd(p["q"], p["k"], p["v"], p["o"], p["lse"], p["do"], window=0, out_bf16=bf16)))
    for variant in (0, 2):
        for sc in ((False, True) if bf16 else (False,)):
            print(f"lowered LSE {'bf16' if bf16 else 'binary32'} variant {variant} score cache {sc}", flush=True)
            got = _gpu_bwd(p, bf16, variant, sc)
            for n in ("dq", "dk", "dv"):
                assert_bits_equal(got[n], ref[n], f"lowered LSE {n} (variant {variant}, cache {sc})")
