"""The forward's closed-form probes (tests/fwd_probes.py) on the GPU.

Each probe runs through the C ABI at D 64 and 128 with bf16 and binary32
inputs, in launch variants 0 and 2, with and without the score cache (bf16).
The probed row's LSE and O columns must equal the contract's hand-derived
bits (the deviations' bits differ, as the CPU pins show), and every O and LSE
byte must equal the oracle's.  The int8-PV forward runs the same probes: its
LSE must be the contract's (l sums the unquantized p), and its O the int8-PV
oracle's.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import fwd_probes as fp
from attn_util import assert_bits_equal
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _host(t):
    return t.detach().float().cpu().numpy()


def _gpu_fwd(p, window, bf16, variant, score_cache, int8pv=False):
    from open_transformers_amd.nn import flash_attention as fa

    dt = torch.bfloat16 if bf16 else torch.float32
    q, k, v = (torch.from_numpy(np.ascontiguousarray(p[n])).to(dt).to(DEV) for n in ("q", "k", "v"))
    if int8pv:
        f = fa.int8pv_flash_attention_forward_sc if score_cache else fa.int8pv_flash_attention_forward
    else:
        f = fa.flash_attention_forward_sc if score_cache else fa.flash_attention_forward
    out = f(q, k, v, window=window, variant=variant)
    torch.cuda.synchronize()
    return {"o": _host(out[0]), "lse": _host(out[1])}


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("bf16", [True, False], ids=["bf16", "binary32"])
def test_forward_probes_on_gpu(D, bf16):
    for name, p, window in fp.all_probes(D):
        ro, rlse = orc.attn_fwd(p["q"], p["k"], p["v"], window=window, out_bf16=bf16)
        for variant in (0, 2):
            for sc in ((False, True) if bf16 else (False,)):
                print(f"forward probe {name} D={D} {'bf16' if bf16 else 'binary32'} variant {variant} "
                      f"score cache {sc}", flush=True)
                got = _gpu_fwd(p, window, bf16, variant, sc)
                fp.check(name, got, p, bf16)
                assert_bits_equal(got["o"], ro, f"probe {name} O (variant {variant}, cache {sc})")
                assert_bits_equal(got["lse"], rlse, f"probe {name} LSE (variant {variant}, cache {sc})")


@pytest.mark.parametrize("D", [64, 128])
def test_forward_probes_int8pv_lse(D):
    for name, p, window in fp.all_probes(D):
        _, rlse = orc.attn_fwd(p["q"], p["k"], p["v"], window=window, out_bf16=True)
        ro8, rlse8 = orc.attn_fwd_int8pv(p["q"], p["k"], p["v"], window=window, out_bf16=True)
        assert_bits_equal(rlse8, rlse, f"probe {name}: oracle int8-PV LSE vs binary32 LSE")
        for variant in (0, 2):
            for sc in (False, True):
                print(f"int8-PV forward probe {name} D={D} variant {variant} score cache {sc}", flush=True)
                got = _gpu_fwd(p, window, True, variant, sc, int8pv=True)
                if name in fp.ROW_PROBES:
                    row = p["_row"]
                    assert got["lse"][0, 0, row] == p["_want"]["lse"], f"probe {name}: int8-PV LSE_{row}"
                else:
                    assert np.array_equal(np.asarray(got["lse"][0, 0], np.float32).view(np.uint32),
                                          p["_rows"]["lse"].view(np.uint32)), f"probe {name}: int8-PV LSE"
                assert_bits_equal(got["lse"], rlse, f"probe {name} int8-PV LSE (variant {variant}, cache {sc})")
                assert_bits_equal(got["o"], ro8, f"probe {name} int8-PV O (variant {variant}, cache {sc})")
