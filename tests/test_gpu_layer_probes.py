"""The decoder-layer and int8-PV closed-form probes (tests/layer_probes.py) on
the GPU, through the C ABI.

RMSNorm forward / backward and SiLU forward / backward run with bf16 and with
binary32 data (the binary32 outputs show the deviations that bf16 rounds
away); the int8-PV forward runs at D 64 and 128 in launch variants 0 and 2,
with and without the score cache.  The probed elements must hold the
contract's hand-derived bits, and every output byte must equal the oracle's.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import fwd_probes as fp
import layer_probes as lp
from attn_util import assert_bits_equal
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _gpu(a, bf16):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16 if bf16 else torch.float32).to(DEV)


def _host(t):
    return t.detach().float().cpu().numpy()


def _call(fn, *args):
    from open_transformers_amd import _lib

    _lib.check(getattr(_lib.load(), fn)(*args, torch.cuda.current_stream().cuda_stream), fn)
    torch.cuda.synchronize()


def _dt(bf16):
    from open_transformers_amd import _lib

    return _lib.DTYPE_BF16 if bf16 else _lib.DTYPE_F32


@pytest.mark.parametrize("bf16", [True, False], ids=["bf16", "binary32"])
def test_rmsnorm_forward_probes(bf16):
    for name, p in lp.rms_fwd_probes():
        print(f"rmsnorm forward probe {name} {'bf16' if bf16 else 'binary32'}", flush=True)
        rows, D = p["x"].shape
        x, w = _gpu(p["x"], bf16), _gpu(p["w"], bf16)
        y = torch.empty_like(x)
        rstd = torch.empty(rows, dtype=torch.float32, device=DEV)
        _call("otx_rmsnorm_fwd", x.data_ptr(), w.data_ptr(), y.data_ptr(), rstd.data_ptr(), rows, D, float(lp.EPS),
              _dt(bf16))
        gy, grstd = _host(y), _host(rstd)
        lp.check_rms_fwd(name, p, gy, grstd, bf16)
        ry, rrstd = orc.rmsnorm_fwd(p["x"], p["w"], float(lp.EPS), out_bf16=bf16)
        assert_bits_equal(gy, ry, f"{name}: y")
        assert_bits_equal(grstd, rrstd, f"{name}: rstd")


@pytest.mark.parametrize("bf16", [True, False], ids=["bf16", "binary32"])
def test_rmsnorm_backward_probes(bf16):
    from open_transformers_amd import _lib

    for name, p in lp.rms_bwd_probes():
        print(f"rmsnorm backward probe {name} {'bf16' if bf16 else 'binary32'}", flush=True)
        rows, D = p["x"].shape
        x, w, dy = _gpu(p["x"], bf16), _gpu(p["w"], bf16), _gpu(p["dy"], bf16)
        rstd = torch.from_numpy(np.ascontiguousarray(p["rstd"], np.float32)).to(DEV)
        dx = torch.empty_like(x)
        dw = torch.empty(D, dtype=torch.float32, device=DEV)
        nbytes = int(_lib.load().otx_rmsnorm_bwd_workspace_bytes(rows, D))
        ws = torch.empty(max(nbytes, 4), dtype=torch.uint8, device=DEV)
        _call("otx_rmsnorm_bwd", x.data_ptr(), w.data_ptr(), rstd.data_ptr(), dy.data_ptr(), dx.data_ptr(),
              dw.data_ptr(), rows, D, _dt(bf16), ws.data_ptr(), nbytes)
        gdx, gdw = _host(dx), _host(dw)
        lp.check_rms_bwd(name, p, gdx, gdw, bf16)
        rdx, rdw = orc.rmsnorm_bwd(p["x"], p["w"], p["rstd"], p["dy"], out_bf16=bf16)
        assert_bits_equal(gdx, rdx, f"{name}: dx")
        assert_bits_equal(gdw, rdw, f"{name}: dw")


@pytest.mark.parametrize("bf16", [True, False], ids=["bf16", "binary32"])
def test_silu_probes(bf16):
    p = lp.silu_fwd()
    x = _gpu(p["x"], bf16)
    y = torch.empty_like(x)
    _call("otx_silu_fwd", x.data_ptr(), y.data_ptr(), x.numel(), _dt(bf16))
    lp.check_silu("silu_fwd", p, _host(y), bf16, "y")
    assert_bits_equal(_host(y), orc.silu_fwd(p["x"], out_bf16=bf16), "silu_fwd")
    p = lp.silu_bwd()
    x, dy = _gpu(p["x"], bf16), _gpu(p["dy"], bf16)
    dx = torch.empty_like(x)
    _call("otx_silu_bwd", x.data_ptr(), dy.data_ptr(), dx.data_ptr(), x.numel(), _dt(bf16))
    lp.check_silu("silu_bwd", p, _host(dx), bf16, "dx")
    assert_bits_equal(_host(dx), orc.silu_bwd(p["x"], p["dy"], out_bf16=bf16), "silu_bwd")


@pytest.mark.parametrize("D", [64, 128])
def test_int8pv_probes(D):
    from open_transformers_amd.nn import flash_attention as fa

    for name, p in lp.int8pv_probes(D):
        ro, rlse = orc.attn_fwd_int8pv(p["q"], p["k"], p["v"], window=p["_window"], out_bf16=True)
        q, k, v = (_gpu(p[n], True) for n in ("q", "k", "v"))
        for variant in (0, 2):
            for sc in (False, True):
                print(f"int8-PV probe {name} D={D} variant {variant} score cache {sc}", flush=True)
                f = fa.int8pv_flash_attention_forward_sc if sc else fa.int8pv_flash_attention_forward
                out = f(q, k, v, window=p["_window"], variant=variant)
                torch.cuda.synchronize()
                got = {"o": _host(out[0]), "lse": _host(out[1])}
                fp.check_row(got, p, True, name)
                assert_bits_equal(got["o"], ro, f"{name}: O (variant {variant}, cache {sc})")
                assert_bits_equal(got["lse"], rlse, f"{name}: LSE (variant {variant}, cache {sc})")
