"""The benchmark's command line on the CPU: more than one GPU is refused with a
message and exit status 2 before anything touches a device, and the HBM
traffic it reports for the dominant kernel is read from the committed
rocprofv3 summary."""

from __future__ import annotations

import importlib.util
import pathlib
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _bench_module():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused():
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         cwd=ROOT, timeout=120)
    assert res.returncode == 2
    assert "--gpus 2 is not supported" in res.stderr
    assert res.stdout == ""


def test_traffic_comes_from_the_committed_profile():
    bench = _bench_module()
    for kernel in ("attn_fwd_bf16_kernel", "attn_dkdv_bf16_kernel", "attn_dq_kernel"):
        t = bench.committed_traffic(kernel)
        assert isinstance(t, int) and t > 0, kernel
    # the dominant kernel's traffic is within a few tenths of its algorithmic bytes (1.29e9 at config 2)
    assert 1.0e9 < bench.committed_traffic("attn_dkdv_bf16_kernel") < 2.0e9
    assert bench.committed_traffic("no_such_kernel") is None
