"""CPU checks of the drop-in boundary: the C-ABI library loads and exports
every function include/otx_attn.h declares, argument validation fails with a
clear error before anything reaches the GPU, and the Python operator and the
device/backend guards behave like the reference's
(src/pretrain/cli/audit_replay.py:1114-1141,1494-1511;
tests/test_audit_device_guard.py, tests/test_audit_kit_provenance.py).
No test here launches a kernel."""

from __future__ import annotations

import ctypes
import json
import pathlib
import re

import pytest
import torch

from open_transformers_amd import _lib, backend
from open_transformers_amd.nn import flash_attention as fa

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _declared_functions() -> list[str]:
    names = []
    for hdr in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", hdr.read_text(), flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(otx_[a-z0-9_]+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_function():
    lib = ctypes.CDLL(str(_lib.lib_path()))
    declared = _declared_functions()
    assert "otx_attn_fwd" in declared and "otx_attn_bwd" in declared
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
    # and the binding covers exactly what the header declares
    assert sorted(_lib.EXPORTED) == declared


def test_build_info_names_rocm_backend():
    info = json.loads(_lib.load().otx_build_info().decode())
    assert info["backends"] == ["rocm"]
    assert info["arch"] == "gfx950"
    assert info["atomics"] is False
    full = backend.build_info()
    assert "rocm" in full["backends"] and full["rocm_arch_list"] == "gfx950"


def _git(*args):
    import subprocess

    root = pathlib.Path(__file__).resolve().parents[1]
    res = subprocess.run(["git", "-C", str(root), *args], capture_output=True, text=True)
    if res.returncode != 0:
        pytest.skip("not a git checkout")
    return res.stdout.strip()


def test_build_info_reports_the_stamp_of_the_loaded_library():
    # backend.build_info() must report what the library carries, not the tree
    info = json.loads(_lib.load().otx_build_info().decode())
    full = backend.build_info()
    for key in ("commit", "dirty", "sources_blake2b"):
        assert full[key] == info[key]
    assert re.fullmatch(r"[0-9a-f]{12}|unknown", info["commit"])
    assert info["dirty"] in (True, False, None)
    # the loaded library was built from the sources of this tree
    from open_transformers_amd import build

    assert info["sources_blake2b"] == build.sources_digest()


def test_rebuilt_library_is_stamped_with_head(tmp_path):
    # Relink the library from the built objects with a fresh stamp (no kernel
    # recompilation) and read the stamp back from the new file.
    from open_transformers_amd import build

    head = _git("rev-parse", "--short=12", "HEAD")
    dirty = bool(_git("status", "--porcelain", "--", *build.STAMP_PATHS))
    if not all((build.OBJ_DIR / (pathlib.Path(s).stem + ".o")).exists() for s in build.SOURCES):
        pytest.skip("objects not built")
    out = build.link(tmp_path / "libotx_stamp_probe.so")
    lib = ctypes.CDLL(str(out))
    lib.otx_build_info.restype = ctypes.c_char_p
    info = json.loads(lib.otx_build_info().decode())
    assert info["commit"] == head
    assert info["dirty"] is dirty
    assert info["sources_blake2b"] == build.sources_digest()
    # an explicit stamp is carried verbatim (a build outside a checkout says "unknown")
    out2 = build.link(tmp_path / "libotx_stamp_probe2.so", stamp={"commit": "unknown", "dirty": None})
    lib2 = ctypes.CDLL(str(out2))
    lib2.otx_build_info.restype = ctypes.c_char_p
    info2 = json.loads(lib2.otx_build_info().decode())
    assert info2["commit"] == "unknown" and info2["dirty"] is None


def test_shape_errors_are_reported_without_a_gpu():
    lib = _lib.load()
    # S % 32 != 0 is rejected by the argument check, before any HIP call
    rc = lib.otx_attn_fwd(16, 16, 16, 16, 16, 1, 1, 1, 48, 64, 0, 1, None)
    assert rc == _lib.OTX_EINVAL
    assert b"multiple of 32" in lib.otx_last_error()
    rc = lib.otx_attn_fwd(16, 16, 16, 16, 16, 1, 2, 1, 64, 96, 0, 1, None)
    assert rc == _lib.OTX_EINVAL and b"head_dim" in lib.otx_last_error()
    rc = lib.otx_attn_fwd(16, 16, 16, 16, 16, 1, 3, 2, 64, 64, 0, 1, None)
    assert rc == _lib.OTX_EINVAL and b"multiple of Hkv" in lib.otx_last_error()
    rc = lib.otx_attn_fwd(16, 16, 16, 16, 16, 1, 2, 2, 64, 64, 40, 1, None)
    assert rc == _lib.OTX_EINVAL and b"window" in lib.otx_last_error()
    rc = lib.otx_attn_fwd(17, 16, 16, 16, 16, 1, 2, 2, 64, 64, 0, 1, None)
    assert rc == _lib.OTX_EINVAL and b"aligned" in lib.otx_last_error()
    rc = lib.otx_attn_bwd(16, 16, 16, 16, 16, 16, 16, 16, 16, 1, 2, 2, 64, 64, 0, 1, 256, 16, None)
    assert rc == _lib.OTX_EINVAL and b"workspace too small" in lib.otx_last_error()
    with pytest.raises(ValueError, match="multiple of 32"):
        _lib.check(lib.otx_attn_fwd(16, 16, 16, 16, 16, 1, 1, 1, 48, 64, 0, 1, None), "fwd")


def test_layer_glue_argument_errors_without_a_gpu():
    lib = _lib.load()
    rc = lib.otx_swiglu_fwd(16, 16, 4, 12, 1, None)
    assert rc == _lib.OTX_EINVAL and b"multiple of 8" in lib.otx_last_error()
    rc = lib.otx_swiglu_fwd(17, 16, 4, 16, 1, None)
    assert rc == _lib.OTX_EINVAL and b"unaligned" in lib.otx_last_error()
    rc = lib.otx_swiglu_bwd(16, 32, 16, 4, 16, 1, None)
    assert rc == _lib.OTX_EINVAL and b"alias" in lib.otx_last_error()
    rc = lib.otx_swiglu_fwd(16, 16, 4, 16, 7, None)
    assert rc == _lib.OTX_EINVAL and b"dtype" in lib.otx_last_error()
    rc = lib.otx_rope_heads_fwd(16, 16, 16, 32, 1, 4, 2, 12, 1, None)
    assert rc == _lib.OTX_EINVAL and b"multiple of 8" in lib.otx_last_error()
    rc = lib.otx_rope_heads_bwd(16, 16, 16, 16, 1, 4, 2, 16, 1, None)
    assert rc == _lib.OTX_EINVAL and b"alias" in lib.otx_last_error()
    rc = lib.otx_rope_heads_fwd(16, 16, 16, 32, 0, 4, 2, 16, 1, None)
    assert rc == _lib.OTX_EINVAL and b"positive" in lib.otx_last_error()
    rc = lib.otx_rope_heads_fwd(16, 20, 16, 32, 1, 4, 2, 16, 1, None)
    assert rc == _lib.OTX_EINVAL and b"unaligned" in lib.otx_last_error()
    rc = lib.otx_swap_heads(16, 16, 1, 4, 2, 16, 1, None)
    assert rc == _lib.OTX_EINVAL and b"alias" in lib.otx_last_error()
    rc = lib.otx_swap_heads(16, 32, 1, 4, 2, 20, 1, None)
    assert rc == _lib.OTX_EINVAL and b"multiple of 8" in lib.otx_last_error()


def test_layer_glue_refuses_cpu_tensors_and_bad_shapes():
    from open_transformers_amd.nn import functional as F

    x = torch.zeros(1, 4, 2, 16, dtype=torch.bfloat16)
    cs = torch.zeros(4, 8)
    for call in (lambda: F.swiglu(torch.zeros(4, 32, dtype=torch.bfloat16)), lambda: F.rope_heads(x, cs, cs),
                 lambda: F.heads(x), lambda: F.merge_heads(x)):
        with pytest.raises(RuntimeError, match="ROCm"):
            call()


def test_workspace_size():
    lib = _lib.load()
    # 4*16*2048 Dsum floats + 64 heads * 2080 processed 32x32 tiles of fp32 dS
    want = 4 * 16 * 2048 * 4 + 64 * (64 * 65 // 2) * 32 * 32 * 4
    assert lib.otx_attn_bwd_workspace_bytes(4, 16, 16, 2048, 128, 0) == want
    assert lib.otx_attn_bwd_workspace_bytes(1, 1, 1, 48, 128, 0) == 0


def test_score_cache_size_and_validation():
    lib = _lib.load()
    # one fp32 32x32 tile per processed (query block, key block) pair
    assert lib.otx_attn_score_cache_bytes(4, 16, 2048, 0) == 64 * (64 * 65 // 2) * 4096
    # window 512 = 16 key blocks: query block i sees min(i, 16) + 1 key blocks
    assert lib.otx_attn_score_cache_bytes(1, 1, 2048, 512) == sum(min(i, 16) + 1 for i in range(64)) * 4096
    assert lib.otx_attn_score_cache_bytes(1, 1, 48, 0) == 0
    need = lib.otx_attn_score_cache_bytes(1, 2, 64, 0)
    # binary32 inputs: the cache is a bf16-path feature
    rc = lib.otx_attn_fwd_sc(16, 16, 16, 16, 16, 16, need, 1, 2, 2, 64, 64, 0, _lib.DTYPE_F32, 0, None)
    assert rc == _lib.OTX_EINVAL and b"bf16" in lib.otx_last_error()
    rc = lib.otx_attn_fwd_sc(16, 16, 16, 16, 16, None, need, 1, 2, 2, 64, 64, 0, _lib.DTYPE_BF16, 0, None)
    assert rc == _lib.OTX_EINVAL and b"null score cache" in lib.otx_last_error()
    rc = lib.otx_attn_fwd_sc(16, 16, 16, 16, 16, 16, need - 4, 1, 2, 2, 64, 64, 0, _lib.DTYPE_BF16, 0, None)
    assert rc == _lib.OTX_EINVAL and b"score cache too small" in lib.otx_last_error()
    rc = lib.otx_attn_fwd_int8pv_sc(16, 16, 16, 16, 16, 24, need, 1, 2, 2, 64, 64, 0, _lib.DTYPE_BF16, 256, 1 << 20, 0,
                                    None)
    assert rc == _lib.OTX_EINVAL and b"aligned" in lib.otx_last_error()
    rc = lib.otx_attn_bwd_sc(*([16] * 10), need, 1, 2, 2, 64, 64, 0, _lib.DTYPE_BF16, 256, 1 << 20, 0, 8, None)
    assert rc == _lib.OTX_EINVAL and b"stage mask" in lib.otx_last_error()


def test_operator_refuses_cpu_tensors_and_dropout():
    q = torch.zeros(1, 2, 64, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm"):
        fa.causal_flash_attention(q, q, q)
    with pytest.raises(ValueError, match="dropout"):
        fa.causal_flash_attention(q, q, q, dropout=0.1)
    with pytest.raises(RuntimeError, match="ROCm"):
        fa.int8pv_causal_flash_attention(q, q, q)


def test_int8pv_workspace_and_validation():
    lib = _lib.load()
    # int8 V (B*Hkv*S*D bytes, 256-aligned) + one binary32 step per (key block, column)
    assert lib.otx_attn_fwd_int8pv_workspace_bytes(4, 16, 4, 2048, 128) == 4 * 4 * 2048 * 128 + 4 * 4 * 64 * 128 * 4
    assert lib.otx_attn_fwd_int8pv_workspace_bytes(1, 1, 1, 48, 128) == 0
    p = ctypes.c_void_p(256)
    # float32 inputs are refused before anything is launched
    rc = lib.otx_attn_fwd_int8pv(p, p, p, p, p, 1, 1, 1, 64, 64, 0, _lib.DTYPE_F32, p, 1 << 20, None)
    assert rc == _lib.OTX_EINVAL and b"bf16" in lib.otx_last_error()
    rc = lib.otx_attn_fwd_int8pv(p, p, p, p, p, 1, 1, 1, 64, 64, 0, _lib.DTYPE_BF16, p, 16, None)
    assert rc == _lib.OTX_EINVAL and b"workspace too small" in lib.otx_last_error()


def test_backend_guard_accepts_rocm_only_with_hip_torch():
    cuda = torch.device("cuda")
    backend.require_backend(cuda, {"backends": ["rocm"]}, hip_version="7.0")
    backend.require_backend(cuda, {"backends": ["cuda", "cpu"]}, hip_version=None)
    with pytest.raises(RuntimeError, match="no CUDA/ROCm backend"):
        backend.require_backend(cuda, {"backends": ["rocm"], "commit": "x"}, hip_version=None)
    with pytest.raises(RuntimeError, match="no CUDA/ROCm backend"):
        backend.require_backend(cuda, {"backends": ["cpu"]}, hip_version="7.0")
    backend.require_backend(torch.device("cpu"), {"backends": []})
    with pytest.raises(RuntimeError, match="Metal"):
        backend.require_backend(torch.device("mps"), {"backends": ["rocm"]})


def test_device_guard(monkeypatch):
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    with pytest.raises(RuntimeError, match="not available"):
        backend.require_device_available("cuda")
    assert backend.require_device_available("cpu").type == "cpu"


def test_score_cache_only_when_a_backward_can_run():
    # the O(S^2) cache is kept only for bf16 inputs with grad mode on and some input requiring grad
    q = torch.zeros(1, 2, 32, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 1, 32, 64, dtype=torch.bfloat16)
    v = torch.zeros(1, 1, 32, 64, dtype=torch.bfloat16)
    prev = fa.set_score_cache(True)
    try:
        assert not fa._use_score_cache(q, k, v)  # nothing requires grad
        kg = k.clone().requires_grad_()
        assert fa._use_score_cache(q, kg, v)
        with torch.no_grad():
            assert not fa._use_score_cache(q, kg, v)
        with torch.inference_mode():
            assert not fa._use_score_cache(q, k, v)
        assert not fa._use_score_cache(q.float(), kg.detach().float().requires_grad_(), v.float())  # bf16 only
        fa.set_score_cache(False)
        assert not fa._use_score_cache(q, kg, v)
    finally:
        fa.set_score_cache(prev)


def test_score_cache_skipped_in_the_first_checkpointed_forward():
    """Under non-reentrant checkpointing (checkpoint_wrapper's mode) the first
    forward's saved tensors are dropped, so it writes no score cache
    (placeholder); the recompute in the backward keeps it.  With the recording
    context_fn the first forward's results are kept and replayed, so it keeps
    the cache.  Reentrant checkpointing runs its first forward under no_grad."""
    from torch.utils.checkpoint import checkpoint

    k = torch.zeros(1, 1, 32, 64, dtype=torch.bfloat16)
    v = torch.zeros(1, 1, 32, 64, dtype=torch.bfloat16)
    q = torch.ones(1, 2, 32, 64, dtype=torch.bfloat16, requires_grad=True)
    modes = []

    def block(x):
        modes.append(fa._score_cache_mode(x, k, v))
        return x * x  # saves x, so the backward unpacks it and the block is recomputed

    prev = fa.set_score_cache(True)
    try:
        assert not fa._checkpoint_discards_saved_tensors()
        checkpoint(block, q, use_reentrant=False).float().sum().backward()
        assert modes == [fa._SC_PLACEHOLDER, fa._SC_KEEP]
        modes.clear()
        checkpoint(block, q, use_reentrant=False, context_fn=fa.attention_checkpoint_contexts).float().sum().backward()
        assert modes == [fa._SC_KEEP, fa._SC_KEEP]
        modes.clear()
        checkpoint(block, q, use_reentrant=True).float().sum().backward()
        assert modes == [fa._SC_NONE, fa._SC_KEEP]
        modes.clear()
        block(q).float().sum().backward()
        assert modes == [fa._SC_KEEP]
    finally:
        fa.set_score_cache(prev)
    # the placeholder is never handed to the backward kernels as a cache
    ph = torch.empty(1, dtype=torch.float32).expand(4096)
    assert fa._saved_score_cache([ph]) is None and fa._saved_score_cache([]) is None
    real = torch.empty(4096, dtype=torch.float32)
    assert fa._saved_score_cache([real]) is real


def test_noalloc_int8pv_refuses_shapes_beyond_its_scratch():
    # checked before any HIP call: B16 H16 Hkv16 S4096 D128 needs 128 MiB of quantized V
    lib = _lib.load()
    rc = lib.otx_attn_fwd_int8pv_noalloc(16, 16, 16, 16, 16, 16, 16, 16, 4096, 128, 0, _lib.DTYPE_BF16, 0, None)
    assert rc == _lib.OTX_EINVAL
    assert b"too large for the allocation-free" in lib.otx_last_error()
    need = lib.otx_attn_fwd_int8pv_workspace_bytes(4, 16, 4, 4096, 128)
    assert 0 < need <= _lib.NOALLOC_SCRATCH_BYTES  # the OPEN-1B training shape fits
    rc = lib.otx_attn_fwd_int8pv_noalloc(16, 16, 16, 16, 16, 1, 2, 2, 64, 64, 0, _lib.DTYPE_F32, 0, None)
    assert rc == _lib.OTX_EINVAL and b"bf16" in lib.otx_last_error()
