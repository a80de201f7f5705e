"""ctypes binding of libotx_attn.so (declared in include/otx_attn.h).

This is the binding a repop-style Python operator uses on ROCm: plain
pointers, sizes and a hipStream_t, no torch types across the boundary.  The
library must have been built (``open-transformers_amd/build.py``); a missing
library is an error, never a silent fallback.
"""

from __future__ import annotations

import ctypes
import json
import pathlib

from .build import LIB_NAME, PKG_DIR

OTX_OK = 0
OTX_EINVAL = 1
OTX_EHIP = 2
DTYPE_F32 = 0
DTYPE_BF16 = 1
NOALLOC_SCRATCH_BYTES = 32 << 20  # OTX_NOALLOC_SCRATCH_BYTES of include/otx_attn.h

_LIB = None

_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t
_l = ctypes.c_long

_SIGNATURES = {
    "otx_attn_fwd": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "otx_attn_fwd_ex": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "otx_attn_fwd_int8pv_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "otx_attn_fwd_int8pv": (_i, [_vp] * 5 + [_i] * 7 + [_vp, _sz, _vp]),
    "otx_attn_fwd_int8pv_ex": (_i, [_vp] * 5 + [_i] * 7 + [_vp, _sz, _i, _vp]),
    "otx_attn_fwd_int8pv_noalloc": (_i, [_vp] * 5 + [_i] * 8 + [_vp]),
    "otx_attn_bwd_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i]),
    "otx_ce_zloss_fwd": (_i, [_vp, _vp, _l, _i, _i, ctypes.c_double, _vp, _vp, _vp]),
    "otx_embedding_bwd_workspace_bytes": (_sz, [_l, _i]),
    "otx_embedding_fwd": (_i, [_vp, _vp, _vp, _l, _i, _i, _i, _vp]),
    "otx_embedding_bwd": (_i, [_vp, _vp, _vp, _l, _i, _i, _i, _vp, _sz, _vp]),
    "otx_ce_zloss_bwd": (_i, [_vp, _vp, _vp, _vp, _l, _i, _i, ctypes.c_double, _vp, _vp]),
    "otx_attn_bwd": (_i, [_vp] * 9 + [_i] * 7 + [_vp, _sz, _vp]),
    "otx_attn_bwd_ex": (_i, [_vp] * 9 + [_i] * 7 + [_vp, _sz, _i, _vp]),
    "otx_attn_bwd_stages": (_i, [_vp] * 9 + [_i] * 7 + [_vp, _sz, _i, _i, _vp]),
    "otx_attn_score_cache_bytes": (_sz, [_i, _i, _i, _i]),
    "otx_attn_fwd_sc": (_i, [_vp] * 6 + [_sz] + [_i] * 8 + [_vp]),
    "otx_attn_fwd_int8pv_sc": (_i, [_vp] * 6 + [_sz] + [_i] * 7 + [_vp, _sz, _i, _vp]),
    "otx_attn_bwd_sc": (_i, [_vp] * 10 + [_sz] + [_i] * 7 + [_vp, _sz, _i, _i, _vp]),
    "otx_gemm_bf16": (_i, [_vp, _l, _l, _vp, _l, _l, _vp, _l, _i, _i, _i, _i, _vp]),
    "otx_gemm_bf16_ex": (_i, [_vp, _l, _l, _vp, _l, _l, _vp, _l, _i, _i, _i, _i, _i, _vp]),
    "otx_rmsnorm_fwd": (_i, [_vp, _vp, _vp, _vp, _l, _i, ctypes.c_float, _i, _vp]),
    "otx_rmsnorm_bwd_workspace_bytes": (_sz, [_l, _i]),
    "otx_rmsnorm_bwd": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _l, _i, _i, _vp, _sz, _vp]),
    "otx_silu_fwd": (_i, [_vp, _vp, _l, _i, _vp]),
    "otx_silu_bwd": (_i, [_vp, _vp, _vp, _l, _i, _vp]),
    "otx_swiglu_fwd": (_i, [_vp, _vp, _l, _i, _i, _vp]),
    "otx_swiglu_bwd": (_i, [_vp, _vp, _vp, _l, _i, _i, _vp]),
    "otx_rope_heads_fwd": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "otx_rope_heads_bwd": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "otx_swap_heads": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "otx_softmax_scale": (ctypes.c_float, [_i]),
    "otx_build_info": (ctypes.c_char_p, []),
    "otx_last_error": (ctypes.c_char_p, []),
    "otx_selftest_mfma": (_i, [_vp, _vp, _vp, _vp, _i, _vp]),
    "otx_selftest_mfma16": (_i, [_vp, _vp, _vp, _vp, _i, _vp]),
    "otx_selftest_math": (_i, [_i, ctypes.c_uint64, ctypes.c_uint64, _vp, _i, _vp]),
    "otx_selftest_mfma_bf16": (_i, [_i, _vp, _vp, _vp, _vp, _i, _vp]),
    "otx_selftest_mfma_i8": (_i, [_vp, _vp, _vp, _vp, _i, _vp]),
}

EXPORTED = tuple(_SIGNATURES)


def lib_path() -> pathlib.Path:
    return PKG_DIR / LIB_NAME


def load() -> ctypes.CDLL:
    """Load the library once; raises RuntimeError if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = lib_path()
    if not path.exists():
        raise RuntimeError(
            f"{path} is missing: the MI355X attention kernels are not built. "
            "Run `python -c 'import __graft_entry__ as g; g.build()'` (or "
            "open-transformers_amd/build.py) first; there is no CPU fallback."
        )
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc == OTX_OK:
        return
    msg = load().otx_last_error().decode(errors="replace")
    if rc == OTX_EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def native_build_info() -> dict:
    return json.loads(load().otx_build_info().decode())
