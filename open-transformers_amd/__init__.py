"""MI355X (gfx950) deterministic causal flash attention.

A drop-in ROCm backend for the attention operator of the gensyn-ai
open-transformers harness (``repop.nn.flash_attention.causal_flash_attention``,
called at src/pretrain/model/modules/attention_repop.py:53 of the reference):

    from open_transformers_amd.nn.flash_attention import causal_flash_attention
    o = causal_flash_attention(q, k, v, dropout=0.0, window=0)

The kernels are hand-written HIP for gfx950 (libotx_attn.so, C ABI in
include/otx_attn.h); outputs are bit-identical across runs, batch sizes and
launch shapes, and follow a written fixed-order arithmetic contract.
"""

from __future__ import annotations

from . import nn  # noqa: F401
from .backend import build_info, capture_contract_env, require_backend, require_device_available  # noqa: F401

__all__ = ["nn", "build_info", "require_backend", "require_device_available"]
