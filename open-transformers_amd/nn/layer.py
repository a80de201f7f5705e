"""Pre-norm decoder layer around the attention.

Mirrors the reference's block, src/pretrain/model/llama3.py:66-74
(``x = x + attn(norm1(x)); x = x + ffn(norm2(x))``), with the attention module
of src/pretrain/model/modules/attention_repop.py:120-156 (Q/K/V projections,
RoPE, ``[B, H, T, D]`` layout, causal flash attention, output projection) and
the SwiGLU of src/pretrain/model/modules/ffn_repop.py:39-54 (fused gate/up
projection, ``silu(gate) * up``, down projection).  The residual adds are torch
additions as in the reference; every other byte-sensitive step comes from
``ops``:

    ops.linear(x, w), ops.rms_norm(x, w, eps),
    ops.rope_heads(x, cos, sin)   apply_rope (rope.py:103-125) + transpose(1, 2).contiguous()
    ops.heads(x), ops.merge_heads(o)   the other layout changes (attention_repop.py:150,155)
    ops.swiglu(gu)                silu(gate) * up over gate, up = gu.chunk(2, -1)
    ops.attention(q, k, v, window), ops.attention_int8pv(q, k, v, window)
    (and, for the whole model, ops.embedding(ids, w), ops.loss(logits, labels, coeff))

The default ``ops`` are this package's ROCm kernels, which give the bytes of
the reference's torch compositions in one pass each.  A test can pass a CPU
implementation with the same interface (there, the reference's compositions
themselves) and compare bytes.
"""

from __future__ import annotations

import types

import torch
import torch.nn as nn

from .. import rope as _rope
from . import embedding as _embedding
from . import flash_attention, functional
from . import loss as _loss

__all__ = ["DecoderLayer", "rope_tables", "ROCM_OPS"]


def _attention(q, k, v, window):
    return flash_attention.causal_flash_attention(q, k, v, dropout=0.0, window=window)


def _attention_int8pv(q, k, v, window):
    return flash_attention.int8pv_causal_flash_attention(q, k, v, window=window)


ROCM_OPS = types.SimpleNamespace(
    linear=functional.linear,
    rms_norm=functional.rms_norm,
    silu=functional.silu,
    swiglu=functional.swiglu,
    rope_heads=functional.rope_heads,
    heads=functional.heads,
    merge_heads=functional.merge_heads,
    attention=_attention,
    attention_int8pv=_attention_int8pv,
    embedding=_embedding.embedding,
    loss=lambda logits, labels, coeff: _loss.fused_ce_z_loss(logits, labels, coeff),
)


def rope_tables(seq_len: int, head_dim: int, theta: float) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin tables [seq_len, head_dim/2] in binary32 (rope.py:21-31): torch
    binary32 inv_freq and angles, correctly rounded cos/sin (the package's rope
    module, shared with the input generator)."""
    cos, sin = _rope.rope_tables(seq_len, head_dim, theta)
    return torch.from_numpy(cos.copy()), torch.from_numpy(sin.copy())


class DecoderLayer(nn.Module):
    """One pre-norm block: RMSNorm -> QKV -> (q/k RMSNorm) -> RoPE -> causal
    attention -> out proj -> residual -> RMSNorm -> SwiGLU -> residual.
    Parameters are bf16 (the compute copies FSDP2 hands the reference's block).
    ``qk_norm`` adds the per-head RMSNorm of q and k over head_dim
    (attention_repop.py:109-140; ``qk_norm_gain=False`` is the gain-free form),
    ``int8_pv`` routes the attention to the int8-PV forward (:51-52)."""

    def __init__(self, d_model: int, n_heads: int, n_kv_heads: int, head_dim: int, d_ff: int,
                 eps: float = 1e-5, window: int = 0, ops=None, dtype=torch.bfloat16, device=None,
                 qk_norm: bool = False, qk_norm_gain: bool = True, int8_pv: bool = False):
        super().__init__()
        self.d_model, self.n_heads, self.n_kv_heads, self.head_dim = d_model, n_heads, n_kv_heads, head_dim
        self.eps, self.window = eps, window
        self.qk_norm, self.int8_pv = qk_norm, int8_pv
        self.ops = ops or ROCM_OPS
        kw = dict(dtype=dtype, device=device)
        self.norm1 = nn.Parameter(torch.ones(d_model, **kw))
        self.wq = nn.Parameter(torch.empty(n_heads * head_dim, d_model, **kw))
        self.wk = nn.Parameter(torch.empty(n_kv_heads * head_dim, d_model, **kw))
        self.wv = nn.Parameter(torch.empty(n_kv_heads * head_dim, d_model, **kw))
        self.wo = nn.Parameter(torch.empty(d_model, n_heads * head_dim, **kw))
        self.norm2 = nn.Parameter(torch.ones(d_model, **kw))
        self.w_gate_up = nn.Parameter(torch.empty(2 * d_ff, d_model, **kw))
        self.w_down = nn.Parameter(torch.empty(d_model, d_ff, **kw))
        if qk_norm:
            if qk_norm_gain:
                self.q_norm = nn.Parameter(torch.ones(head_dim, **kw))
                self.k_norm = nn.Parameter(torch.ones(head_dim, **kw))
            else:  # unit gain: RN(RN(x * rstd) * 1) is RN(x * rstd)
                self.register_buffer("q_norm", torch.ones(head_dim, **kw), persistent=False)
                self.register_buffer("k_norm", torch.ones(head_dim, **kw), persistent=False)

    def attn(self, h: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        B, T, _ = h.shape
        q = self.ops.linear(h, self.wq).view(B, T, self.n_heads, self.head_dim)
        k = self.ops.linear(h, self.wk).view(B, T, self.n_kv_heads, self.head_dim)
        v = self.ops.linear(h, self.wv).view(B, T, self.n_kv_heads, self.head_dim)
        if self.qk_norm:
            D = self.head_dim
            q = self.ops.rms_norm(q.reshape(B * T * self.n_heads, D), self.q_norm, self.eps).reshape(B, T, -1, D)
            k = self.ops.rms_norm(k.reshape(B * T * self.n_kv_heads, D), self.k_norm, self.eps).reshape(B, T, -1, D)
        q = self.ops.rope_heads(q, cos, sin)  # [B, H, T, D]
        k = self.ops.rope_heads(k, cos, sin)
        v = self.ops.heads(v)
        attend = self.ops.attention_int8pv if self.int8_pv else self.ops.attention
        out = self.ops.merge_heads(attend(q, k, v, self.window))  # [B, T, H * D]
        return self.ops.linear(out, self.wo)

    def ffn(self, h: torch.Tensor) -> torch.Tensor:
        return self.ops.linear(self.ops.swiglu(self.ops.linear(h, self.w_gate_up)), self.w_down)

    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(self.ops.rms_norm(x, self.norm1, self.eps), cos, sin)
        x = x + self.ffn(self.ops.rms_norm(x, self.norm2, self.eps))
        return x
