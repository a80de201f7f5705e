"""Pre-norm decoder layer around the attention.

Mirrors the reference's block, src/pretrain/model/llama3.py:66-74
(``x = x + attn(norm1(x)); x = x + ffn(norm2(x))``), with the attention module
of src/pretrain/model/modules/attention_repop.py:120-156 (Q/K/V projections,
RoPE, ``[B, H, T, D]`` layout, causal flash attention, output projection) and
the SwiGLU of src/pretrain/model/modules/ffn_repop.py:39-54 (fused gate/up
projection, ``silu(gate) * up``, down projection).  RoPE, the residual adds and
the SwiGLU product are the same torch elementwise operations as in the
reference (rope.py:103-125); every byte-sensitive operator comes from ``ops``:

    ops.linear(x, w), ops.rms_norm(x, w, eps), ops.silu(x),
    ops.attention(q, k, v, window)

The default ``ops`` are this package's ROCm kernels.  A test can pass a CPU
implementation with the same interface and compare bytes.
"""

from __future__ import annotations

import types

import torch
import torch.nn as nn

from . import flash_attention, functional

__all__ = ["DecoderLayer", "apply_rope", "rope_tables", "ROCM_OPS"]


def _attention(q, k, v, window):
    return flash_attention.causal_flash_attention(q, k, v, dropout=0.0, window=window)


ROCM_OPS = types.SimpleNamespace(
    linear=functional.linear, rms_norm=functional.rms_norm, silu=functional.silu, attention=_attention
)


def rope_tables(seq_len: int, head_dim: int, theta: float) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin tables [seq_len, head_dim/2] in binary32 (rope.py:21-31): inv_freq =
    1/theta^(2i/D) and freqs = pos * inv_freq in binary32, then cos/sin of each
    binary32 angle evaluated in binary64 and rounded once."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    pos = torch.arange(seq_len, dtype=torch.float32)
    freqs = torch.outer(pos, inv_freq).to(torch.float64)
    return torch.cos(freqs).to(torch.float32), torch.sin(freqs).to(torch.float32)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [B, T, H, D]; cos/sin [T, D/2] binary32 (rope.py:103-125 arithmetic)."""
    x1 = x[..., 0::2]
    x2 = x[..., 1::2]
    c = cos.unsqueeze(-2).unsqueeze(0)
    s = sin.unsqueeze(-2).unsqueeze(0)
    rx1 = x1 * c - x2 * s
    rx2 = x1 * s + x2 * c
    out = torch.empty_like(x)
    out[..., 0::2] = rx1
    out[..., 1::2] = rx2
    return out


class DecoderLayer(nn.Module):
    """One pre-norm block: RMSNorm -> QKV -> RoPE -> causal attention -> out proj
    -> residual -> RMSNorm -> SwiGLU -> residual.  Parameters are bf16 (the
    compute copies FSDP2 hands the reference's block)."""

    def __init__(self, d_model: int, n_heads: int, n_kv_heads: int, head_dim: int, d_ff: int,
                 eps: float = 1e-5, window: int = 0, ops=None, dtype=torch.bfloat16, device=None):
        super().__init__()
        self.d_model, self.n_heads, self.n_kv_heads, self.head_dim = d_model, n_heads, n_kv_heads, head_dim
        self.eps, self.window = eps, window
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

    def attn(self, h: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        B, T, _ = h.shape
        q = self.ops.linear(h, self.wq).view(B, T, self.n_heads, self.head_dim)
        k = self.ops.linear(h, self.wk).view(B, T, self.n_kv_heads, self.head_dim)
        v = self.ops.linear(h, self.wv).view(B, T, self.n_kv_heads, self.head_dim)
        q = apply_rope(q, cos, sin)
        k = apply_rope(k, cos, sin)
        q = q.transpose(1, 2).contiguous()
        k = k.transpose(1, 2).contiguous()
        v = v.transpose(1, 2).contiguous()
        out = self.ops.attention(q, k, v, self.window)
        out = out.transpose(1, 2).contiguous().view(B, T, self.n_heads * self.head_dim)
        return self.ops.linear(out, self.wo)

    def ffn(self, h: torch.Tensor) -> torch.Tensor:
        gate, up = self.ops.linear(h, self.w_gate_up).chunk(2, dim=-1)
        return self.ops.linear(self.ops.silu(gate.contiguous()) * up, self.w_down)

    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(self.ops.rms_norm(x, self.norm1, self.eps), cos, sin)
        x = x + self.ffn(self.ops.rms_norm(x, self.norm2, self.eps))
        return x
