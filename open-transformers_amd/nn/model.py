"""Decoder-only language model assembled from the ROCm operators.

Mirrors the reference's ``Llama3`` (src/pretrain/model/llama3.py:78-137) with
the repop module set of configs/model/llama3_1b_proxy_repop.yaml: untied
embedding (embedding_repop.py:33-43: token lookup + output projection),
``n_layers`` pre-norm blocks whose attention window follows
attention_repop.py:88-96 (the last layer of every ``swa_full_every`` group and
the model's last layer are full causal, the others use ``swa_window``), optional
q/k RMSNorm and int8-PV attention, a final RMSNorm, and the fused CE + z-loss of
the training loop (fused_loss.py:107-120).  RoPE tables are built once per
sequence length (rope.py:21-31).

Every byte-sensitive operator comes from ``ops`` (see ``layer.ROCM_OPS``), so
the same module runs on the GPU kernels and, in the tests, on the CPU oracle.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from .layer import ROCM_OPS, DecoderLayer, rope_tables

__all__ = ["Llama3", "layer_window"]


def layer_window(layer_idx: int, n_layers: int, swa_window: int, swa_full_every: int) -> int:
    """The attention window of one layer (attention_repop.py:88-96)."""
    is_full = (layer_idx % swa_full_every) == (swa_full_every - 1)
    is_last = n_layers > 0 and layer_idx == n_layers - 1
    return 0 if (is_full or is_last) else swa_window


class Llama3(nn.Module):
    def __init__(self, vocab_size: int, d_model: int, n_layers: int, n_heads: int, n_kv_heads: int, head_dim: int,
                 d_ff: int, eps: float = 1e-5, rope_theta: float = 500000.0, swa_window: int = 0,
                 swa_full_every: int = 1, qk_norm: bool = False, attn_int8_pv: bool = False, ops=None,
                 dtype=torch.bfloat16, device=None):
        super().__init__()
        self.ops = ops or ROCM_OPS
        self.vocab_size, self.head_dim, self.eps, self.rope_theta = vocab_size, head_dim, eps, rope_theta
        kw = dict(dtype=dtype, device=device)
        self.tok_embeddings = nn.Parameter(torch.empty(vocab_size, d_model, **kw))
        self.blocks = nn.ModuleList([
            DecoderLayer(d_model, n_heads, n_kv_heads, head_dim, d_ff, eps=eps,
                         window=layer_window(i, n_layers, swa_window, swa_full_every), ops=self.ops, dtype=dtype,
                         device=device, qk_norm=qk_norm, int8_pv=attn_int8_pv)
            for i in range(n_layers)
        ])
        self.norm_out = nn.Parameter(torch.ones(d_model, **kw))
        self.output = nn.Parameter(torch.empty(vocab_size, d_model, **kw))
        self._rope = {}

    def rope(self, T: int, device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
        key = (T, str(device))
        if key not in self._rope:
            cos, sin = rope_tables(T, self.head_dim, self.rope_theta)
            self._rope[key] = (cos.to(device), sin.to(device))
        return self._rope[key]

    def forward_hidden(self, input_ids: torch.Tensor) -> torch.Tensor:
        cos, sin = self.rope(input_ids.shape[1], self.tok_embeddings.device)
        h = self.ops.embedding(input_ids, self.tok_embeddings)
        for block in self.blocks:
            h = block(h, cos, sin)
        return self.ops.rms_norm(h, self.norm_out, self.eps)

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Logits [B, T, vocab] in the parameter dtype."""
        return self.ops.linear(self.forward_hidden(input_ids), self.output)

    def loss(self, input_ids: torch.Tensor, labels: torch.Tensor, z_coeff: float):
        """(ce, z_loss) of the next-token labels, the training loop's fused loss."""
        return self.ops.loss(self(input_ids), labels, z_coeff)
