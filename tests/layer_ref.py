"""CPU implementation of the decoder layer's byte-sensitive operators on top of
the C oracle, with the same interface as ``open_transformers_amd.nn.layer.ROCM_OPS``
(test infrastructure: lets the same ``DecoderLayer`` code run on CPU tensors as
the checker of the GPU run)."""

from __future__ import annotations

import types

import numpy as np
import torch

from oracle import oracle as orc


def _f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.float32).contiguous().numpy()


def _to(a: np.ndarray, like: torch.Tensor) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(like.dtype)


class _Linear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w):
        ctx.save_for_backward(x, w)
        x2 = _f32(x).reshape(-1, x.shape[-1])
        y = orc.gemm(x2, _f32(w), out_bf16=True)
        return _to(y, x).view(*x.shape[:-1], w.shape[0])

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        K, N = x.shape[-1], w.shape[0]
        x2 = _f32(x).reshape(-1, K)
        dy2 = _f32(dy).reshape(-1, N)
        dx = orc.gemm(dy2, _f32(w).T, out_bf16=True)       # dx[m][k] = sum_n dy[m][n] w[n][k]
        dw = orc.gemm(dy2.T, x2.T, out_bf16=True)           # dw[n][k] = sum_m dy[m][n] x[m][k]
        return _to(dx, x).view(x.shape), _to(dw, w)


class _RMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, eps):
        y, rstd = orc.rmsnorm_fwd(_f32(x), _f32(w), eps, out_bf16=x.dtype == torch.bfloat16)
        ctx.save_for_backward(x, w)
        ctx.rstd = rstd
        return _to(y, x)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        dx, dw = orc.rmsnorm_bwd(_f32(x), _f32(w), ctx.rstd, _f32(dy), out_bf16=x.dtype == torch.bfloat16)
        return _to(dx, x), torch.from_numpy(dw).to(w.dtype), None


class _SiLU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        ctx.save_for_backward(x)
        return _to(orc.silu_fwd(_f32(x), out_bf16=x.dtype == torch.bfloat16), x)

    @staticmethod
    def backward(ctx, dy):
        (x,) = ctx.saved_tensors
        return _to(orc.silu_bwd(_f32(x), _f32(dy), out_bf16=x.dtype == torch.bfloat16), x)


class _Attention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, window):
        bf = q.dtype == torch.bfloat16
        o, lse = orc.attn_fwd(_f32(q), _f32(k), _f32(v), window=window, out_bf16=bf)
        ctx.save_for_backward(q, k, v)
        ctx.o, ctx.lse, ctx.window = o, lse, window
        return _to(o, q)

    @staticmethod
    def backward(ctx, do):
        q, k, v = ctx.saved_tensors
        bf = q.dtype == torch.bfloat16
        dq, dk, dv = orc.attn_bwd(_f32(q), _f32(k), _f32(v), ctx.o, ctx.lse, _f32(do), window=ctx.window, out_bf16=bf)
        return _to(dq, q), _to(dk, k), _to(dv, v), None


class _AttentionInt8PV(torch.autograd.Function):
    """int8-PV forward, binary32 straight-through backward at its O and LSE."""

    @staticmethod
    def forward(ctx, q, k, v, window):
        o, lse = orc.attn_fwd_int8pv(_f32(q), _f32(k), _f32(v), window=window, out_bf16=True)
        ctx.save_for_backward(q, k, v)
        ctx.o, ctx.lse, ctx.window = o, lse, window
        return _to(o, q)

    @staticmethod
    def backward(ctx, do):
        q, k, v = ctx.saved_tensors
        dq, dk, dv = orc.attn_bwd(_f32(q), _f32(k), _f32(v), ctx.o, ctx.lse, _f32(do), window=ctx.window,
                                  out_bf16=True)
        return _to(dq, q), _to(dk, k), _to(dv, v), None


class _Embedding(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ids, w):
        ctx.save_for_backward(ids)
        ctx.V = w.shape[0]
        ctx.wdtype = w.dtype
        return w.detach()[ids]  # a row gather: no arithmetic

    @staticmethod
    def backward(ctx, g):
        (ids,) = ctx.saved_tensors
        gw = orc.embedding_bwd(ids.numpy(), _f32(g), ctx.V, out_bf16=ctx.wdtype == torch.bfloat16)
        return None, torch.from_numpy(gw).to(ctx.wdtype)


class _Loss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, labels, coeff):
        x = _f32(logits).reshape(-1, logits.shape[-1])
        ce, z, st = orc.ce_zloss_fwd(x, labels.reshape(-1).numpy(), coeff)
        ctx.save_for_backward(logits, labels)
        ctx.st, ctx.coeff = st, coeff
        return torch.tensor(ce), torch.tensor(z)

    @staticmethod
    def backward(ctx, gce, gz):
        logits, labels = ctx.saved_tensors
        x = _f32(logits).reshape(-1, logits.shape[-1])
        g = orc.ce_zloss_bwd(x, labels.reshape(-1).numpy(), ctx.st, ctx.coeff, gce=float(gce), gz=float(gz),
                             out_bf16=logits.dtype == torch.bfloat16)
        return torch.from_numpy(g).to(logits.dtype).view(logits.shape), None, None


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """The reference's rotary embedding as torch operations (rope.py:103-125):
    x [B, T, H, D] in pairs (x[2i], x[2i+1]); cos/sin [T, D/2] binary32."""
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


def rope_heads_ref(x, cos, sin):
    """apply_rope then the attention layout (attention_repop.py:143-149), torch autograd."""
    return apply_rope(x, cos, sin).transpose(1, 2).contiguous()


def heads_ref(x):
    return x.transpose(1, 2).contiguous()


def merge_heads_ref(o):
    B, H, T, D = o.shape
    return o.transpose(1, 2).contiguous().view(B, T, H * D)


def swiglu_ref(gu, silu=None):
    """ffn_repop.py:52-54: gate, up = gu.chunk(2, -1); silu(gate) * up (torch product
    and chunk backward; SiLU from the C oracle unless given)."""
    gate, up = gu.chunk(2, dim=-1)
    return (silu or _SiLU.apply)(gate.contiguous()) * up


ORACLE_OPS = types.SimpleNamespace(
    linear=_Linear.apply,
    rms_norm=lambda x, w, eps: _RMSNorm.apply(x, w, float(eps)),
    silu=_SiLU.apply,
    swiglu=swiglu_ref,
    rope_heads=rope_heads_ref,
    heads=heads_ref,
    merge_heads=merge_heads_ref,
    attention=lambda q, k, v, window: _Attention.apply(q, k, v, window),
    attention_int8pv=lambda q, k, v, window: _AttentionInt8PV.apply(q, k, v, window),
    embedding=_Embedding.apply,
    loss=lambda logits, labels, coeff: _Loss.apply(logits, labels, float(coeff)),
)
