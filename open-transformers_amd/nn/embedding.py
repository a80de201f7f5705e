"""ROCm implementation of ``repop.nn.embedding.Embedding``.

The reference's untied embedding (src/pretrain/model/modules/
embedding_repop.py:33-40) looks tokens up with repop's Embedding, a drop-in
for ``torch.nn.Embedding`` whose backward is a deterministic fixed-order
scatter-add (docs/MODEL_OP_DTYPE_TRACE.md:75,106).  Here the forward is a row
gather and the backward folds, per token id, the gradient rows of its
positions in ascending position order in binary32, on the gfx950 kernels of
csrc/embedding.hip.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from .. import _lib

__all__ = ["Embedding", "embedding"]

_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


class _EmbeddingFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ids, weight):
        if weight.device.type != "cuda":
            raise RuntimeError(f"weight is on {weight.device}: this Embedding is the ROCm (HIP) backend")
        if weight.dtype not in _DTYPES or weight.dim() != 2 or not weight.is_contiguous():
            raise ValueError("weight must be a contiguous 2-D bfloat16 or float32 tensor")
        if ids.device != weight.device:
            # the kernels dereference the ids pointer on the GPU: a host pointer would fault.
            # RuntimeError, as torch.nn.Embedding raises for the same mismatch.
            raise RuntimeError(f"ids are on {ids.device} but weight is on {weight.device}: "
                               "Expected all tensors to be on the same device")
        flat = ids.reshape(-1).to(torch.int64).contiguous()
        V, D = weight.shape
        out = torch.empty((flat.numel(), D), dtype=weight.dtype, device=weight.device)
        with torch.cuda.device(weight.device):
            rc = _lib.load().otx_embedding_fwd(flat.data_ptr(), weight.data_ptr(), out.data_ptr(), flat.numel(), V, D,
                                               _DTYPES[weight.dtype], _stream(weight))
        _lib.check(rc, "otx_embedding_fwd")
        ctx.save_for_backward(flat)
        ctx.wshape, ctx.wdtype = (V, D), weight.dtype
        return out.view(*ids.shape, D)

    @staticmethod
    def backward(ctx, grad_out):
        (flat,) = ctx.saved_tensors
        V, D = ctx.wshape
        if grad_out.device != flat.device:
            raise RuntimeError(f"grad_output is on {grad_out.device} but the ids are on {flat.device}")
        g = grad_out.reshape(-1, D).to(ctx.wdtype).contiguous()
        gw = torch.empty((V, D), dtype=ctx.wdtype, device=g.device)
        lib = _lib.load()
        with torch.cuda.device(g.device):
            nbytes = int(lib.otx_embedding_bwd_workspace_bytes(flat.numel(), V))
            ws = torch.empty(nbytes + 256, dtype=torch.uint8, device=g.device)
            aligned = (ws.data_ptr() + 255) & ~255
            rc = lib.otx_embedding_bwd(flat.data_ptr(), g.data_ptr(), gw.data_ptr(), flat.numel(), V, D,
                                       _DTYPES[ctx.wdtype], aligned, nbytes, _stream(g))
        _lib.check(rc, "otx_embedding_bwd")
        return None, gw


def embedding(ids: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    return _EmbeddingFn.apply(ids, weight)


class Embedding(nn.Module):
    """``Embedding(num_embeddings, embedding_dim)`` with ``.weight`` [V, D]."""

    def __init__(self, num_embeddings: int, embedding_dim: int, dtype=torch.bfloat16, device=None):
        super().__init__()
        self.num_embeddings, self.embedding_dim = num_embeddings, embedding_dim
        self.weight = nn.Parameter(torch.empty(num_embeddings, embedding_dim, dtype=dtype, device=device))

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        return embedding(ids, self.weight)
