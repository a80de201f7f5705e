"""ROCm implementation of the reference's fused cross-entropy + z-loss.

Mirrors ``pretrain.model.fused_loss.fused_ce_z_loss(logits, labels, coeff,
*, chunk_rows=...) -> (ce, z_loss)`` (src/pretrain/model/fused_loss.py:107-120)
and its autograd function (:40-104): ``ce = mean(lse - logit[label])``,
``z_loss = coeff * mean(lse ** 2)``, one shared logsumexp per row, a single
combined gradient of the logits in the logits' dtype.  Both passes run the
gfx950 kernels of libotx_attn.so (csrc/loss.hip) on the current stream; only
the per-row (max, Z, lse) statistics are kept between forward and backward, so
nothing [N, V] in binary32 is ever materialised (the reason the reference
chunks its rows; ``chunk_rows`` is accepted and has no effect on the bytes).
"""

from __future__ import annotations

import torch

from .. import _lib

__all__ = ["fused_ce_z_loss", "ce_zloss_forward", "ce_zloss_backward"]

_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}


def _check(logits: torch.Tensor, labels: torch.Tensor) -> tuple[int, int]:
    if logits.device.type != "cuda":
        raise RuntimeError(f"logits are on {logits.device}: this fused loss is the ROCm (HIP) backend")
    if logits.dim() != 2 or labels.dim() != 1 or labels.shape[0] != logits.shape[0]:
        raise ValueError(f"expected logits [N, V] and labels [N], got {tuple(logits.shape)} and {tuple(labels.shape)}")
    if logits.dtype not in _DTYPES:
        raise ValueError(f"logits dtype {logits.dtype} not supported (bfloat16 or float32)")
    if labels.dtype != torch.int64 or labels.device != logits.device:
        raise ValueError("labels must be int64 on the logits' device")
    return logits.shape[0], logits.shape[1]


def ce_zloss_forward(logits: torch.Tensor, labels: torch.Tensor, coeff: float):
    """(ce, z, stats) for contiguous logits [N, V] and int64 labels [N]."""
    N, V = _check(logits, labels)
    logits, labels = logits.contiguous(), labels.contiguous()
    stats = torch.empty((5, N), dtype=torch.float32, device=logits.device)
    loss = torch.empty(2, dtype=torch.float32, device=logits.device)
    with torch.cuda.device(logits.device):
        rc = _lib.load().otx_ce_zloss_fwd(logits.data_ptr(), labels.data_ptr(), N, V, _DTYPES[logits.dtype],
                                          float(coeff), stats.data_ptr(), loss.data_ptr(),
                                          torch.cuda.current_stream(logits.device).cuda_stream)
    _lib.check(rc, "otx_ce_zloss_fwd")
    return loss[0], loss[1], stats


def ce_zloss_backward(logits, labels, stats, grad_ce, grad_z, coeff: float) -> torch.Tensor:
    N, V = _check(logits, labels)
    logits, labels = logits.contiguous(), labels.contiguous()
    g = torch.stack([grad_ce.reshape(()).float(), grad_z.reshape(()).float()]).contiguous()
    grad = torch.empty_like(logits)
    with torch.cuda.device(logits.device):
        rc = _lib.load().otx_ce_zloss_bwd(logits.data_ptr(), labels.data_ptr(), stats.data_ptr(), g.data_ptr(), N, V,
                                          _DTYPES[logits.dtype], float(coeff), grad.data_ptr(),
                                          torch.cuda.current_stream(logits.device).cuda_stream)
    _lib.check(rc, "otx_ce_zloss_bwd")
    return grad


class _FusedCEZLoss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, labels, coeff):
        ce, z, stats = ce_zloss_forward(logits, labels, coeff)
        ctx.save_for_backward(logits, labels, stats)
        ctx.coeff = coeff
        return ce, z

    @staticmethod
    def backward(ctx, grad_ce, grad_z):
        logits, labels, stats = ctx.saved_tensors
        return ce_zloss_backward(logits, labels, stats, grad_ce, grad_z, ctx.coeff), None, None


def fused_ce_z_loss(logits: torch.Tensor, labels: torch.Tensor, coeff: float, *, chunk_rows: int = 2048):
    """Fused ``(ce, z_loss)`` over ``[..., V]`` logits and matching labels;
    ``coeff == 0`` gives ``z_loss == 0`` and no z gradient."""
    del chunk_rows  # row chunking is a memory device of the reference; the kernels need none
    flat_logits = logits.reshape(-1, logits.shape[-1])
    flat_labels = labels.reshape(-1)
    return _FusedCEZLoss.apply(flat_logits, flat_labels, float(coeff))
