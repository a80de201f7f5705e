"""ROCm operators for the decoder layer around the attention.

Mirrors the repop operators the reference's modules call:
  linear(x, w)          repop.nn.linear.Linear forward (src/pretrain/model/modules/_linear.py:31-65)
  rms_norm(x, w, eps)   repop.nn.rmsnorm.rms_norm (src/pretrain/model/modules/norm_repop.py:19-22)
  silu(x)               repop.nn.activations.silu (src/pretrain/model/modules/ffn_repop.py:28-36)
Each is a torch.autograd.Function over the C ABI of libotx_attn.so: bf16 in,
binary32 arithmetic in a fixed order, bf16 out; weight gradients come back in
the weight's dtype.  GPU tensors only; there is no CPU fallback.
"""

from __future__ import annotations

import torch

from .. import _lib

__all__ = ["linear", "rms_norm", "silu"]

_DT = {torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _need_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if t.device.type != "cuda":
            raise RuntimeError(f"tensor on {t.device}: this operator is the ROCm (HIP) backend and only accepts GPU tensors")


def gemm_bf16(a: torch.Tensor, a_strides: tuple[int, int], b: torch.Tensor, b_strides: tuple[int, int],
              M: int, N: int, R: int, out_dtype: torch.dtype = torch.bfloat16, variant: int = 0) -> torch.Tensor:
    """C[M, N] with C[i][j] = serial fold over r of A(i, r) * B(j, r) (strides in elements).
    ``variant``: 0 lets the library choose the tile form, 1 and 2 force the wide and
    the narrow one (same bytes)."""
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise ValueError("gemm_bf16 takes bfloat16 operands")
    c = torch.empty((M, N), dtype=out_dtype, device=a.device)
    lib = _lib.load()
    rc = lib.otx_gemm_bf16_ex(a.data_ptr(), a_strides[0], a_strides[1], b.data_ptr(), b_strides[0], b_strides[1],
                              c.data_ptr(), N, M, N, R, _DT[out_dtype], variant, _stream(a))
    _lib.check(rc, "otx_gemm_bf16_ex")
    return c


class _Linear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w):
        K = x.shape[-1]
        N = w.shape[0]
        x2 = x.reshape(-1, K).contiguous()
        wc = w.contiguous()
        M = x2.shape[0]
        y = gemm_bf16(x2, (K, 1), wc, (K, 1), M, N, K)  # y = x @ w^T
        ctx.save_for_backward(x2, wc)
        ctx.xshape = x.shape
        return y.view(*x.shape[:-1], N)

    @staticmethod
    def backward(ctx, dy):
        x2, w = ctx.saved_tensors
        M, K = x2.shape
        N = w.shape[0]
        dy2 = dy.reshape(M, N).contiguous()
        dx = dw = None
        if ctx.needs_input_grad[0]:  # dx[m][k] = sum_n dy[m][n] w[n][k]
            dx = gemm_bf16(dy2, (N, 1), w, (1, K), M, K, N).view(ctx.xshape)
        if ctx.needs_input_grad[1]:  # dw[n][k] = sum_m dy[m][n] x[m][k]
            dw = gemm_bf16(dy2, (1, N), x2, (1, K), N, K, M)
        return dx, dw


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """y = x @ w^T (no bias), bf16 operands, serial binary32 fold, bf16 result."""
    _need_gpu(x, w)
    return _Linear.apply(x, w)


class _RMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, eps):
        D = x.shape[-1]
        xc = x.contiguous()
        wc = w.to(x.dtype).contiguous()
        rows = xc.numel() // D
        y = torch.empty_like(xc)
        rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
        rc = _lib.load().otx_rmsnorm_fwd(xc.data_ptr(), wc.data_ptr(), y.data_ptr(), rstd.data_ptr(), rows, D, eps,
                                         _DT[x.dtype], _stream(x))
        _lib.check(rc, "otx_rmsnorm_fwd")
        ctx.save_for_backward(xc, wc, rstd)
        ctx.wdtype = w.dtype
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w, rstd = ctx.saved_tensors
        D = x.shape[-1]
        rows = x.numel() // D
        dyc = dy.contiguous()
        dx = torch.empty_like(x)
        dw = torch.empty(D, dtype=torch.float32, device=x.device)
        lib = _lib.load()
        nbytes = int(lib.otx_rmsnorm_bwd_workspace_bytes(rows, D))
        ws = torch.empty(max(nbytes, 4), dtype=torch.uint8, device=x.device)
        rc = lib.otx_rmsnorm_bwd(x.data_ptr(), w.data_ptr(), rstd.data_ptr(), dyc.data_ptr(), dx.data_ptr(),
                                 dw.data_ptr(), rows, D, _DT[x.dtype], ws.data_ptr(), nbytes, _stream(x))
        _lib.check(rc, "otx_rmsnorm_bwd")
        return dx, dw.to(ctx.wdtype), None


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over the last dimension; output in x's dtype, rstd kept for backward."""
    _need_gpu(x, w)
    if x.dtype not in _DT:
        raise ValueError(f"dtype {x.dtype} not supported")
    return _RMSNorm.apply(x, w, float(eps))


class _SiLU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        xc = x.contiguous()
        y = torch.empty_like(xc)
        rc = _lib.load().otx_silu_fwd(xc.data_ptr(), y.data_ptr(), xc.numel(), _DT[x.dtype], _stream(x))
        _lib.check(rc, "otx_silu_fwd")
        ctx.save_for_backward(xc)
        return y

    @staticmethod
    def backward(ctx, dy):
        (x,) = ctx.saved_tensors
        dyc = dy.contiguous()
        dx = torch.empty_like(x)
        rc = _lib.load().otx_silu_bwd(x.data_ptr(), dyc.data_ptr(), dx.data_ptr(), x.numel(), _DT[x.dtype],
                                      _stream(x))
        _lib.check(rc, "otx_silu_bwd")
        return dx


def silu(x: torch.Tensor) -> torch.Tensor:
    """SiLU with a correctly rounded exp, in x's dtype."""
    _need_gpu(x)
    if x.dtype not in _DT:
        raise ValueError(f"dtype {x.dtype} not supported")
    return _SiLU.apply(x)
