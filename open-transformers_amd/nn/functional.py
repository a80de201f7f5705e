"""ROCm operators for the decoder layer around the attention.

Mirrors the repop operators the reference's modules call:
  linear(x, w)          repop.nn.linear.Linear forward (src/pretrain/model/modules/_linear.py:31-65)
  rms_norm(x, w, eps)   repop.nn.rmsnorm.rms_norm (src/pretrain/model/modules/norm_repop.py:19-22)
  silu(x)               repop.nn.activations.silu (src/pretrain/model/modules/ffn_repop.py:28-36)
and the torch compositions around them, each fused into one pass:
  swiglu(gu)            gate, up = gu.chunk(2, -1); silu(gate) * up (ffn_repop.py:52-54)
  rope_heads(x, c, s)   apply_rope(x, c, s).transpose(1, 2).contiguous()
                        (rope.py:103-125, attention_repop.py:143-149)
  heads(x)              x.transpose(1, 2).contiguous() (attention_repop.py:150)
  merge_heads(o)        o.transpose(1, 2).contiguous().view(B, T, H * D) (attention_repop.py:155)
Each is a torch.autograd.Function over the C ABI of libotx_attn.so: bf16 in,
binary32 arithmetic in a fixed order, bf16 out, and for the compositions the
bytes torch's own forward and autograd backward give; weight gradients come
back in the weight's dtype.  GPU tensors only; there is no CPU fallback.
"""

from __future__ import annotations

import torch

from .. import _lib

__all__ = ["linear", "rms_norm", "silu", "swiglu", "rope_heads", "heads", "merge_heads"]

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
    ``variant``: 0 lets the library choose the tile form, 1, 2 and 3 force the wide
    (128 x 128), the narrow (128 x 64) and the small (64 x 64) one (same bytes)."""
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


class _SwiGLU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gu):
        F = gu.shape[-1] // 2
        guc = gu.contiguous()
        rows = guc.numel() // (2 * F)
        h = torch.empty(*gu.shape[:-1], F, dtype=gu.dtype, device=gu.device)
        rc = _lib.load().otx_swiglu_fwd(guc.data_ptr(), h.data_ptr(), rows, F, _DT[gu.dtype], _stream(gu))
        _lib.check(rc, "otx_swiglu_fwd")
        ctx.save_for_backward(guc)
        return h

    @staticmethod
    def backward(ctx, dh):
        (gu,) = ctx.saved_tensors
        F = gu.shape[-1] // 2
        rows = gu.numel() // (2 * F)
        dhc = dh.contiguous()
        dgu = torch.empty_like(gu)
        rc = _lib.load().otx_swiglu_bwd(gu.data_ptr(), dhc.data_ptr(), dgu.data_ptr(), rows, F, _DT[gu.dtype],
                                        _stream(gu))
        _lib.check(rc, "otx_swiglu_bwd")
        return dgu


def swiglu(gu: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up for gate, up = gu.chunk(2, -1), in one pass; the last
    dimension of gu is 2F with F a multiple of 8."""
    _need_gpu(gu)
    if gu.dtype not in _DT:
        raise ValueError(f"dtype {gu.dtype} not supported")
    if gu.shape[-1] % 16:
        raise ValueError(f"swiglu: last dimension {gu.shape[-1]} is not a multiple of 16")
    return _SwiGLU.apply(gu)


class _RopeHeads(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, cos, sin):
        B, T, H, D = x.shape
        xc = x.contiguous()
        y = torch.empty((B, H, T, D), dtype=x.dtype, device=x.device)
        rc = _lib.load().otx_rope_heads_fwd(xc.data_ptr(), cos.data_ptr(), sin.data_ptr(), y.data_ptr(), B, T, H, D,
                                            _DT[x.dtype], _stream(x))
        _lib.check(rc, "otx_rope_heads_fwd")
        ctx.save_for_backward(cos, sin)
        return y

    @staticmethod
    def backward(ctx, dy):
        cos, sin = ctx.saved_tensors
        B, H, T, D = dy.shape
        dyc = dy.contiguous()
        dx = torch.empty((B, T, H, D), dtype=dy.dtype, device=dy.device)
        rc = _lib.load().otx_rope_heads_bwd(dyc.data_ptr(), cos.data_ptr(), sin.data_ptr(), dx.data_ptr(), B, T, H, D,
                                            _DT[dy.dtype], _stream(dy))
        _lib.check(rc, "otx_rope_heads_bwd")
        return dx, None, None


def rope_heads(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """RoPE of x [B, T, H, D] (interleaved pairs, cos/sin binary32 [T, D/2]) into
    the attention layout [B, H, T, D]."""
    _need_gpu(x, cos, sin)
    if x.dtype not in _DT:
        raise ValueError(f"dtype {x.dtype} not supported")
    if x.dim() != 4 or x.shape[-1] % 8:
        raise ValueError(f"rope_heads takes x [B, T, H, D] with D a multiple of 8, got {tuple(x.shape)}")
    T, D = x.shape[1], x.shape[3]
    for name, t in (("cos", cos), ("sin", sin)):
        if t.dtype != torch.float32 or tuple(t.shape) != (T, D // 2):
            raise ValueError(f"rope_heads: {name} must be binary32 [{T}, {D // 2}], got {t.dtype} {tuple(t.shape)}")
    return _RopeHeads.apply(x, cos.contiguous(), sin.contiguous())


def _swap12(x: torch.Tensor) -> torch.Tensor:
    B, X, Y, D = x.shape
    xc = x.contiguous()
    y = torch.empty((B, Y, X, D), dtype=x.dtype, device=x.device)
    rc = _lib.load().otx_swap_heads(xc.data_ptr(), y.data_ptr(), B, X, Y, D, _DT[x.dtype], _stream(x))
    _lib.check(rc, "otx_swap_heads")
    return y


class _SwapHeads(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        return _swap12(x)

    @staticmethod
    def backward(ctx, dy):
        return _swap12(dy)


def heads(x: torch.Tensor) -> torch.Tensor:
    """[B, T, H, D] -> [B, H, T, D] (contiguous)."""
    _need_gpu(x)
    if x.dtype not in _DT or x.dim() != 4 or x.shape[-1] % 8:
        raise ValueError(f"heads takes a bf16/binary32 [B, T, H, D] tensor with D a multiple of 8, got {x.dtype} "
                         f"{tuple(x.shape)}")
    return _SwapHeads.apply(x)


def merge_heads(o: torch.Tensor) -> torch.Tensor:
    """[B, H, T, D] -> [B, T, H * D] (contiguous)."""
    _need_gpu(o)
    if o.dtype not in _DT or o.dim() != 4 or o.shape[-1] % 8:
        raise ValueError(f"merge_heads takes a bf16/binary32 [B, H, T, D] tensor with D a multiple of 8, got "
                         f"{o.dtype} {tuple(o.shape)}")
    B, H, T, D = o.shape
    return _SwapHeads.apply(o).view(B, T, H * D)
