"""ROCm implementation of ``repop.nn.flash_attention``.

Mirrors the operator the reference harness calls at
src/pretrain/model/modules/attention_repop.py:53::

    causal_flash_attention(q, k, v, dropout=0.0, window=window) -> Tensor

q is [B, H, T, D]; k and v are [B, Hkv, T, D] (GQA-native: query head h reads
KV head h // (H // Hkv), attention_repop.py:83,146-147); the 1/sqrt(D) scale is
applied inside (attention_repop.py:17,152); window == 0 is full causal,
otherwise a sliding window of ``window`` keys (attention_repop.py:94-96,153).
The forward returns only O; the fp32 logsumexp is kept for the backward, which
returns dq, dk, dv in the input dtype (docs/MODEL_OP_DTYPE_TRACE.md:102).

Every call runs the gfx950 kernels of libotx_attn.so through its C ABI on the
current HIP stream.  Tensors on any other device are refused: this package is
the ROCm backend, and a silent CPU fallback would void the bit-exactness claim.
"""

from __future__ import annotations

import contextlib
import threading

import torch

from .. import _lib

__all__ = [
    "causal_flash_attention",
    "int8pv_causal_flash_attention",
    "flash_attention_forward",
    "flash_attention_forward_sc",
    "flash_attention_backward",
    "int8pv_flash_attention_forward",
    "int8pv_flash_attention_forward_sc",
    "set_score_cache",
    "score_cache_enabled",
    "attention_checkpoint_contexts",
    "cpu_attention_checkpoint_contexts",
]

_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}

# Score cache: with bf16 inputs the forward also stores its scaled scores
# (one binary32 32x32 tile per processed block pair, about 4 bytes per causal
# pair) and the backward reads them instead of recomputing Q K^T.  The bytes of
# every result are the same either way; the cache trades that memory for the
# backward's score recompute.
_SCORE_CACHE = True


def set_score_cache(enabled: bool) -> bool:
    """Turn the score cache of the autograd operators on or off; returns the previous setting."""
    global _SCORE_CACHE
    prev = _SCORE_CACHE
    _SCORE_CACHE = bool(enabled)
    return prev


def score_cache_enabled() -> bool:
    return _SCORE_CACHE


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _check_inputs(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int) -> tuple[int, int, int, int, int]:
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if t.device.type != "cuda" or t.is_meta:
            raise RuntimeError(
                f"{name} is on {t.device}: this causal_flash_attention is the ROCm (HIP) backend "
                "and only accepts GPU tensors"
            )
        if t.dim() != 4:
            raise ValueError(f"{name} must be 4-D [B, H, T, D], got shape {tuple(t.shape)}")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous (the kernel reads raw row-major pointers)")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"q, k, v dtypes differ: {q.dtype}, {k.dtype}, {v.dtype}")
    if q.dtype not in _DTYPES:
        raise ValueError(f"dtype {q.dtype} not supported (bfloat16 or float32)")
    if not (q.device == k.device == v.device):
        raise ValueError("q, k, v must be on the same device")
    B, H, S, D = q.shape
    Bk, Hkv, Sk, Dk = k.shape
    if tuple(v.shape) != tuple(k.shape):
        raise ValueError(f"k and v shapes differ: {tuple(k.shape)} vs {tuple(v.shape)}")
    if Bk != B or Sk != S or Dk != D:
        raise ValueError(f"k/v shape {tuple(k.shape)} incompatible with q shape {tuple(q.shape)}")
    if H % Hkv != 0:
        raise ValueError(f"n_heads ({H}) must be a multiple of n_kv_heads ({Hkv})")
    if S % 32 != 0:
        raise ValueError(f"sequence length {S} must be a multiple of 32")
    if D not in (64, 128):
        raise ValueError(f"head_dim {D} not supported (64 or 128)")
    if not isinstance(window, int) or window < 0 or window % 32 != 0:
        raise ValueError(f"window must be 0 (full causal) or a positive multiple of 32, got {window!r}")
    return B, H, Hkv, S, D


def flash_attention_forward(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int = 0, variant: int = 0
) -> tuple[torch.Tensor, torch.Tensor]:
    """Forward pass returning (O, LSE).  ``variant`` selects a launch shape
    (0 default, 1, 2); all variants give identical bits."""
    B, H, Hkv, S, D = _check_inputs(q, k, v, window)
    o = torch.empty_like(q)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
    lib = _lib.load()
    with torch.cuda.device(q.device):
        rc = lib.otx_attn_fwd_ex(
            _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), B, H, Hkv, S, D, window, _DTYPES[q.dtype], variant,
            _stream(q.device),
        )
    _lib.check(rc, "otx_attn_fwd")
    return o, lse


def score_cache_bytes(B: int, H: int, S: int, window: int) -> int:
    return int(_lib.load().otx_attn_score_cache_bytes(B, H, S, window))


def _new_score_cache(B: int, H: int, S: int, window: int, device: torch.device) -> torch.Tensor:
    return torch.empty(score_cache_bytes(B, H, S, window) // 4, dtype=torch.float32, device=device)


def flash_attention_forward_sc(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int = 0, variant: int = 0
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """:func:`flash_attention_forward` that also returns the score cache (bf16 only)."""
    B, H, Hkv, S, D = _check_inputs(q, k, v, window)
    if q.dtype != torch.bfloat16:
        raise ValueError(f"the score cache is defined for bfloat16 inputs, got {q.dtype}")
    o = torch.empty_like(q)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
    sc = _new_score_cache(B, H, S, window, q.device)
    lib = _lib.load()
    with torch.cuda.device(q.device):
        rc = lib.otx_attn_fwd_sc(
            _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), _ptr(sc), sc.numel() * 4, B, H, Hkv, S, D, window,
            _DTYPES[q.dtype], variant, _stream(q.device),
        )
    _lib.check(rc, "otx_attn_fwd_sc")
    return o, lse, sc


def workspace_bytes(B: int, H: int, Hkv: int, S: int, D: int, window: int) -> int:
    return int(_lib.load().otx_attn_bwd_workspace_bytes(B, H, Hkv, S, D, window))


def flash_attention_backward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    o: torch.Tensor,
    lse: torch.Tensor,
    dout: torch.Tensor,
    window: int = 0,
    variant: int = 0,
    score_cache: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Backward pass returning (dq, dk, dv) in the input dtype.  With
    ``score_cache`` (from a ``*_forward_sc`` call on the same q, k), the
    scores are read instead of recomputed; the result bytes are the same."""
    B, H, Hkv, S, D = _check_inputs(q, k, v, window)
    if dout.shape != q.shape or dout.dtype != q.dtype or dout.device != q.device:
        raise ValueError("grad_output must match q in shape, dtype and device")
    if o.shape != q.shape or o.dtype != q.dtype or o.device != q.device:
        raise ValueError("o must match q in shape, dtype and device")
    if lse.shape != (B, H, S) or lse.dtype != torch.float32 or lse.device != q.device:
        raise ValueError("lse must be float32 [B, H, T] on q's device")
    dout = dout.contiguous()
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    nbytes = workspace_bytes(B, H, Hkv, S, D, window)
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device=q.device)
    base = ws.data_ptr()
    aligned = (base + 255) & ~255
    lib = _lib.load()
    with torch.cuda.device(q.device):
        if score_cache is None:
            rc = lib.otx_attn_bwd_ex(
                _ptr(q), _ptr(k), _ptr(v), _ptr(o.contiguous()), _ptr(lse.contiguous()), _ptr(dout), _ptr(dq),
                _ptr(dk), _ptr(dv), B, H, Hkv, S, D, window, _DTYPES[q.dtype], aligned, nbytes, variant,
                _stream(q.device),
            )
        else:
            if score_cache.dtype != torch.float32 or score_cache.device != q.device or not score_cache.is_contiguous():
                raise ValueError("score_cache must be a contiguous float32 tensor on q's device")
            rc = lib.otx_attn_bwd_sc(
                _ptr(q), _ptr(k), _ptr(v), _ptr(o.contiguous()), _ptr(lse.contiguous()), _ptr(dout), _ptr(dq),
                _ptr(dk), _ptr(dv), _ptr(score_cache), score_cache.numel() * 4, B, H, Hkv, S, D, window,
                _DTYPES[q.dtype], aligned, nbytes, variant, 7, _stream(q.device),
            )
    _lib.check(rc, "otx_attn_bwd")
    return dq, dk, dv


# ---- activation checkpointing: keep the attention results of the first forward ----
_ckpt = threading.local()


@contextlib.contextmanager
def _ckpt_mode(mode, cache):
    prev = getattr(_ckpt, "state", None)
    _ckpt.state = (mode, cache)
    try:
        yield
    finally:
        _ckpt.state = prev


def attention_checkpoint_contexts():
    """``context_fn`` for ``torch.utils.checkpoint`` / ``checkpoint_wrapper``
    (the role of repop's ``cpu_attention_checkpoint_contexts``,
    src/pretrain/parallel/parallelize_llama3_repop.py:118-124): the checkpointed
    forward records each attention call's results (O, LSE and, when enabled,
    the score cache) in call order, and the recompute in the backward takes
    them back instead of launching the forward again.  The kernels are
    deterministic, so the bytes are those a recompute would produce; the trade
    is the memory of those results against one attention forward per
    checkpointed block."""
    cache: list = []
    return _ckpt_mode("record", cache), _ckpt_mode("replay", cache)


cpu_attention_checkpoint_contexts = attention_checkpoint_contexts  # the reference's name for the same hook


def _forward_cached(fwd, q, k, v, window):
    """Runs ``fwd`` (returning O, LSE and optionally the score cache) unless a
    checkpoint replay hands back the recorded results of the first forward."""
    state = getattr(_ckpt, "state", None)
    if state is not None and state[0] == "replay" and state[1]:
        return tuple(t.detach() for t in state[1].pop(0))
    out = fwd(q, k, v, window)
    if state is not None and state[0] == "record":
        state[1].append(tuple(t.detach() for t in out))
    return out


def _use_score_cache(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
    """Keep the score cache only for bf16 inputs whose backward can run: grad
    mode on and some input requiring grad (under no_grad, or for inputs that
    need no gradient, the O(S^2) cache would be written and never read).  The
    checkpointed forward of activation checkpointing qualifies: it runs with
    grad enabled.  Decided before ``Function.apply``, inside which grad mode is
    always off."""
    return (_SCORE_CACHE and q.dtype == torch.bfloat16 and torch.is_grad_enabled()
            and (q.requires_grad or k.requires_grad or v.requires_grad))


def _checkpoint_discards_saved_tensors() -> bool:
    """True inside the first forward of non-reentrant activation checkpointing
    (``torch.utils.checkpoint(..., use_reentrant=False)``, the mode of the
    ``checkpoint_wrapper`` that src/pretrain/parallel/parallelize_llama3_repop.py:
    107-130 puts around every block): the pack hook it installs keeps none of
    the tensors an operator saves, and the block's forward runs again in the
    backward to make them.  Recognised by that hook's qualified name."""
    try:
        top = torch._C._autograd._top_saved_tensors_default_hooks(False)
    except (AttributeError, RuntimeError, TypeError):
        return False
    return bool(top) and getattr(top[0], "__qualname__", "").startswith("_checkpoint_hook.")


# What the forward does with the score cache (decided before Function.apply).
_SC_NONE, _SC_KEEP, _SC_PLACEHOLDER = 0, 1, 2


def _score_cache_mode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> int:
    """_SC_KEEP when the backward will read the cache this forward writes.
    _SC_PLACEHOLDER in the first forward of non-reentrant checkpointing without
    the recording ``context_fn``: the cache would be written and dropped at
    once, and the recompute in the backward writes the one the backward reads.
    The first forward then writes no cache and saves a placeholder of the same
    shape, dtype and device (torch requires the recompute to save tensors with
    the same metadata), which holds 4 bytes."""
    if not _use_score_cache(q, k, v):
        return _SC_NONE
    state = getattr(_ckpt, "state", None)
    if _checkpoint_discards_saved_tensors() and not (state is not None and state[0] == "record"):
        return _SC_PLACEHOLDER
    return _SC_KEEP


def _forward_with_mode(fwd_plain, fwd_sc, q, k, v, window, mode):
    if mode == _SC_KEEP:
        return _forward_cached(fwd_sc, q, k, v, window)
    out = _forward_cached(fwd_plain, q, k, v, window)
    if mode == _SC_PLACEHOLDER:
        B, H, S, _ = q.shape
        n = score_cache_bytes(B, H, S, window) // 4
        out = (*out, torch.empty(1, dtype=torch.float32, device=q.device).expand(n))
    return out


def _saved_score_cache(sc):
    """The score cache saved by the forward, or None where there is none or it
    is the checkpoint placeholder (no storage behind its shape: never read)."""
    if not sc or sc[0].numel() == 0 or sc[0].stride(0) == 0:
        return None
    return sc[0]


class _CausalFlashAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, window, mode):
        out = _forward_with_mode(flash_attention_forward, flash_attention_forward_sc, q, k, v, window, mode)
        ctx.save_for_backward(q, k, v, *out)
        ctx.window = window
        return out[0]

    @staticmethod
    def backward(ctx, dout):
        q, k, v, o, lse, *sc = ctx.saved_tensors
        dq, dk, dv = flash_attention_backward(q, k, v, o, lse, dout, ctx.window, score_cache=_saved_score_cache(sc))
        return dq, dk, dv, None, None


def causal_flash_attention(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, dropout: float = 0.0, window: int = 0
) -> torch.Tensor:
    """Deterministic GQA-native causal (optionally sliding-window) attention."""
    if dropout != 0.0:
        raise ValueError("causal_flash_attention is deterministic: dropout must be 0.0")
    _check_inputs(q, k, v, window)
    return _CausalFlashAttention.apply(q, k, v, window, _score_cache_mode(q, k, v))


def int8pv_workspace_bytes(B: int, H: int, Hkv: int, S: int, D: int) -> int:
    return int(_lib.load().otx_attn_fwd_int8pv_workspace_bytes(B, H, Hkv, S, D))


def int8pv_flash_attention_forward(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int = 0, variant: int = 0
) -> tuple[torch.Tensor, torch.Tensor]:
    """int8-PV forward returning (O, LSE); bf16 inputs only.  LSE is
    bit-identical to :func:`flash_attention_forward`'s."""
    B, H, Hkv, S, D = _check_inputs(q, k, v, window)
    if q.dtype != torch.bfloat16:
        raise ValueError(f"int8pv_causal_flash_attention takes bfloat16 inputs, got {q.dtype}")
    o = torch.empty_like(q)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
    nbytes = int8pv_workspace_bytes(B, H, Hkv, S, D)
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device=q.device)
    aligned = (ws.data_ptr() + 255) & ~255
    lib = _lib.load()
    with torch.cuda.device(q.device):
        rc = lib.otx_attn_fwd_int8pv_ex(
            _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), B, H, Hkv, S, D, window, _DTYPES[q.dtype], aligned, nbytes,
            variant, _stream(q.device),
        )
    _lib.check(rc, "otx_attn_fwd_int8pv")
    return o, lse


def int8pv_flash_attention_forward_sc(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int = 0, variant: int = 0
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """:func:`int8pv_flash_attention_forward` that also returns the score cache
    (the scores are the binary32 forward's, so the cache is the same)."""
    B, H, Hkv, S, D = _check_inputs(q, k, v, window)
    if q.dtype != torch.bfloat16:
        raise ValueError(f"int8pv_causal_flash_attention takes bfloat16 inputs, got {q.dtype}")
    o = torch.empty_like(q)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
    sc = _new_score_cache(B, H, S, window, q.device)
    nbytes = int8pv_workspace_bytes(B, H, Hkv, S, D)
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device=q.device)
    aligned = (ws.data_ptr() + 255) & ~255
    lib = _lib.load()
    with torch.cuda.device(q.device):
        rc = lib.otx_attn_fwd_int8pv_sc(
            _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), _ptr(sc), sc.numel() * 4, B, H, Hkv, S, D, window,
            _DTYPES[q.dtype], aligned, nbytes, variant, _stream(q.device),
        )
    _lib.check(rc, "otx_attn_fwd_int8pv_sc")
    return o, lse, sc


class _Int8PVFlashAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, window, mode):
        out = _forward_with_mode(int8pv_flash_attention_forward, int8pv_flash_attention_forward_sc, q, k, v, window,
                                 mode)
        ctx.save_for_backward(q, k, v, *out)
        ctx.window = window
        return out[0]

    @staticmethod
    def backward(ctx, dout):
        # straight-through: the binary32 flash backward on the int8-PV forward's
        # O and LSE (docs/MODEL_OP_DTYPE_TRACE.md:102,117-119 of the reference)
        q, k, v, o, lse, *sc = ctx.saved_tensors
        dq, dk, dv = flash_attention_backward(q, k, v, o, lse, dout, ctx.window, score_cache=_saved_score_cache(sc))
        return dq, dk, dv, None, None


def int8pv_causal_flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int = 0) -> torch.Tensor:
    """GQA-native causal (optionally sliding-window) attention with int8 P.V
    (attention_repop.py:52): P quantized per (query, 32-key block), V per
    (32-key block, column), int32 products, binary32 dequantization and
    accumulation, bf16 output.  The backward is the binary32 flash backward."""
    _check_inputs(q, k, v, window)
    if q.dtype != torch.bfloat16:
        raise ValueError(f"int8pv_causal_flash_attention takes bfloat16 inputs, got {q.dtype}")
    return _Int8PVFlashAttention.apply(q, k, v, window, _score_cache_mode(q, k, v))
