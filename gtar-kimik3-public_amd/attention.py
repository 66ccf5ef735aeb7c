"""Causal grouped-query softmax attention for the hybrid stack's attention layer, on gfx950 (gdr_attention_fwd and
gdr_attention_bwd).

Drop-in for `flash_attention` (src/ops/flash_attention_2.py:210-222) and its autograd function `FlashAttention`
(:159-207): same name, arguments, default scale (`softmax_scale or head_dim ** -0.5`), autocast rule, layout (q
[B, H, T, D], k and v [B, Hkv, T, D] with Hkv dividing H) and gradients, plus an optional `cu_seqlens` (int32
[N + 1], batch 1) that confines attention to each packed sequence -- the reference pads batches instead and has no
packed form (:154-156).  Under autograd the forward also keeps each row's log-sum-exp (fp32 [B, H, T]) for the
backward, as the reference's saves its `lse` (:175).  Differences, both deliberate: CPU tensors raise (the reference
falls back to SDPA there, :220-221), and fp32 inputs raise (the kernels compute on bf16 / f16 MFMA).
"""

from __future__ import annotations

import torch

from . import _lib
from ._common import _as_row_aligned


class _FlashAttentionFunction(torch.autograd.Function):
    """Forward with the row log-sum-exp kept; backward = gdr_attention_bwd (dQ, then dK / dV per key block)."""

    @staticmethod
    def forward(ctx, query, key, value, softmax_scale, cu_seqlens):
        out = torch.empty(query.shape, device=query.device, dtype=query.dtype)
        lse = torch.empty(query.shape[:3], device=query.device, dtype=torch.float32)
        _lib.attention(query, key, value, out, softmax_scale, cu_seqlens, query.device, lse=lse)
        ctx.save_for_backward(query, key, value, out, lse, cu_seqlens)
        ctx.softmax_scale = softmax_scale
        return out

    @staticmethod
    def backward(ctx, d_out):
        query, key, value, out, lse, cu_seqlens = ctx.saved_tensors
        d_out = _as_row_aligned(d_out)
        d_q = torch.empty(query.shape, device=query.device, dtype=query.dtype)
        d_k = torch.empty(key.shape, device=key.device, dtype=key.dtype)
        d_v = torch.empty(value.shape, device=value.device, dtype=value.dtype)
        delta = torch.empty_like(lse)
        _lib.attention_bwd(query, key, value, out, lse, ctx.softmax_scale, cu_seqlens, d_out.to(query.dtype), d_q,
                           d_k, d_v, delta, query.device)
        return d_q, d_k, d_v, None, None


@torch.compiler.disable
def flash_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    softmax_scale: float | None = None,
    cu_seqlens: torch.Tensor | None = None,
) -> torch.Tensor:
    """Causal attention; returns [B, H, T, D] in the query dtype (differentiable in q, k and v)."""
    name = "flash_attention"
    softmax_scale = softmax_scale or query.shape[-1] ** -0.5
    if torch.is_autocast_enabled("cuda"):
        dtype = torch.get_autocast_dtype("cuda")
        query, key, value = query.to(dtype), key.to(dtype), value.to(dtype)
    tensors = [t for t in (query, key, value, cu_seqlens) if t is not None]
    if not all(t.is_cuda for t in tensors):
        raise ValueError(f"{name}: all tensors must be on the GPU (this implementation has no CPU path)")
    if query.dtype not in (torch.bfloat16, torch.float16) or key.dtype != query.dtype or value.dtype != query.dtype:
        raise ValueError(f"{name}: q, k, v must share one dtype, bf16 or f16 (got {query.dtype}, {key.dtype}, "
                         f"{value.dtype})")
    if query.dim() != 4 or key.dim() != 4 or key.shape != value.shape or key.shape[0] != query.shape[0] or \
            key.shape[2:] != query.shape[2:] or query.shape[1] % key.shape[1]:
        raise ValueError(f"{name}: expected q [B,H,T,D] and k, v [B,Hkv,T,D] with Hkv dividing H, got "
                         f"{tuple(query.shape)}, {tuple(key.shape)}, {tuple(value.shape)}")
    if cu_seqlens is not None:
        if query.shape[0] != 1:
            raise ValueError(f"{name}: cu_seqlens requires batch size 1 (packed sequences)")
        cu_seqlens = cu_seqlens.to(torch.int32).contiguous()
    query, key, value = (_as_row_aligned(x) for x in (query, key, value))
    if torch.is_grad_enabled() and any(t.requires_grad for t in (query, key, value)):
        return _FlashAttentionFunction.apply(query, key, value, softmax_scale, cu_seqlens)
    out = torch.empty(query.shape, device=query.device, dtype=query.dtype)
    _lib.attention(query, key, value, out, softmax_scale, cu_seqlens, query.device)
    return out
