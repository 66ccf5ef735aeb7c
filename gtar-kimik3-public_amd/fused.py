"""Chunkwise KDA / GLA prefill with the layer's prologue fused into the preparation kernel (gdr_chunk_fwd_fused).

The reference's KDA layer prepares the op's inputs in PyTorch (src/layers/kimi_delta_attention.py:45-49):

    query = F.normalize(q, dim=-1);  key = F.normalize(k, dim=-1)
    beta  = sigmoid(beta_proj(x))
    gate  = -exp(A_log)[h] * softplus(decay_proj[1](decay_proj[0](x)))        # [B, T, H, K] fp32

and then calls `chunk_kimi_delta_attention` (:51-55).  The fp32 gate is the op's largest input (512 bytes per token
and head at K = 128), written by the layer and read back by the op.  Here the op takes the rank-R activations
z = decay_proj[0](x) instead (R bf16 values per token, shared by all heads), together with decay_proj[1]'s weight
and bias and A_log, and computes the gate inside the kernel on MFMA; it also normalises q and k and applies the
beta sigmoid there.  With `conv_weights`, q, k and v are the short convolutions' inputs (q_proj(x), k_proj(x),
v_proj(x)) and the kernel also applies the three depthwise convolutions (any width from 2 to 8, 4 in the layer)
and their SiLU
(ShortConvolution, src/layers/short_convolution.py:11-20), reading each sequence's conv state and, like the
reference's cache path (:16-19), updating it in place.  Gradients are not provided: training keeps the unfused op,
which is differentiable.
"""

from __future__ import annotations

import torch

from . import _lib
from ._common import _VARIANT_NAMES, _as_row_aligned, _autocast, _wants_grad


def _aligned16(x: torch.Tensor) -> torch.Tensor:
    return x if x.data_ptr() % 16 == 0 else x.clone()


def _fused(variant, query, key, value, gate_lowrank, gate_weight, gate_bias, a_log, beta, scale, initial_state,
           output_final_state, cu_seqlens, normalize_qk, beta_logits, conv_weights=None, conv_states=None):
    name = _VARIANT_NAMES[variant] + " (fused prologue)"
    conv_weights = tuple(conv_weights) if conv_weights is not None else None
    conv_states = tuple(conv_states) if conv_states is not None else None
    if conv_states is not None and conv_weights is None:
        raise ValueError(f"{name}: conv_states needs conv_weights")
    if _wants_grad(query, key, value, gate_lowrank, gate_weight, gate_bias, a_log, beta, initial_state,
                   *(conv_weights or ())):
        raise NotImplementedError(f"{name}: no backward; train with the unfused chunk op, which has one")
    tensors = [t for t in (query, key, value, gate_lowrank, gate_weight, gate_bias, a_log, beta, initial_state,
                           cu_seqlens, *(conv_weights or ()), *(conv_states or ())) if t is not None]
    if not all(t.is_cuda for t in tensors):
        raise ValueError(f"{name}: all tensors must be on the GPU (this implementation has no CPU path)")
    device = query.device
    if any(t.device != device for t in tensors):
        raise ValueError(f"{name}: all tensors must be on one device")
    if query.dim() != 4 or key.shape != query.shape or value.dim() != 4 or value.shape[:3] != query.shape[:3]:
        raise ValueError(f"{name}: expected q, k [B,H,T,K] and v [B,H,T,V], got {tuple(query.shape)}, "
                         f"{tuple(key.shape)}, {tuple(value.shape)}")
    batch, heads, seq_len, key_dim = query.shape
    value_dim = value.shape[-1]
    if gate_lowrank.dim() != 3 or gate_lowrank.shape[:2] != (batch, seq_len):
        raise ValueError(f"{name}: gate_lowrank must be [B, T, R] = [{batch}, {seq_len}, R], got "
                         f"{tuple(gate_lowrank.shape)}")
    rank = gate_lowrank.shape[-1]
    if tuple(gate_weight.shape) != (heads * key_dim, rank):
        raise ValueError(f"{name}: gate_weight must be [H*K, R] = [{heads * key_dim}, {rank}], got "
                         f"{tuple(gate_weight.shape)}")
    if gate_bias is not None and tuple(gate_bias.shape) != (heads * key_dim,):
        raise ValueError(f"{name}: gate_bias must be [H*K], got {tuple(gate_bias.shape)}")
    if tuple(a_log.shape) != (heads,):
        raise ValueError(f"{name}: a_log must be [H], got {tuple(a_log.shape)}")
    if beta is not None and tuple(beta.shape) != (batch, heads, seq_len):
        raise ValueError(f"{name}: beta must have shape {(batch, heads, seq_len)}, got {tuple(beta.shape)}")

    scale = scale or key_dim ** -0.5
    query, key, value = _autocast(query, key, value)
    out_dtype = value.dtype
    query, key, value = (_as_row_aligned(x.to(torch.bfloat16)) for x in (query, key, value))
    z = gate_lowrank.to(torch.bfloat16)
    if z.stride(-1) != 1 or z.data_ptr() % 16 or (z.stride(0) * 2) % 16 or (z.stride(1) * 2) % 16:
        z = z.contiguous()
    w = _aligned16(gate_weight.to(torch.bfloat16).contiguous())
    bias = _aligned16(gate_bias.float().contiguous()) if gate_bias is not None else None
    a_log = a_log.float().contiguous()
    if beta is not None:
        beta = beta.float()

    n_states = batch
    if cu_seqlens is not None:
        if batch != 1:
            raise ValueError(f"{name}: cu_seqlens requires batch size 1 (packed sequences), got {batch}")
        cu_seqlens = cu_seqlens.to(torch.int32).contiguous()
        n_states = cu_seqlens.numel() - 1
        if n_states < 1:
            raise ValueError(f"{name}: cu_seqlens needs at least two offsets")
    state_shape = (n_states, heads, key_dim, value_dim)
    if initial_state is not None:
        if tuple(initial_state.shape) != state_shape:
            raise ValueError(f"{name}: initial_state must have shape {state_shape}, got {tuple(initial_state.shape)}")
        initial_state = initial_state.float().contiguous()

    conv_w = states_in = states_out = None
    if conv_weights is not None:
        if len(conv_weights) != 3:
            raise ValueError(f"{name}: conv_weights must hold the q, k and v convolution weights")
        channels = (heads * key_dim, heads * key_dim, heads * value_dim)
        width = conv_weights[0].shape[-1]
        if not 2 <= width <= 8:
            raise NotImplementedError(f"{name}: in-kernel convolution of width {width}; widths 2 to 8 are supported")
        conv_w = []
        for wt, ch, nm in zip(conv_weights, channels, "qkv"):
            wt = wt.reshape(wt.shape[0], -1) if wt.dim() == 3 else wt
            if tuple(wt.shape) != (ch, width):
                raise ValueError(f"{name}: {nm} conv weight must be [{ch}, {width}] (or [{ch}, 1, {width}]), one width "
                                 f"for q, k and v; got {tuple(conv_weights[len(conv_w)].shape)}")
            conv_w.append(_aligned16(wt.to(torch.bfloat16).contiguous()))
        if conv_states is not None:
            if len(conv_states) != 3:
                raise ValueError(f"{name}: conv_states must hold the q, k and v conv states")
            states_in = []
            for st, ch, nm in zip(conv_states, channels, "qkv"):
                if tuple(st.shape) != (n_states, ch, width - 1):
                    raise ValueError(f"{name}: {nm} conv state must be [{n_states}, {ch}, {width - 1}], got "
                                     f"{tuple(st.shape)}")
                states_in.append(st.to(torch.bfloat16).contiguous())
            states_out = [st.clone() for st in states_in]  # a sequence of length 0 keeps its state

    out = torch.empty(batch, heads, seq_len, value_dim, device=device, dtype=out_dtype)
    final_state = torch.empty(state_shape, device=device, dtype=torch.float32) if output_final_state else None
    args = _lib.make_args(variant, query, key, value, None, beta, out, scale, initial_state, final_state, cu_seqlens)
    workspace = _lib.chunk_workspace(args, device)  # noqa: F841 (alive until enqueued)
    flags = _lib.PRO_GATE_LOWRANK
    if normalize_qk:
        flags |= _lib.PRO_NORM_QK
    if beta is not None and beta_logits:
        flags |= _lib.PRO_BETA_LOGITS
    if conv_w is not None:
        flags |= _lib.PRO_CONV
    pro = _lib.make_prologue(flags, z, w, bias, a_log, conv_w, states_in, states_out)
    _lib.launch_fused(args, pro, device)
    if states_out is not None:
        for st, new in zip(conv_states, states_out):
            st.copy_(new)
    return (out, final_state) if output_final_state else out


@torch.compiler.disable
def chunk_kimi_delta_attention_fused(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    gate_lowrank: torch.Tensor,
    gate_weight: torch.Tensor,
    gate_bias: torch.Tensor | None,
    a_log: torch.Tensor,
    beta: torch.Tensor,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    cu_seqlens: torch.Tensor | None = None,
    normalize_qk: bool = True,
    beta_logits: bool = True,
    conv_weights=None,
    conv_states=None,
):
    """KDA prefill from the layer's pre-op tensors: q, k [B,H,T,K] before F.normalize (when `normalize_qk`),
    v [B,H,T,V], the gate's rank-R activations `gate_lowrank` [B,T,R] = decay_proj[0](x), `gate_weight` [H*K, R]
    and `gate_bias` [H*K] of decay_proj[1], `a_log` [H], and `beta` [B,H,T] as logits (when `beta_logits`).
    With `conv_weights` (the q, k, v ShortConvolution weights, [C, 1, 4] each), q, k, v are the convolutions'
    inputs; `conv_states` (three [N, C, 3] tensors, N sequences) are read and then updated in place.
    Returns what chunk_kimi_delta_attention returns for the prepared inputs."""
    return _fused(_lib.KDA, query, key, value, gate_lowrank, gate_weight, gate_bias, a_log, beta, scale,
                  initial_state, output_final_state, cu_seqlens, normalize_qk, beta_logits, conv_weights,
                  conv_states)


@torch.compiler.disable
def chunk_gated_linear_attention_fused(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    gate_lowrank: torch.Tensor,
    gate_weight: torch.Tensor,
    gate_bias: torch.Tensor | None,
    a_log: torch.Tensor,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    cu_seqlens: torch.Tensor | None = None,
    normalize_qk: bool = False,
    conv_weights=None,
    conv_states=None,
):
    """GLA prefill with the same low-rank gate (and optionally the same short convolutions) computed in the kernel
    (no beta)."""
    return _fused(_lib.GLA, query, key, value, gate_lowrank, gate_weight, gate_bias, a_log, None, scale,
                  initial_state, output_final_state, cu_seqlens, normalize_qk, False, conv_weights, conv_states)
