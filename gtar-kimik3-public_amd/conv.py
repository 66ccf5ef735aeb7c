"""Segment-aware depthwise causal convolution + SiLU for the layers' short convolution, on gfx950
(gdr_short_conv_fwd).

The reference's ShortConvolution (src/layers/short_convolution.py:6-20) runs nn.Conv1d with left padding over the
batch layout, or F.conv1d over [conv_state, x] with the state updated in place.  With packed sequences it would mix
the end of one sequence into the start of the next (:9, :15); here `cu_seqlens` restarts the convolution at every
sequence, from that sequence's state.
"""

from __future__ import annotations

import torch

from . import _lib


def short_convolution(
    hidden_states: torch.Tensor,
    weight: torch.Tensor,
    conv_state: torch.Tensor | None = None,
    cu_seqlens: torch.Tensor | None = None,
    activation: bool = True,
) -> torch.Tensor:
    """silu(conv(x)) for x [B, T, C] (batch 1 with `cu_seqlens`), weight [C, 1, W] or [C, W] (nn.Conv1d with
    groups=C).  `conv_state` [N, C, W - 1] (N = B, or the number of packed sequences) supplies the inputs before each
    sequence and is updated in place to its last W - 1 inputs, as the reference updates its cache (:16-19)."""
    name = "short_convolution"
    x = hidden_states
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (x, weight, conv_state)):
        raise NotImplementedError(f"{name}: forward only; run under torch.no_grad()")
    tensors = [t for t in (x, weight, conv_state, cu_seqlens) if t is not None]
    if not all(t.is_cuda for t in tensors):
        raise ValueError(f"{name}: all tensors must be on the GPU (this implementation has no CPU path)")
    if x.dim() != 3:
        raise ValueError(f"{name}: expected x [B, T, C], got {tuple(x.shape)}")
    batch, _, channels = x.shape
    w = weight.reshape(weight.shape[0], weight.shape[-1])
    if w.shape[0] != channels:
        raise ValueError(f"{name}: weight must be [C, 1, W] for C = {channels}, got {tuple(weight.shape)}")
    width = w.shape[1]
    w = w.to(x.dtype).contiguous()
    if cu_seqlens is not None:
        if batch != 1:
            raise ValueError(f"{name}: cu_seqlens requires batch size 1 (packed sequences)")
        cu_seqlens = cu_seqlens.to(torch.int32).contiguous()
    n_states = batch if cu_seqlens is None else cu_seqlens.numel() - 1
    if conv_state is not None and tuple(conv_state.shape) != (n_states, channels, width - 1):
        raise ValueError(f"{name}: conv_state must be {(n_states, channels, width - 1)}, got {tuple(conv_state.shape)}")
    if x.stride(-1) != 1 or x.data_ptr() % 16 or (x.stride(0) * x.element_size()) % 16 or \
            (x.stride(1) * x.element_size()) % 16:
        x = x.contiguous()
    out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    state_in = conv_state.to(x.dtype).contiguous() if conv_state is not None else None
    # The kernel writes the new state of every sequence that has tokens; a sequence of length 0 (and every sequence
    # when T == 0, which launches nothing) keeps its state, as the reference's does.
    state_out = state_in.clone() if state_in is not None else None
    _lib.short_conv(x, out, w, state_in, state_out, cu_seqlens, activation, x.device)
    if conv_state is not None:
        conv_state.copy_(state_out)
    return out
