"""The KDA layer's output epilogue on gfx950 (gdr_norm_gate_fwd).

The reference's KimiDeltaAttention.forward ends (src/layers/kimi_delta_attention.py:58-59) with

    out_gate = F.silu(self.output_gate_proj(hidden_states).view(head_shape))
    out = self.norm(out.transpose(1, 2)) * out_gate

where self.norm is RMSNorm over the head dimension (src/layers/rmsnorm.py:11-16).  `output_norm_gate` does the
normalisation, the SiLU and both products in one pass over the op's output and the gate's pre-activation, with the
same roundings; the gate's two projections stay in PyTorch (GEMMs).
"""

from __future__ import annotations

import torch

from . import _lib


def output_norm_gate(x: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """weight * rmsnorm(x) * silu(gate) for x, gate [B, T, H, V] (x may be the op's [B, H, T, V] output transposed),
    weight [V].  Returns [B, T, H, V], float32 when the weight is float32 (PyTorch's type promotion), else x's
    dtype."""
    name = "output_norm_gate"
    if torch.is_grad_enabled() and any(t.requires_grad for t in (x, gate, weight)):
        raise NotImplementedError(f"{name}: forward only; run under torch.no_grad()")
    if not (x.is_cuda and gate.is_cuda and weight.is_cuda):
        raise ValueError(f"{name}: all tensors must be on the GPU (this implementation has no CPU path)")
    if x.dim() != 4 or gate.shape != x.shape:
        raise ValueError(f"{name}: expected x, gate [B, T, H, V] of one shape, got {tuple(x.shape)}, "
                         f"{tuple(gate.shape)}")
    if tuple(weight.shape) != (x.shape[-1],):
        raise ValueError(f"{name}: weight must be [{x.shape[-1]}], got {tuple(weight.shape)}")
    gate = gate.to(x.dtype)
    if weight.dtype != torch.float32:
        weight = weight.to(x.dtype)
    weight = weight.contiguous()
    views = []
    for t in (x, gate):
        if t.stride(-1) != 1 or t.data_ptr() % 16 or any((s * t.element_size()) % 16 for s in t.stride()[:3]):
            t = t.contiguous()
        views.append(t)
    out_dtype = torch.float32 if weight.dtype == torch.float32 else x.dtype
    out = torch.empty(x.shape, device=x.device, dtype=out_dtype)
    _lib.norm_gate(views[0], views[1], weight, out, eps, x.device)
    return out
