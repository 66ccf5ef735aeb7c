"""Seeded synthetic inputs for the benchmark configurations of this op family.

The generators follow the input recipes attached to each configuration: q and k drawn N(0, 1) and
L2-normalised along the key dimension, v ~ N(0, 1), beta = sigmoid(N(0, 1)) per (b, t, h), log-gates
g = -softplus(N(0, 1)) (per channel for KDA and GLA, one per (b, t, h) for Gated DeltaNet), initial state
~ N(0, sigma) or zero.  Tensors are drawn on the CPU from one `torch.Generator` in the layer's [B, T, H, D]
order (as src/layers/kimi_delta_attention.py:41-49 produces them), moved to `device`, and returned in the op
layout [B, H, T, D] -- as contiguous tensors, or as the layer's transposed views when `layer_layout` is set
(src/layers/kimi_delta_attention.py:53), so both code paths of the strided loads get exercised.
"""

from __future__ import annotations

import dataclasses

import torch
import torch.nn.functional as F

GATES = {"kda": "channel", "gla": "channel", "gdn": "scalar", "deltanet": None}
BETAS = {"kda": True, "gdn": True, "gla": False, "deltanet": True}


@dataclasses.dataclass
class Inputs:
    query: torch.Tensor
    key: torch.Tensor
    value: torch.Tensor
    gate: torch.Tensor | None
    beta: torch.Tensor | None
    initial_state: torch.Tensor | None

    def args(self):
        """Positional op arguments in the reference order for the variant (gate and beta only if it takes them)."""
        return [x for x in (self.query, self.key, self.value, self.gate, self.beta) if x is not None]

    def to(self, device):
        move = lambda x: None if x is None else x.to(device)
        return Inputs(*(move(x) for x in dataclasses.astuple(self)))


def make_inputs(variant: str, batch: int, seq_len: int, heads: int, key_dim: int, value_dim: int, *,
                seed: int = 0, dtype=torch.bfloat16, state_std: float | None = None, gate_scale: float = 1.0,
                device="cpu", layer_layout: bool = False) -> Inputs:
    """Draw one seeded input set.  `gate_scale` divides the log-gates (the reference tests' gate/16 ... gate/0.1
    knob); `state_std` None means a zero (absent) initial state."""
    gen = torch.Generator("cpu").manual_seed(seed)
    randn = lambda *shape: torch.randn(*shape, generator=gen, dtype=torch.float32)
    shape_k = (batch, seq_len, heads, key_dim)
    shape_v = (batch, seq_len, heads, value_dim)
    query = F.normalize(randn(shape_k), dim=-1).to(dtype)
    key = F.normalize(randn(shape_k), dim=-1).to(dtype)
    value = randn(shape_v).to(dtype)
    gate = None
    if GATES[variant] == "channel":
        gate = -F.softplus(randn(shape_k)) / gate_scale
    elif GATES[variant] == "scalar":
        gate = -F.softplus(randn(batch, seq_len, heads)) / gate_scale
    beta = torch.sigmoid(randn(batch, seq_len, heads)) if BETAS[variant] else None
    state = None
    if state_std is not None:
        state = randn(batch, heads, key_dim, value_dim) * state_std

    def place(x):
        if x is None:
            return None
        x = x.to(device)
        x = x.transpose(1, 2)
        return x if layer_layout else x.contiguous()

    return Inputs(place(query), place(key), place(value), place(gate), place(beta),
                  None if state is None else state.to(device))


def decode_inputs(variant: str, batch: int, heads: int, key_dim: int, value_dim: int, *, seed: int = 0,
                  dtype=torch.bfloat16, device="cpu") -> Inputs:
    """One decode token per sequence ([B, H, 1, D] views), without an initial state."""
    return make_inputs(variant, batch, 1, heads, key_dim, value_dim, seed=seed, dtype=dtype, device=device)


def decode_state(batch: int, heads: int, key_dim: int, value_dim: int, *, std: float = 0.02, seed: int = 0,
                 device="cpu") -> torch.Tensor:
    """fp32 decode state ~ N(0, std), drawn in slabs so a multi-GB state never needs a second host copy."""
    gen = torch.Generator("cpu").manual_seed(seed)
    out = torch.empty(batch, heads, key_dim, value_dim, dtype=torch.float32, device=device)
    for b in range(batch):
        out[b].copy_(torch.randn(heads, key_dim, value_dim, generator=gen, dtype=torch.float32) * std)
    return out


def varlen_lengths(n_seqs: int = 32, low: int = 256, high: int = 4096, *, seed: int = 0) -> list[int]:
    """Sequence lengths ~ U[low, high] (inclusive), seeded: the packed-prefill configuration's length mix."""
    gen = torch.Generator("cpu").manual_seed(seed)
    return [int(x) for x in torch.randint(low, high + 1, (n_seqs,), generator=gen)]


def make_varlen_inputs(variant: str, lengths: list[int], heads: int, key_dim: int, value_dim: int, *, seed: int = 0,
                       dtype=torch.bfloat16, state_std: float | None = 0.02, device="cpu"):
    """Packed [1, H, sum(lengths), D] inputs with int32 `cu_seqlens` [N + 1] and a per-sequence initial state
    [N, H, K, V] (None when `state_std` is None).  Returns (Inputs, cu_seqlens)."""
    total = sum(lengths)
    inp = make_inputs(variant, 1, total, heads, key_dim, value_dim, seed=seed, dtype=dtype, device=device)
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)), dtype=torch.int32, device=device)
    if state_std is not None:
        gen = torch.Generator("cpu").manual_seed(seed + 1)
        inp.initial_state = (torch.randn(len(lengths), heads, key_dim, value_dim, generator=gen,
                                         dtype=torch.float32) * state_std).to(device)
    return inp, cu
