"""Gated DeltaNet (delta rule with a scalar per-head forget gate) on gfx950.

    S_t = exp(g_t) S_{t-1},   u_t = beta_t (v_t - k_t S_t),   S_t = S_t + k_t^T u_t,   o_t = scale q_t S_t

Drop-in for src/ops/gated_deltanet.py: `chunk_gated_deltanet` (:479-494) and `recurrent_gated_deltanet`
(:497-520), same signatures and conventions.  gate and beta are (batch, heads, seq_len).
"""

from __future__ import annotations

import torch

from . import _lib
from ._common import run
from .verify import verify


@torch.compiler.disable
def chunk_gated_deltanet(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    gate: torch.Tensor,
    beta: torch.Tensor,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    cu_seqlens: torch.Tensor | None = None,
):
    """Chunkwise (prefill) Gated DeltaNet forward; `cu_seqlens` as in chunk_kimi_delta_attention."""
    return run(_lib.GDN, True, query, key, value, gate, beta, scale, initial_state, output_final_state, cu_seqlens)


def recurrent_gated_deltanet(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    gate: torch.Tensor,
    beta: torch.Tensor,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
):
    """Token-by-token (decode) Gated DeltaNet forward."""
    return run(_lib.GDN, False, query, key, value, gate, beta, scale, initial_state, output_final_state)


def verify_gated_deltanet(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    gate: torch.Tensor,
    beta: torch.Tensor,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    pending=None,
    accepted=None,
    committed_out: torch.Tensor | None = None,
):
    """Speculative-decoding verify over a block of tokens: the recurrent forward plus a `VerifiedBlock` whose
    `commit(accepted)` rebuilds the state after any accepted prefix.  Returns `(out, final_state or None, block)`.
    With `pending` (the previous block) the state is `pending.commit(accepted)`, computed in the same launch and
    returned as the new block's `initial_state`; `initial_state` must then be None."""
    return verify(_lib.GDN, query, key, value, gate, beta, scale, initial_state, output_final_state, pending,
                  accepted, committed_out)
