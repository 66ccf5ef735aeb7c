"""Gated linear attention (per-channel forget gate, no delta rule) on gfx950.

    S_t = diag(exp(g_t)) S_{t-1} + k_t^T v_t,   o_t = scale q_t S_t

Drop-in for src/ops/gated_linear_attention.py: `chunk_gated_linear_attention` (:444-458) and
`recurrent_gated_linear_attention` (:461-483), same signatures (no beta) and conventions.
"""

from __future__ import annotations

import torch

from . import _lib
from ._common import run
from .verify import verify


@torch.compiler.disable
def chunk_gated_linear_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    gate: torch.Tensor,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    cu_seqlens: torch.Tensor | None = None,
):
    """Chunkwise (prefill) GLA forward; `cu_seqlens` as in chunk_kimi_delta_attention."""
    return run(_lib.GLA, True, query, key, value, gate, None, scale, initial_state, output_final_state, cu_seqlens)


def recurrent_gated_linear_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    gate: torch.Tensor,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
):
    """Token-by-token (decode) GLA forward."""
    return run(_lib.GLA, False, query, key, value, gate, None, scale, initial_state, output_final_state)


def verify_gated_linear_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    gate: torch.Tensor,
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
    return verify(_lib.GLA, query, key, value, gate, None, scale, initial_state, output_final_state, pending,
                  accepted, committed_out)
