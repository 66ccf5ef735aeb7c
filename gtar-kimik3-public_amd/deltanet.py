"""DeltaNet (delta rule, no decay) on gfx950.

    u_t = beta_t (v_t - k_t S_{t-1}),   S_t = S_{t-1} + k_t^T u_t,   o_t = scale q_t S_t

Drop-in for src/ops/deltanet.py: `chunk_deltanet` (:406-420) and `recurrent_deltanet` (:423-445), same
signatures (no gate) and conventions.
"""

from __future__ import annotations

import torch

from . import _lib
from ._common import run
from .verify import verify


@torch.compiler.disable
def chunk_deltanet(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    beta: torch.Tensor,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    cu_seqlens: torch.Tensor | None = None,
):
    """Chunkwise (prefill) DeltaNet forward; `cu_seqlens` as in chunk_kimi_delta_attention."""
    return run(_lib.DELTANET, True, query, key, value, None, beta, scale, initial_state, output_final_state,
               cu_seqlens)


def recurrent_deltanet(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    beta: torch.Tensor,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
):
    """Token-by-token (decode) DeltaNet forward."""
    return run(_lib.DELTANET, False, query, key, value, None, beta, scale, initial_state, output_final_state)


def verify_deltanet(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
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
    return verify(_lib.DELTANET, query, key, value, None, beta, scale, initial_state, output_final_state, pending,
                  accepted, committed_out)
