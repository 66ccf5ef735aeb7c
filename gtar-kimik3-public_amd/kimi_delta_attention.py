"""Kimi Delta Attention (delta rule with a per-channel forget gate) on gfx950.

    S_t = diag(exp(g_t)) S_{t-1},   u_t = beta_t (v_t - k_t S_t),   S_t = S_t + k_t^T u_t,   o_t = scale q_t S_t

Drop-in for src/ops/kimi_delta_attention.py: same names, argument order, defaults, dtype rules and return
convention as `chunk_kimi_delta_attention` (:645-663) and `recurrent_kimi_delta_attention` (:666-692).
Layouts are (batch, heads, seq_len, dim); gate is (batch, heads, seq_len, head_dim) fp32, beta is
(batch, heads, seq_len).  Both run hand-written HIP kernels from libgdr.so (include/gdr.h).
"""

from __future__ import annotations

import torch

from . import _lib
from ._common import run
from .verify import verify


@torch.compiler.disable
def chunk_kimi_delta_attention(
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
    """Chunkwise (prefill) KDA forward.  `cu_seqlens` (int32 [N+1], batch 1) packs N independent sequences; then
    `initial_state` and the returned final state are [N, H, K, V]."""
    return run(_lib.KDA, True, query, key, value, gate, beta, scale, initial_state, output_final_state, cu_seqlens)


def recurrent_kimi_delta_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    gate: torch.Tensor,
    beta: torch.Tensor,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
):
    """Token-by-token (decode) KDA forward; the state stays in registers for all T tokens."""
    return run(_lib.KDA, False, query, key, value, gate, beta, scale, initial_state, output_final_state)


def verify_kimi_delta_attention(
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
    return verify(_lib.KDA, query, key, value, gate, beta, scale, initial_state, output_final_state, pending,
                  accepted, committed_out)
