"""Multi-token verify for speculative decoding, with the state kept as a replayable record instead of a clone.

The reference verifies a block of T = 1 + K tokens (the pending token and K drafts) by cloning the layer's
recurrent state (`RecurrentCache.fork`, src/cache.py:59-69), running the chunk op on the block padded to 64 tokens
(src/speculative.py:351-356, src/ops/utils.py:70-72), and on a rejection restoring the clone and replaying the
accepted prefix through the model (src/speculative.py:425-449).

Here `verify` runs the recurrent kernel over the block (the state is read once and kept in registers for all T
tokens) and records each token's update row u_t, fp32 [B, H, T, V]: beta_t (v_t - k_t S_t) for the delta-rule
variants and v_t for GLA.  `VerifiedBlock.commit(accepted)` then rebuilds the state after the first accepted[b]
tokens of each sequence from the state the block started from, k, the gate and that record (gdr_recurrent_commit),
so nothing is cloned before the verify and nothing is re-run after a rejection.  The block's initial state is only
read, never written, which is why holding a reference to it is a valid snapshot.

`verify(..., pending=block, accepted=n)` runs one whole speculative cycle in one launch
(gdr_recurrent_commit_verify): the previous block's accepted prefix is applied to the state held in registers,
the committed state is written out (it becomes the new block's initial state), and the new block is verified from
it.  The results are bit-identical to `block.commit(n)` followed by `verify(..., initial_state=that state)`, and the
state crosses HBM once each way per cycle instead of twice in and once out.
"""

from __future__ import annotations

import torch

from . import _lib
from ._common import _VARIANT_NAMES, _wants_grad


class VerifiedBlock:
    """What gdr_recurrent_commit needs to rebuild any accepted prefix's state: the block's initial state (None for
    zero), k and the gate as the kernel read them, and the update record."""

    def __init__(self, variant, key, gate, initial_state, updates, value_dim):
        self.variant = variant
        self.key = key
        self.gate = gate
        self.initial_state = initial_state
        self.updates = updates
        self.value_dim = value_dim

    @property
    def num_tokens(self) -> int:
        return self.key.shape[2]

    def _accepted(self, accepted):
        """The accept count as the kernels take it: None (all T tokens) or a device int32 [B] tensor."""
        batch, _, seq_len, _ = self.key.shape
        device = self.key.device
        if accepted is not None and not torch.is_tensor(accepted):
            n = int(accepted)
            if not 0 <= n <= seq_len:
                raise ValueError(f"accepted={n} outside [0, {seq_len}]")
            return None if n == seq_len else torch.full((batch,), n, dtype=torch.int32, device=device)
        if accepted is not None:
            if accepted.shape != (batch,) or accepted.device != device:
                raise ValueError(f"accepted must be a [{batch}] tensor on {device}, got {tuple(accepted.shape)} on "
                                 f"{accepted.device}")
            accepted = accepted.to(torch.int32).contiguous()
        return accepted

    def _state_out(self, out):
        batch, heads, _, key_dim = self.key.shape
        shape = (batch, heads, key_dim, self.value_dim)
        if out is None:
            return torch.empty(shape, device=self.key.device, dtype=torch.float32)
        if tuple(out.shape) != shape or out.dtype != torch.float32 or not out.is_contiguous():
            raise ValueError(f"out must be a contiguous fp32 tensor of shape {shape}")
        return out

    def _commit_args(self, out):
        args = _lib.make_args(self.variant, self.key, self.key, self.key, self.gate, None, None, 1.0,
                              self.initial_state, out)
        args.value_dim = self.value_dim
        return args

    def commit(self, accepted=None, out: torch.Tensor | None = None) -> torch.Tensor:
        """State after the first `accepted` tokens: an int for every sequence, a device int tensor [B] (one count
        per sequence, clamped to [0, T] on the device, never read by the host), or None for all T tokens.  Returns
        a fresh fp32 [B, H, K, V] tensor, or writes `out` (which may be the block's initial state)."""
        accepted = self._accepted(accepted)
        out = self._state_out(out)
        _lib.commit(self._commit_args(out), self.updates, accepted, self.key.device)
        return out


def verify(variant: int, query, key, value, gate, beta, scale=None, initial_state=None, output_final_state=False,
           pending: VerifiedBlock | None = None, accepted=None, committed_out: torch.Tensor | None = None):
    """Recurrent forward over a verify block that also returns a `VerifiedBlock`:
    `(out, final_state or None, block)`.  Arguments and dtype rules are those of the recurrent ops.

    With `pending` (the previous cycle's block) the verify starts from `pending.commit(accepted)`, computed in the
    same launch and written to `committed_out` (a fresh tensor when None; it may be `pending.initial_state`);
    `initial_state` must then be None, and the committed state is the returned block's `initial_state`."""
    name = _VARIANT_NAMES[variant]
    if pending is not None:
        if initial_state is not None:
            raise ValueError(f"{name}: pass either initial_state or pending, not both")
        if pending.variant != variant:
            raise ValueError(f"{name}: the pending block is of another variant")
    elif accepted is not None or committed_out is not None:
        raise ValueError(f"{name}: accepted and committed_out need a pending block")
    if _wants_grad(query, key, value, gate, beta, initial_state):
        raise NotImplementedError(f"{name}: verify has no backward; run it under torch.no_grad()")
    tensors = [t for t in (query, key, value, gate, beta, initial_state) if t is not None]
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
    scale = scale or key_dim ** -0.5
    out_dtype = value.dtype
    if gate is not None:
        expect = (batch, heads, seq_len) if variant == _lib.GDN else (batch, heads, seq_len, key_dim)
        if tuple(gate.shape) != expect:
            raise ValueError(f"{name}: gate must have shape {expect}, got {tuple(gate.shape)}")
        gate = gate.float()
    if beta is not None:
        if tuple(beta.shape) != (batch, heads, seq_len):
            raise ValueError(f"{name}: beta must have shape {(batch, heads, seq_len)}, got {tuple(beta.shape)}")
        beta = beta.float()
    state_shape = (batch, heads, key_dim, value_dim)
    if pending is not None:
        if tuple(pending.key.shape[:2]) != (batch, heads) or pending.key.shape[3] != key_dim or \
                pending.value_dim != value_dim:
            raise ValueError(f"{name}: the pending block has other sizes than this block")
        if pending.key.device != device:
            raise ValueError(f"{name}: the pending block is on another device")
    if initial_state is not None:
        if tuple(initial_state.shape) != state_shape:
            raise ValueError(f"{name}: initial_state must have shape {state_shape}, got {tuple(initial_state.shape)}")
        initial_state = initial_state.float().contiguous()
    if not (query.dtype == key.dtype == value.dtype == torch.bfloat16):
        query, key, value = (x if x.dtype == torch.float32 else x.float() for x in (query, key, value))

    out = torch.empty(batch, heads, seq_len, value_dim, device=device, dtype=out_dtype)
    final_state = torch.empty(state_shape, device=device, dtype=torch.float32) if output_final_state else None
    updates = torch.empty(batch, heads, seq_len, value_dim, device=device, dtype=torch.float32)
    if pending is not None and pending.key.dtype != query.dtype:
        # The one-launch cycle reads both blocks' k in one dtype; with mixed dtypes, commit then verify.
        initial_state, pending = pending.commit(accepted, committed_out), None
    if pending is not None:
        acc = pending._accepted(accepted)
        initial_state = pending._state_out(committed_out)
        args = _lib.make_args(variant, query, key, value, gate, beta, out, scale, initial_state, final_state)
        _lib.commit_verify(pending._commit_args(initial_state), pending.updates, acc, args, updates, device)
    else:
        args = _lib.make_args(variant, query, key, value, gate, beta, out, scale, initial_state, final_state)
        _lib.verify(args, updates, device)
    block = VerifiedBlock(variant, key, gate, initial_state, updates, value_dim)
    return out, final_state, block
