"""Decode-state owner for one gated delta-rule layer, mirroring `RecurrentCache` (src/cache.py:48-86).

The state is one fp32 [B, H, K, V] tensor (V contiguous, the layout libgdr's kernels stream) plus three
depthwise-convolution tails.  `update` swaps in the op's fresh final state, as the reference does (:55-57);
`fork` snapshots, `commit` drops the snapshot and `rollback` restores it (:59-86), which is how a speculative
verify pass is undone.

One deliberate difference: `fork` keeps the state tensor itself rather than a clone.  No op of this package writes
its initial state (every final state is a fresh tensor, and `update` rebinds rather than copies), so the tensor
held at fork time is unchanged at rollback; a clone would stream the whole state (268 MB per layer at batch 256,
16 heads, 128 x 128) through HBM twice for nothing.  Code that writes `cache.state` in place between fork and
rollback must clone it itself.  The conv tails are written in place by their owner, so they are still copied.
`accept` finishes a verify with `VerifiedBlock.commit`: it adopts the state after the accepted prefix without
restoring and replaying anything.
"""

from __future__ import annotations

import torch


class RecurrentCache:
    def __init__(self, batch_size: int, num_heads: int, head_dim: int, value_dim: int, inner_size: int,
                 conv_size: int, device, dtype):
        self.state = torch.zeros(batch_size, num_heads, head_dim, value_dim, device=device, dtype=torch.float32)
        self.conv_states = [torch.zeros(batch_size, inner_size, conv_size - 1, device=device, dtype=dtype)
                            for _ in range(3)]
        self.seq_len = 0
        self._snapshot = None

    def update(self, state: torch.Tensor, seq_len: int) -> None:
        """Adopt the op's final state (the op always returns a fresh tensor) and advance the length."""
        self.state = state.contiguous()
        self.seq_len += seq_len

    def fork(self) -> None:
        """Snapshot the state (by reference: nothing writes it in place) and copies of the conv tails."""
        self._snapshot = (self.state, [c.clone() for c in self.conv_states], self.seq_len)

    def commit(self, n_accepted: int) -> None:
        """Keep the current state and drop the snapshot."""
        if self._snapshot is None:
            raise RuntimeError("commit() called without fork()")
        self._snapshot = None

    def rollback(self) -> None:
        """Restore the state and conv tails captured by the last fork()."""
        if self._snapshot is None:
            raise RuntimeError("rollback() called without fork()")
        state, conv_states, seq_len = self._snapshot
        self.state = state
        for dst, src in zip(self.conv_states, conv_states):
            dst.copy_(src)
        self.seq_len = seq_len
        self._snapshot = None

    def accept(self, n_accepted: int, block, conv_states=None) -> torch.Tensor:
        """Keep the first `n_accepted` tokens of a verified block and drop the snapshot: the state becomes
        `block.commit(n_accepted)` (the block started from the state held at fork time) and `seq_len` advances by
        n_accepted from the fork point.  This replaces rollback + replay (src/speculative.py:425-449) and, with
        n_accepted equal to the block length, commit (:397).  The conv tails belong to the layer's short
        convolution, which this package does not run: pass the tails after the accepted prefix as `conv_states`,
        or leave them as they are by passing None.  Returns the new state."""
        if self._snapshot is None:
            raise RuntimeError("accept() called without fork()")
        state, _, seq_len = self._snapshot
        if block.initial_state is not None and block.initial_state.data_ptr() != state.data_ptr():
            raise ValueError("the verified block did not start from the state held at fork()")
        self.state = block.commit(n_accepted)
        if conv_states is not None:
            for dst, src in zip(self.conv_states, conv_states):
                dst.copy_(src)
        self.seq_len = seq_len + int(n_accepted)
        self._snapshot = None
        return self.state
