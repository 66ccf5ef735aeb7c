"""Decode-state owner for one gated delta-rule layer, mirroring `RecurrentCache` (src/cache.py:48-86).

The state is one fp32 [B, H, K, V] tensor (V contiguous, the layout libgdr's kernels stream) plus three
depthwise-convolution tails.  `update` swaps in the op's fresh final state, as the reference does (:55-57);
`fork` snapshots deep copies, `commit` drops the snapshot and `rollback` restores it (:59-86), which is how a
speculative verify pass is undone.
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
        """Snapshot deep copies of the state and conv tails; recurrent state cannot be shared or truncated."""
        self._snapshot = (self.state.clone(), [c.clone() for c in self.conv_states], self.seq_len)

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
        self.state = state.clone()
        for dst, src in zip(self.conv_states, conv_states):
            dst.copy_(src)
        self.seq_len = seq_len
        self._snapshot = None
