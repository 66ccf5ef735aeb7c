// Host-side declarations shared between the C-ABI layer (gdr_api.hip) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/gdr.h"

namespace gdr {

// Raises a kernel's dynamic-LDS limit to `bytes` once per process.  The function-local static is initialised by
// exactly one thread (C++11 guarantees it), so concurrent first calls from several host threads are race-free; a
// failure is remembered and returned by every later call.
template <auto Kernel>
hipError_t configure_lds(int bytes) {
  static const hipError_t status = hipFuncSetAttribute(reinterpret_cast<const void*>(Kernel),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  return status;
}

// Enqueue the recurrent forward; `a` has been validated.
hipError_t launch_recurrent(const gdr_args& a, hipStream_t stream);

// The recurrent forward that also records each token's update row u_t, fp32 [B, H, T, V], into `updates`.
hipError_t launch_verify(const gdr_args& a, float* updates, hipStream_t stream);

// a.ht <- the state after the first clamp(accepted[b], 0, T) tokens (all T when accepted is NULL), rebuilt from
// a.h0, k, the gate and a verify record.
hipError_t launch_commit(const gdr_args& a, const float* updates, const int32_t* accepted, hipStream_t stream);

// launch_commit(prev, prev_updates, accepted) into prev.ht, then launch_verify(a, updates) from that state, in one
// launch; a.h0 == prev.ht.
hipError_t launch_commit_verify(const gdr_args& prev, const float* prev_updates, const int32_t* accepted,
                                const gdr_args& a, float* updates, hipStream_t stream);

// Enqueue the chunkwise forward; `a` has been validated (q, k, v share one dtype).
hipError_t launch_chunk(const gdr_args& a, hipStream_t stream);

// Causal grouped-query attention and the segment-aware short convolution; arguments validated.
hipError_t launch_attention(const gdr_attention_args& a, hipStream_t stream);
hipError_t launch_attention_bwd(const gdr_attention_args& a, const gdr_attention_grads& g, hipStream_t stream);
hipError_t launch_short_conv(const gdr_conv_args& a, hipStream_t stream);
// The layer's output epilogue (RMSNorm x SiLU gate); arguments validated.
hipError_t launch_norm_gate(const gdr_norm_gate_args& a, hipStream_t stream);

// Value columns per state-scan workgroup (forward and reverse): the widest of 64 and 32 whose workgroups, bh
// (sequence, head) pairs times value_dim / width, still cover every CU of the current device, else 16.
int scan_slice(int64_t bh, int value_dim);

// Chunkwise forward as a chunk-parallel preparation launch plus a state-scan launch over a workspace of
// chunk_workspace_bytes(a) bytes at a.workspace; `pro` is the fused layer prologue (flags 0 for the plain op).
int64_t chunk_workspace_bytes(const gdr_args& a);
hipError_t launch_chunk_split(const gdr_args& a, const gdr_prologue& pro, hipStream_t stream);

// Byte offsets of the chunkwise-backward buffers inside its workspace (each 256-aligned).  Per (sequence, head,
// chunk):
//   rec      the forward record (chunk_workspace_bytes layout)
//   states   bf16 [K][V]   the state entering the chunk
//   dstates  bf16 [K][V]   the gradient of the state leaving it
//   ubuf     bf16 [64][V]  u = U - W S of the chunk's rows
//   dubt     bf16 [V][64]  its gradient, transposed
struct BwdLayout {
  int64_t rec, states, dstates, ubuf, dubt, total;
};
BwdLayout chunk_bwd_layout(const gdr_args& a);

// Forward recompute for the backward: the preparation launch, then the state scan in its states mode (writes
// states and ubuf instead of the output).  `ws` is the backward workspace.
hipError_t launch_chunk_states(const gdr_args& a, const BwdLayout& L, unsigned char* ws, hipStream_t stream);

// Forward for training: the chunk forward's output and final state, leaving in `ws` the records, states and u that
// launch_chunk_bwd reads (what launch_chunk_states would recompute).
hipError_t launch_chunk_train(const gdr_args& a, const BwdLayout& L, unsigned char* ws, hipStream_t stream);

// The backward proper (after launch_chunk_states or launch_chunk_train): reverse state scan, chunk-local gradients.
hipError_t launch_chunk_bwd(const gdr_args& a, const gdr_grads& g, const BwdLayout& L, unsigned char* ws,
                            hipStream_t stream);

}  // namespace gdr
