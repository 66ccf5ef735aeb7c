// Recurrent (decode) forward of the gated delta-rule family on gfx950.
//
// Reference semantics: `_recurrent_forward` in src/ops/kimi_delta_attention.py:38-68 (KDA),
// src/ops/gated_deltanet.py:29-59 (GDN), src/ops/gated_linear_attention.py:30-56 (GLA) and
// src/ops/deltanet.py:30-57 (DeltaNet).  Per token t, with S the fp32 [K, V] state of one (batch, head):
//   S <- diag(e^{g_t}) S                    (per-channel decay; scalar for GDN; none for DeltaNet)
//   u <- beta_t (v_t - k_t S)               (delta rule; GLA uses u = v_t)
//   S <- S + k_t^T u
//   o_t <- scale q_t S  = scale (q_t S_decayed + (q_t . k_t) u)
//
// Design: the state is streamed exactly once per call (one 128-bit load and one 128-bit store per float4),
// so the kernel is HBM-bound at T = 1.  One workgroup owns a [K, VS] column slice of one (b, h) state: 512
// threads for 128-column slices (large batches), 256 threads for 32-column slices (small batches, so they still
// launch enough workgroups).  Thread (quad, rg) holds float4 column quad `quad` of rows rg, rg + RG, ... in
// registers for the whole call; few rows per thread keep the register count low enough for 6+ waves per SIMD,
// which together with non-temporal state loads keeps enough bytes in flight.  Both dk-reductions (k S and q S)
// come out of one pass over the registers, are reduced across lanes with shuffles and across waves through LDS,
// and the rank-1 update is applied in place in registers before the single store.  Only the tiny per-token
// vectors go through LDS.
//
// Speculative verify (recurrent_verify_kernel) runs the same body over the 1 + draft tokens of a block and writes
// each token's update row u_t to an fp32 record as well; recurrent_commit_kernel rebuilds the state after any
// accepted prefix from the block's initial state, k, the gate and that record, with the same fp32 operations in the
// same order, so its state after all T tokens equals the verify kernel's final state bit for bit.
#include "recurrent_impl.h"

namespace gdr {

template <int VARIANT, typename InT>
static hipError_t launch_recurrent_v(const gdr_args& a, hipStream_t stream, int vs, RecMode mode, const RecExtra& x) {
  if (mode == RecMode::kCommitVerify ? x.prev->h0 != nullptr : a.h0 != nullptr)
    return a.key_dim == 64 ? launch_recurrent_k<VARIANT, 64, InT, true>(a, stream, vs, mode, x)
                           : launch_recurrent_k<VARIANT, 128, InT, true>(a, stream, vs, mode, x);
  return a.key_dim == 64 ? launch_recurrent_k<VARIANT, 64, InT, false>(a, stream, vs, mode, x)
                         : launch_recurrent_k<VARIANT, 128, InT, false>(a, stream, vs, mode, x);
}

template <typename InT>
static hipError_t launch_recurrent_t(const gdr_args& a, hipStream_t stream, int vs, RecMode mode, const RecExtra& x) {
  switch (a.variant) {
    case GDR_KDA: return launch_recurrent_v<GDR_KDA, InT>(a, stream, vs, mode, x);
    case GDR_GDN: return launch_recurrent_v<GDR_GDN, InT>(a, stream, vs, mode, x);
    case GDR_GLA: return launch_recurrent_v<GDR_GLA, InT>(a, stream, vs, mode, x);
    default: return launch_recurrent_v<GDR_DELTANET, InT>(a, stream, vs, mode, x);
  }
}

static hipError_t launch_family(const gdr_args& a, hipStream_t stream, RecMode mode, const RecExtra& x,
                                int dtype) {
  // Wide slices stream the most bytes per workgroup; narrow slices give small batches enough workgroups.
  const long long wide_blocks = (long long)(a.cu_seqlens ? a.n_seqs : a.batch) * a.heads * (a.value_dim / 128);
  const int vs = (a.value_dim % 128 == 0 && wide_blocks >= 1024) ? 128 : 32;
  if (a.key_dim != 64 && a.key_dim != 128) return launch_recurrent_other_k(a, stream, vs, mode, x, dtype);
  return dtype == GDR_BF16 ? launch_recurrent_t<__bf16>(a, stream, vs, mode, x)
                           : launch_recurrent_t<float>(a, stream, vs, mode, x);
}

hipError_t launch_recurrent(const gdr_args& a, hipStream_t stream) {
  return launch_family(a, stream, RecMode::kForward, RecExtra{}, a.q.dtype);
}

hipError_t launch_verify(const gdr_args& a, float* updates, hipStream_t stream) {
  return launch_family(a, stream, RecMode::kVerify, RecExtra{updates, nullptr, nullptr, nullptr}, a.q.dtype);
}

hipError_t launch_commit(const gdr_args& a, const float* updates, const int32_t* accepted, hipStream_t stream) {
  return launch_family(a, stream, RecMode::kCommit, RecExtra{nullptr, updates, accepted, nullptr}, a.k.dtype);
}

hipError_t launch_commit_verify(const gdr_args& prev, const float* prev_updates, const int32_t* accepted,
                                const gdr_args& a, float* updates, hipStream_t stream) {
  return launch_family(a, stream, RecMode::kCommitVerify, RecExtra{updates, prev_updates, accepted, &prev},
                       a.q.dtype);
}

}  // namespace gdr
