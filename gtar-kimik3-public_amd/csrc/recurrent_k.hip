// The recurrent (decode) family at key dims 32, 192 and 256: the kernels of recurrent_impl.h instantiated for the
// key dims the reference's recurrent kernel also takes (any power of two, src/ops/kimi_delta_attention.py:46) or its
// chunk kernels do (multiples of 64, :88, :126), beyond the 64 and 128 of recurrent.hip.  A separate file so the two
// sets of instantiations build in parallel.
#include "recurrent_impl.h"

namespace gdr {

namespace {

template <int VARIANT, int K, typename InT>
hipError_t launch_k(const gdr_args& a, hipStream_t stream, int vs, RecMode mode, const RecExtra& x) {
  if (mode == RecMode::kCommitVerify ? x.prev->h0 != nullptr : a.h0 != nullptr)
    return launch_recurrent_k<VARIANT, K, InT, true>(a, stream, vs, mode, x);
  return launch_recurrent_k<VARIANT, K, InT, false>(a, stream, vs, mode, x);
}

template <int VARIANT, typename InT>
hipError_t launch_v(const gdr_args& a, hipStream_t stream, int vs, RecMode mode, const RecExtra& x) {
  switch (a.key_dim) {
    case 32: return launch_k<VARIANT, 32, InT>(a, stream, vs, mode, x);
    case 192: return launch_k<VARIANT, 192, InT>(a, stream, vs, mode, x);
    default: return launch_k<VARIANT, 256, InT>(a, stream, vs, mode, x);
  }
}

template <typename InT>
hipError_t launch_t(const gdr_args& a, hipStream_t stream, int vs, RecMode mode, const RecExtra& x) {
  switch (a.variant) {
    case GDR_KDA: return launch_v<GDR_KDA, InT>(a, stream, vs, mode, x);
    case GDR_GDN: return launch_v<GDR_GDN, InT>(a, stream, vs, mode, x);
    case GDR_GLA: return launch_v<GDR_GLA, InT>(a, stream, vs, mode, x);
    default: return launch_v<GDR_DELTANET, InT>(a, stream, vs, mode, x);
  }
}

}  // namespace

hipError_t launch_recurrent_other_k(const gdr_args& a, hipStream_t stream, int vs, RecMode mode, const RecExtra& x,
                                    int dtype) {
  return dtype == GDR_BF16 ? launch_t<__bf16>(a, stream, vs, mode, x) : launch_t<float>(a, stream, vs, mode, x);
}

}  // namespace gdr
