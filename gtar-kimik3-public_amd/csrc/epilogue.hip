// Output epilogue of the KDA layer (src/layers/kimi_delta_attention.py:58-59 with RMSNorm src/layers/rmsnorm.py:11-16):
//
//   out = weight * round_x(x * rsqrt(mean(x^2) + eps)) * round_x(silu(gate))
//
// over each (token, head) row of V values, in one HBM-bound pass.  One wave per row: lane l holds the V / 64
// consecutive values l * V / 64 ..; the row's sum of squares is a wave reduction in fp32.  The roundings follow
// PyTorch's evaluation of the layer: the normalised row is cast back to x's dtype before the weight multiplies it,
// silu(gate) is produced in gate's dtype, and both products are taken in out's dtype (fp32 when the weight is fp32,
// by type promotion; otherwise x's dtype, rounded after each product).
#include <type_traits>

#include "gdr_common.h"
#include "gdr_internal.h"

namespace gdr {
namespace {

constexpr float kLog2eF = 1.4426950408889634f;

template <typename T>
__device__ __forceinline__ float to_f(T v) { return static_cast<float>(v); }

template <typename T, typename WT, int EPL>
__global__ __launch_bounds__(256) void norm_gate_kernel(const gdr_norm_gate_args a, int64_t rows) {
  using OT = typename std::conditional<std::is_same<WT, float>::value, float, T>::type;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int h = int(row % a.heads);
  const int64_t bt = row / a.heads;
  const int t = int(bt % a.seq_len), b = int(bt / a.seq_len);
  const int c0 = lane * EPL;
  const T* xp = static_cast<const T*>(a.x.ptr) + b * a.x.stride_b + int64_t(t) * a.x.stride_t + h * a.x.stride_h + c0;
  const T* gp = static_cast<const T*>(a.gate.ptr) + b * a.gate.stride_b + int64_t(t) * a.gate.stride_t +
                h * a.gate.stride_h + c0;
  OT* op = static_cast<OT*>(const_cast<void*>(a.out.ptr)) + b * a.out.stride_b + int64_t(t) * a.out.stride_t +
           h * a.out.stride_h + c0;
  const WT* wp = static_cast<const WT*>(a.weight) + c0;

  float xv[EPL], gv[EPL];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    xv[e] = to_f(xp[e]);
    gv[e] = to_f(gp[e]);
    ss += xv[e] * xv[e];
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, kWave);
  const float r = rsqrtf(ss / float(EPL * 64) + a.eps);
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const float n = to_f(static_cast<T>(xv[e] * r));                                           // .to(input_dtype)
    const float s = to_f(static_cast<T>(gv[e] / (1.f + __builtin_amdgcn_exp2f(-gv[e] * kLog2eF))));  // F.silu
    if constexpr (std::is_same<WT, float>::value) {
      op[e] = (wp[e] * n) * s;
    } else {
      op[e] = static_cast<OT>(to_f(static_cast<OT>(to_f(wp[e]) * n)) * s);
    }
  }
}

template <typename T, typename WT>
hipError_t launch_typed(const gdr_norm_gate_args& a, hipStream_t stream) {
  const int64_t rows = int64_t(a.batch) * a.seq_len * a.heads;
  if (rows == 0) return hipSuccess;
  const dim3 grid(unsigned((rows + 3) / 4));
  switch (a.value_dim / 64) {
#define GDR_NG_CASE(E) \
  case E: hipLaunchKernelGGL((norm_gate_kernel<T, WT, E>), grid, dim3(256), 0, stream, a, rows); break;
    GDR_NG_CASE(1) GDR_NG_CASE(2) GDR_NG_CASE(3) GDR_NG_CASE(4)
#undef GDR_NG_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T>
hipError_t launch_weight(const gdr_norm_gate_args& a, hipStream_t stream) {
  return a.weight_dtype == GDR_F32 ? launch_typed<T, float>(a, stream) : launch_typed<T, T>(a, stream);
}

}  // namespace

hipError_t launch_norm_gate(const gdr_norm_gate_args& a, hipStream_t stream) {
  switch (a.x.dtype) {
    case GDR_BF16: return launch_weight<__bf16>(a, stream);
    case GDR_F16: return launch_weight<_Float16>(a, stream);
    default: return launch_typed<float, float>(a, stream);
  }
}

}  // namespace gdr
