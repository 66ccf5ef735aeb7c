// Output epilogue of the KDA layer (src/layers/kimi_delta_attention.py:58-59 with RMSNorm src/layers/rmsnorm.py:11-16):
//
//   out = weight * round_x(x * rsqrt(mean(x^2) + eps)) * round_x(silu(gate))
//
// over each (token, head) row of V values, in one HBM-bound pass.  Sixteen lanes hold a row (V / 16 consecutive
// values each, moved with 8- or 16-byte accesses); a thread keeps kIter rows in flight, so a 256-thread block covers
// 16 kIter rows.  The row's sum of squares is a 16-lane reduction in fp32.  The roundings follow PyTorch's evaluation
// of the layer: the normalised row is cast back to x's dtype before the weight multiplies it, silu(gate) is produced
// in gate's dtype, and both products are taken in out's dtype (fp32 when the weight is fp32, by type promotion;
// otherwise x's dtype, rounded after each product).
#include <type_traits>

#include "gdr_common.h"
#include "gdr_internal.h"

namespace gdr {
namespace {

constexpr float kLog2eF = 1.4426950408889634f;
constexpr int kIter = 4;  // rows in flight per thread

template <typename T>
__device__ __forceinline__ float to_f(T v) { return static_cast<float>(v); }

// EPL values of type T as whole 16-byte (or, when the size is not a multiple of 16, 8-byte) words.
template <typename T, int EPL>
struct Lane {
  static constexpr int kBytes = EPL * int(sizeof(T));
  using Word = typename std::conditional<kBytes % 16 == 0, uint4, uint2>::type;
  static constexpr int kWords = kBytes / int(sizeof(Word));
  Word w[kWords];
  __device__ __forceinline__ void load(const T* p) {
#pragma unroll
    for (int i = 0; i < kWords; ++i) w[i] = reinterpret_cast<const Word*>(p)[i];
  }
  __device__ __forceinline__ void store(T* p) const {
#pragma unroll
    for (int i = 0; i < kWords; ++i) reinterpret_cast<Word*>(p)[i] = w[i];
  }
  __device__ __forceinline__ T& operator[](int e) { return reinterpret_cast<T*>(w)[e]; }
};

template <typename T, typename WT, int EPL>
__global__ __launch_bounds__(256) void norm_gate_kernel(const gdr_norm_gate_args a, int64_t rows) {
  using OT = typename std::conditional<std::is_same<WT, float>::value, float, T>::type;
  const int sub = threadIdx.x & 15;  // lane within the row's 16
  const int c0 = sub * EPL;
  const int64_t row0 = int64_t(blockIdx.x) * 16 * kIter + (threadIdx.x >> 4);
  Lane<T, EPL> xr[kIter], gr[kIter];
  int64_t xo[kIter], go[kIter], oo[kIter];
#pragma unroll
  for (int it = 0; it < kIter; ++it) {  // row row0 + 16 it (clamped: rows past the end are computed, not stored)
    const uint32_t row = uint32_t(min(row0 + 16 * it, rows - 1));  // rows < 2^31 (checked on the host)
    const uint32_t h = row % uint32_t(a.heads), bt = row / uint32_t(a.heads);
    const uint32_t t = bt % uint32_t(a.seq_len), b = bt / uint32_t(a.seq_len);
    xo[it] = int64_t(b) * a.x.stride_b + int64_t(t) * a.x.stride_t + int64_t(h) * a.x.stride_h + c0;
    go[it] = int64_t(b) * a.gate.stride_b + int64_t(t) * a.gate.stride_t + int64_t(h) * a.gate.stride_h + c0;
    oo[it] = int64_t(b) * a.out.stride_b + int64_t(t) * a.out.stride_t + int64_t(h) * a.out.stride_h + c0;
    xr[it].load(static_cast<const T*>(a.x.ptr) + xo[it]);
    gr[it].load(static_cast<const T*>(a.gate.ptr) + go[it]);
  }
  float wv[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) wv[e] = to_f(static_cast<const WT*>(a.weight)[c0 + e]);
#pragma unroll
  for (int it = 0; it < kIter; ++it) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) ss += to_f(xr[it][e]) * to_f(xr[it][e]);
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) ss = xor_sum(ss, m);  // within the 16-lane row
    const float r = rsqrtf(ss / float(16 * EPL) + a.eps);
    Lane<OT, EPL> o;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const float xv = to_f(xr[it][e]), gv = to_f(gr[it][e]);
      const float n = to_f(static_cast<T>(xv * r));                                        // .to(input_dtype)
      const float sg = to_f(static_cast<T>(gv / (1.f + __builtin_amdgcn_exp2f(-gv * kLog2eF))));  // F.silu
      if constexpr (std::is_same<WT, float>::value) {
        o[e] = (wv[e] * n) * sg;
      } else {
        o[e] = static_cast<OT>(to_f(static_cast<OT>(wv[e] * n)) * sg);
      }
    }
    if (row0 + 16 * it < rows) o.store(static_cast<OT*>(const_cast<void*>(a.out.ptr)) + oo[it]);
  }
}

template <typename T, typename WT>
hipError_t launch_typed(const gdr_norm_gate_args& a, hipStream_t stream) {
  const int64_t rows = int64_t(a.batch) * a.seq_len * a.heads;
  if (rows == 0) return hipSuccess;
  const dim3 grid(unsigned((rows + 16 * kIter - 1) / (16 * kIter)));
  switch (a.value_dim / 64) {
#define GDR_NG_CASE(E) \
  case E: hipLaunchKernelGGL((norm_gate_kernel<T, WT, 4 * E>), grid, dim3(256), 0, stream, a, rows); break;
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
