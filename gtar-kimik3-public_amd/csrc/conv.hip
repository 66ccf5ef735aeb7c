// Segment-aware depthwise causal convolution + SiLU (the layers' ShortConvolution, src/layers/short_convolution.py:
// 11-20) on gfx950.
//
//   out[t, c] = silu(sum_{j < W} w[c, j] x[t - W + 1 + j, c])
//
// where an input position before the first token of t's sequence comes from that sequence's conv state (the W - 1
// inputs that preceded it; zero without one) and never from the previous packed sequence.  One thread produces 16
// bytes of channels for kConvTok consecutive tokens: inside a sequence it loads the W - 1 + kConvTok input rows
// once, the W taps of its channels with W 16-byte loads, accumulates in fp32 in tap order and stores each output
// once; a tile at a sequence's start or end goes token by token.  HBM-bound: x read about once (neighbouring
// threads' overlapping rows hit L2), out written once.
#include "gdr_common.h"
#include "varlen_index.h"
#include "gdr_internal.h"

namespace gdr {
namespace {

template <typename T>
__device__ __forceinline__ float to_f32(T x) { return static_cast<float>(x); }

// Sequence of packed token t (largest n with cu[n] <= t).
__device__ __forceinline__ int seq_of(const int32_t* cu, int n_seqs, int t) {
  int lo = 0, hi = n_seqs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

constexpr int kConvTok = 8;  // consecutive tokens per thread: the W - 1 shared input rows are loaded once

__device__ __forceinline__ float silu_or_not(float acc, bool silu) {
  return silu ? silu_rcp(acc) : acc;
}

template <typename T, int W>
__global__ __launch_bounds__(256) void short_conv_kernel(const gdr_conv_args a, int64_t n_items) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int ROWS = W - 1 + kConvTok;
  // Workgroup b runs on XCD b mod 8; XCD x takes the consecutive logical blocks [x per + min(x, rem), ...), so a
  // tile's W - 1 halo rows, loaded by the previous tile's workgroup, are found in the same L2.
  const unsigned per = gridDim.x / 8, rem = gridDim.x % 8, xcd = blockIdx.x % 8;
  const unsigned lblock = xcd * per + min(xcd, rem) + blockIdx.x / 8;
  const int64_t item = int64_t(lblock) * 256 + threadIdx.x;
  if (item >= n_items) return;
  const int C = a.channels, groups = C / VEC;
  const int c0 = int(item % groups) * VEC;
  const int64_t tile = item / groups;  // kConvTok tokens of one row
  const int per_row = (a.seq_len + kConvTok - 1) / kConvTok;
  const int b = a.cu_seqlens ? 0 : int(tile / per_row);
  const int t0 = int(tile % per_row) * kConvTok;
  const T* xp = static_cast<const T*>(a.x.ptr) + b * a.x.stride_b;
  const T* sin = static_cast<const T*>(a.state_in);
  T* op = static_cast<T*>(const_cast<void*>(a.out.ptr)) + b * a.out.stride_b;
  auto row16 = [&](int p) { return *reinterpret_cast<const uint4*>(xp + int64_t(p) * a.x.stride_t + c0); };

  // the W taps of this thread's VEC channels: VEC * W contiguous values, W 16-byte loads
  T wv[VEC * W];
#pragma unroll
  for (int j = 0; j < W; ++j)
    *reinterpret_cast<uint4*>(wv + VEC * j) =
        *reinterpret_cast<const uint4*>(static_cast<const T*>(a.weight) + size_t(c0) * W + VEC * j);

  int n = b, bos = 0, end = a.seq_len;
  if (a.cu_seqlens) {
    n = seq_of(a.cu_seqlens, a.n_seqs, t0);
    bos = packed_begin(a.cu_seqlens, n, a.seq_len);
    end = packed_end(a.cu_seqlens, n, a.seq_len);
  }

  // Interior tiles (every input row inside this thread's sequence, every token before its end, and no token whose
  // input row belongs to the state written after the sequence): the input rows t0 - W + 1 .. t0 + kConvTok - 1 are
  // loaded once and every index into them is a compile-time constant.
  if (t0 - (W - 1) >= bos && t0 + kConvTok <= end && !(a.state_out && t0 + kConvTok > end - (W - 1))) {
    T xr[ROWS][VEC];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) *reinterpret_cast<uint4*>(xr[r]) = row16(t0 - (W - 1) + r);
#pragma unroll
    for (int k = 0; k < kConvTok; ++k) {
      T ov[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < W; ++j) acc += to_f32(wv[e * W + j]) * to_f32(xr[k + j][e]);
        ov[e] = static_cast<T>(silu_or_not(acc, a.apply_silu));
      }
      *reinterpret_cast<uint4*>(op + int64_t(t0 + k) * a.out.stride_t + c0) = *reinterpret_cast<const uint4*>(ov);
    }
    return;
  }

  // Tiles at a sequence's start or end, or past the last token: token by token, each input row loaded where it is
  // used (rows before the sequence come from its conv state, or are zero).
  for (int k = 0; k < kConvTok; ++k) {
    const int t = t0 + k;
    if (t >= a.seq_len) break;
    while (t >= end && n + 1 < a.n_seqs) {  // the next packed sequence starts inside this thread's tokens
      ++n;
      bos = packed_begin(a.cu_seqlens, n, a.seq_len);
      end = packed_end(a.cu_seqlens, n, a.seq_len);
    }
    // past the last sequence's end, or before this sequence's start (offsets that break the contract): nothing to do
    if (t >= end || t < bos) break;
    const size_t state_row = size_t(n) * C;  // [N, C, W - 1]
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
    T cur[VEC];  // input row t (the last tap's)
#pragma unroll
    for (int j = 0; j < W; ++j) {
      const int p = t - (W - 1) + j;
      T xv[VEC];
      if (p >= bos) {
        *reinterpret_cast<uint4*>(xv) = row16(p);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          xv[e] = sin ? sin[(state_row + c0 + e) * (W - 1) + (W - 1) - (bos - p)] : T(0.f);
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] += to_f32(wv[e * W + j]) * to_f32(xv[e]);
      if (j == W - 1) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) cur[e] = xv[e];
      }
    }
    T ov[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) ov[e] = static_cast<T>(silu_or_not(acc[e], a.apply_silu));
    *reinterpret_cast<uint4*>(op + int64_t(t) * a.out.stride_t + c0) = *reinterpret_cast<const uint4*>(ov);

    // The state after the sequence: its last W - 1 inputs, reaching back into state_in when it is shorter.
    if (a.state_out) {
      T* sout = static_cast<T*>(a.state_out);
      const int len = end - bos;
      if (t >= end - (W - 1)) {
        const int slot = (W - 1) - (end - t);
#pragma unroll
        for (int e = 0; e < VEC; ++e) sout[(state_row + c0 + e) * (W - 1) + slot] = cur[e];
      }
      if (t == bos) {
        for (int slot = 0; slot < (W - 1) - len; ++slot)
#pragma unroll
          for (int e = 0; e < VEC; ++e)
            sout[(state_row + c0 + e) * (W - 1) + slot] =
                sin ? sin[(state_row + c0 + e) * (W - 1) + slot + len] : T(0.f);
      }
    }
  }
}

template <typename T>
hipError_t launch_conv_typed(const gdr_conv_args& a, hipStream_t stream) {
  const int64_t tiles = int64_t(a.cu_seqlens ? 1 : a.batch) * ((a.seq_len + kConvTok - 1) / kConvTok);
  const int64_t items = tiles * (a.channels / (16 / int(sizeof(T))));
  if (items == 0) return hipSuccess;
  const dim3 grid(unsigned((items + 255) / 256));
  switch (a.kernel_size) {
#define GDR_CONV_CASE(W) \
  case W: hipLaunchKernelGGL((short_conv_kernel<T, W>), grid, dim3(256), 0, stream, a, items); break;
    GDR_CONV_CASE(2) GDR_CONV_CASE(3) GDR_CONV_CASE(4) GDR_CONV_CASE(5) GDR_CONV_CASE(6) GDR_CONV_CASE(7)
    GDR_CONV_CASE(8)
#undef GDR_CONV_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_short_conv(const gdr_conv_args& a, hipStream_t stream) {
  switch (a.x.dtype) {
    case GDR_BF16: return launch_conv_typed<__bf16>(a, stream);
    case GDR_F16: return launch_conv_typed<_Float16>(a, stream);
    default: return launch_conv_typed<float>(a, stream);
  }
}

}  // namespace gdr
