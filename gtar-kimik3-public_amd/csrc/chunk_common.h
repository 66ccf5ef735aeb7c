// Device helpers shared by the chunkwise kernels: MFMA wrappers, bf16 packing, the transposing LDS read, the
// causal tile indexing of a 64-token chunk and the exact elementwise evaluation of "hot" diagonal blocks.
#pragma once

#include "gdr_common.h"

namespace gdr {
namespace chunk {

constexpr int kChunk = 64;      // tokens per chunk
constexpr float kHotSpan = 60.f;  // a channel whose 16-row decay span exceeds this is handled elementwise

__device__ __forceinline__ floatx4 mfma32(bf16x8 a, bf16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mfma16(bf16x4 a, bf16x4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ __bf16 bf(float x) { return static_cast<__bf16>(x); }
__device__ __forceinline__ float f32(__bf16 x) { return static_cast<float>(x); }
__device__ __forceinline__ bf16x4 pack4(floatx4 v) { return bf16x4{bf(v[0]), bf(v[1]), bf(v[2]), bf(v[3])}; }
__device__ __forceinline__ bf16x8 concat(bf16x4 lo, bf16x4 hi) {
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
__device__ __forceinline__ void unpack8(uint4 raw, float* out) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ int tri_tile(int i, int j) { return i * (i + 1) / 2 + j; }  // j <= i
__device__ __forceinline__ int strict_tile(int i, int j) { return i * (i - 1) / 2 + j; }  // j < i

// Transposing LDS read of four bf16 (ds_read_b64_tr_b16): within each 16-lane group, lane c slot r receives
// element c % 4 of the 8 bytes addressed by lane 4 r + c / 4 of the group.
__device__ __forceinline__ bf16x4 lds_read_tr(const unsigned char* smem, int byte_off) {
  typedef short short4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) short4_t lds_short4;
  const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_short4*)((__attribute__((address_space(3))) const unsigned char*)smem + byte_off));
  return __builtin_bit_cast(bf16x4, v);
}

// Workgroup barrier that orders LDS only: global stores issued before it are not waited for (a full
// __syncthreads() also drains outstanding global memory operations).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

constexpr float kLog2e = 1.4426950408889634f;

// Per-workgroup view of the problem: base pointers already offset to (sequence, head), strides, lengths.
struct ChunkCtx {
  const __bf16* qp;
  const __bf16* kp;
  const __bf16* vp;
  const float* gp;
  const float* betap;
  void* op;
  int64_t q_st, k_st, v_st, g_st, b_st, o_st;
  int len, nchunks, v0, V;
  size_t sbase;
  const float* h0;
  float* ht;
  float scale;
};

// Exact evaluation of the diagonal 16x16 block of the gated scores and kernel matrix for the channels of this
// lane whose in-block decay span is too large for the block-start factorisation (bit c of hot_mask <-> channel
// c0 + c).  Re-reads the block's q, k and gate rows (L2-resident), rebuilds the in-block cumulative gate and adds
//   Sc(t, s) += sum_{hot c} q_tc k_sc e^{b_tc - b_sc}   (t >= s),   L(t, s) += beta_t sum_{hot c} k_tc k_sc e^{...}  (t > s)
// to the tiles the MFMA pass produced with zero key operands for those channels.
template <int K, bool kDelta, int kGate, int CH0>
__device__ __forceinline__ void hot_diag_fixup(const ChunkCtx& x, int chunk_row0, int pw, uint32_t hot_mask,
                                               __bf16* sc_tile, float* lii_tile, const float* beta_rows) {
  // one pass over the 4 channels c0 + CH0 .. c0 + CH0 + 3 of this lane (two passes keep the live data small)
  constexpr int LPR = K / 8, RSG = kWave / LPR, RPL = 16 / RSG, NC = 4;
  const int lane = threadIdx.x & 63;
  const int cg = lane % LPR, rs = lane / LPR, c0 = 8 * cg + CH0;
  float hq[RPL][NC], hk[RPL][NC], hb[RPL][NC];
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    const int t = chunk_row0 + 16 * pw + rs * RPL + j;
    const int tc = min(t, x.len - 1);
    const bool ok = t < x.len;
    const uint2 qv = *reinterpret_cast<const uint2*>(x.qp + tc * x.q_st + c0);
    const uint2 kv = *reinterpret_cast<const uint2*>(x.kp + tc * x.k_st + c0);
    const uint32_t qw[2] = {qv.x, qv.y}, kw[2] = {kv.x, kv.y};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float qe = __uint_as_float((c & 1) ? (qw[c >> 1] & 0xffff0000u) : (qw[c >> 1] << 16));
      const float ke = __uint_as_float((c & 1) ? (kw[c >> 1] & 0xffff0000u) : (kw[c >> 1] << 16));
      const float g = kGate == 2 ? x.gp[tc * x.g_st + c0 + c] : x.gp[tc * x.g_st];
      hq[j][c] = ok ? qe : 0.f;
      hk[j][c] = ok ? ke : 0.f;
      hb[j][c] = ok ? g * kLog2e : 0.f;
    }
  }
#pragma unroll
  for (int j = 1; j < RPL; ++j)
#pragma unroll
    for (int c = 0; c < NC; ++c) hb[j][c] += hb[j - 1][c];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const float own = hb[RPL - 1][c];
    float incl = own;
#pragma unroll
    for (int off = LPR; off < kWave; off *= 2) {
      const float y = __shfl_up(incl, off, kWave);
      if (lane >= off) incl += y;
    }
#pragma unroll
    for (int j = 0; j < RPL; ++j) hb[j][c] += incl - own;
  }
#pragma unroll 1
  for (int sr = 0; sr < 16; ++sr) {
    const int src = cg + LPR * (sr / RPL);
    const int js = sr % RPL;
    float pa[RPL], sa[RPL];
#pragma unroll
    for (int j = 0; j < RPL; ++j) pa[j] = sa[j] = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float kv = 0.f, bv = 0.f;
#pragma unroll
      for (int jj = 0; jj < RPL; ++jj) {
        if (jj == js) {
          kv = hk[jj][c];
          bv = hb[jj][c];
        }
      }
      const float ks = __shfl(kv, src, kWave), bs = __shfl(bv, src, kWave);
      if (hot_mask & (1u << (CH0 + c))) {
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
          const float d = ks * __builtin_amdgcn_exp2f(fminf(hb[j][c] - bs, 0.f));
          pa[j] += hk[j][c] * d;
          sa[j] += hq[j][c] * d;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < RPL; ++j) {
#pragma unroll
      for (int m = 1; m < LPR; m *= 2) {
        pa[j] += shfl_xor(pa[j], m);
        sa[j] += shfl_xor(sa[j], m);
      }
      const int t = rs * RPL + j;
      if (cg == 0 && t >= sr) {
        __bf16* dst = sc_tile + t * 16 + sr;
        *dst = bf(f32(*dst) + sa[j]);
        if (kDelta && t > sr) lii_tile[t * 16 + sr] += beta_rows[t] * pa[j];
      }
    }
  }
}

}  // namespace chunk
}  // namespace gdr
