// Device helpers shared by the chunkwise kernels: MFMA wrappers, bf16 packing, the transposing LDS read, the
// causal tile indexing of a 64-token chunk and the exact elementwise evaluation of "hot" diagonal blocks.
#pragma once

#include "gdr_common.h"

namespace gdr {
namespace chunk {

constexpr int kChunk = 64;      // tokens per chunk
constexpr float kHotSpan = 60.f;  // a channel whose 16-row decay span exceeds this is handled elementwise

typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 f16x4;

// MFMA operand vectors of the two 16-bit operand types (bf16 for bf16 inputs, f16 for f16 inputs).
template <typename T> struct OpVec;
template <> struct OpVec<__bf16> { using v8 = bf16x8; using v4 = bf16x4; };
template <> struct OpVec<_Float16> { using v8 = f16x8; using v4 = f16x4; };
template <typename T> using vec8 = typename OpVec<T>::v8;
template <typename T> using vec4 = typename OpVec<T>::v4;

__device__ __forceinline__ floatx4 mfma32(bf16x8 a, bf16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mfma16(bf16x4 a, bf16x4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mfma32(f16x8 a, f16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mfma16(f16x4 a, f16x4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ __bf16 bf(float x) { return static_cast<__bf16>(x); }
template <typename T>
__device__ __forceinline__ T cv(float x) { return static_cast<T>(x); }  // round to the operand type
__device__ __forceinline__ float f32(__bf16 x) { return static_cast<float>(x); }
__device__ __forceinline__ float f32(_Float16 x) { return static_cast<float>(x); }
template <typename T = __bf16>
__device__ __forceinline__ vec4<T> pack4(floatx4 v) { return vec4<T>{cv<T>(v[0]), cv<T>(v[1]), cv<T>(v[2]), cv<T>(v[3])}; }
__device__ __forceinline__ bf16x8 concat(bf16x4 lo, bf16x4 hi) {
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
__device__ __forceinline__ f16x8 concat(f16x4 lo, f16x4 hi) {
  return f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
// Eight 16-bit values (16 bytes) of type T to fp32 (exact).
template <typename T = __bf16>
__device__ __forceinline__ void unpack8(uint4 raw, float* out) {
  if constexpr (__is_same(T, __bf16)) {
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __uint_as_float(w[i] << 16);
      out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
    const f16x8 h = __builtin_bit_cast(f16x8, raw);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = static_cast<float>(h[i]);
  }
}

__device__ __forceinline__ int tri_tile(int i, int j) { return i * (i + 1) / 2 + j; }  // j <= i
__device__ __forceinline__ int strict_tile(int i, int j) { return i * (i - 1) / 2 + j; }  // j < i

// Transposing LDS read of four bf16 (ds_read_b64_tr_b16): within each 16-lane group, lane c slot r receives
// element c % 4 of the 8 bytes addressed by lane 4 r + c / 4 of the group.
template <typename T = __bf16>
__device__ __forceinline__ vec4<T> lds_read_tr(const unsigned char* smem, int byte_off) {
  typedef short short4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) short4_t lds_short4;
  const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_short4*)((__attribute__((address_space(3))) const unsigned char*)smem + byte_off));
  return __builtin_bit_cast(vec4<T>, v);
}

// 16 bytes from global memory straight into LDS (global_load_lds_dwordx4): lane i's bytes land at the wave-uniform
// LDS address `lds_base` + 16 i.
__device__ __forceinline__ void lds_dma16(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_base, 16, 0, 0);
}

// Non-temporal (`nt`) 16-byte accesses.  The prefill's records, written by the prep and read back by the scan,
// come from the memory-side cache when they are still in it; for calls where that pays, input rows that no other
// workgroup reads and outputs that the call does not read back are loaded and stored with the hint, so that they
// do not displace the records.  `load_nt16` is a global load whose form is fixed at compile time (the kernels that
// use it are instantiated with and without the hint: two global loads of one address that differ only in the hint
// would be merged into one plain load).  `store_nt16` is a raw buffer store with the `nt` cache-policy bit, a
// different instruction from the plain global store, so a kernel can choose between the two at run time; its
// base is wave-uniform and the byte offset must satisfy off + 16 <= 2^32.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
template <typename R>
__device__ __forceinline__ R load_nt16(const void* p) {
  static_assert(sizeof(R) == 16, "16-byte vector");
  return __builtin_bit_cast(R, __builtin_nontemporal_load(static_cast<const u32x4*>(p)));
}
template <typename V>
__device__ __forceinline__ void store_nt16(void* base, uint32_t off, const V& v) {
  static_assert(sizeof(V) == 16, "16-byte vector");
  constexpr int kCachePolicyNT = 2;  // the `nt` bit of a buffer access's cache-policy operand
  // raw buffer (stride 0) over the 4 GiB from base, held in scalar registers (base is wave-uniform); third dword
  // 0x00020000: the 32-bit data format gfx9 expects
  // (readfirstlane returns a signed int: each half goes through uint32_t so that it is zero-extended)
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(b))));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(b >> 32))));
  void* ub = reinterpret_cast<void*>(uint64_t(lo) | (uint64_t(hi) << 32));
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(ub, 0, -1, 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rsrc, off, 0, kCachePolicyNT);
}

// Workgroup barrier that orders LDS only: global stores issued before it are not waited for (a full
// __syncthreads() also drains outstanding global memory operations).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Per-workgroup view of the problem: base pointers already offset to (sequence, head), strides, lengths.  T is the
// element type of q, k, v.
template <typename T>
struct ChunkCtxT {
  const T* qp;
  const T* kp;
  const T* vp;
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
using ChunkCtx = ChunkCtxT<__bf16>;

// Inclusive prefix sum over the 16 lanes of each DPP row (v_add_f32 with row_shr:1, 2, 4, 8; lanes shifted in from
// outside the row contribute 0).
__device__ __forceinline__ float row_scan16(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x111, 0xf, 0xf, true));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x112, 0xf, 0xf, true));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x114, 0xf, 0xf, true));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x118, 0xf, 0xf, true));
  return x;
}

// Cross-lane moves on the VALU (DPP and the gfx950 permlane swaps) instead of ds_bpermute round trips through LDS.
// dpp_row<CTRL>: one DPP move within each 16-lane row (CTRL is the dpp_ctrl code, every lane of the row valid).
template <int CTRL>
__device__ __forceinline__ float dpp_row(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
// Lane N of each 16-lane row, in every lane of that row (row_newbcast).
template <int N>
__device__ __forceinline__ float row_lane(float x) {
  return dpp_row<0x150 + N>(x);
}
// Sum over the 16 lanes of each row (quad_perm [1,0,3,2] and [2,3,0,1], then the row rotated by 4 and by 8).  Every
// lane of the row ends with the sum, but the association differs between its quads, so callers use one lane's.
__device__ __forceinline__ float row_sum16(float x) {
  x += dpp_row<0xB1>(x);
  x += dpp_row<0x4E>(x);
  x += dpp_row<0x124>(x);
  x += dpp_row<0x128>(x);
  return x;
}
// Row R (lanes 16 R .. 16 R + 15) in every row, lane l reading lane 16 R + l % 16: v_permlane32_swap of two copies
// gives the lower half's rows (first result) or the upper half's (second) in both halves, and v_permlane16_swap of
// two copies of that gives its even row (first) or odd row (second) in every row.
template <int R>
__device__ __forceinline__ float from_row(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const unsigned h = R < 2 ? a[0] : a[1];
  const auto b = __builtin_amdgcn_permlane16_swap(h, h, false, false);
  return __uint_as_float((R & 1) ? b[1] : b[0]);
}
// Per lane l16 of the four 16-lane rows g = lane / 16: the inclusive prefix (rows g' <= g) or suffix (rows g' >= g) of
// x over the rows, and the total of the four, in every lane: the row pairs (0, 1) and (2, 3) are combined with a
// permlane16 swap, then the two pair sums with a permlane32 swap.
__device__ __forceinline__ float rows_scan(float x, bool suffix, float& total) {
  const int g = (threadIdx.x & 63) >> 4;
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float pair = __uint_as_float(p[0]) + __uint_as_float(p[1]);  // rows 0, 1: x0 + x1; rows 2, 3: x2 + x3
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(pair), __float_as_uint(pair), false, false);
  const float lo = __uint_as_float(q[0]), hi = __uint_as_float(q[1]);  // x0 + x1 and x2 + x3, in every lane
  total = lo + hi;
  if (suffix) return ((g & 1) ? x : pair) + (g < 2 ? hi : 0.f);
  return ((g & 1) ? pair : x) + (g >= 2 ? lo : 0.f);
}

// One channel of one row of the op's inputs, for the hot-channel fix-up: q, k (element type T) and the gate (per channel for
// KDA / GLA, per token for GDN).
template <typename T>
struct InputRowsT {
  const ChunkCtxT<T>& x;
  int gate_mode;  // 2: per-channel gate, 1: scalar gate
  __device__ __forceinline__ void operator()(int tc, int ch, float& q, float& k, float& g) const {
    q = static_cast<float>(x.qp[tc * x.q_st + ch]);
    k = static_cast<float>(x.kp[tc * x.k_st + ch]);
    g = gate_mode == 2 ? x.gp[tc * x.g_st + ch] : x.gp[tc * x.g_st];
  }
};
using InputRows = InputRowsT<__bf16>;

// Exact evaluation of the diagonal 16x16 block of the gated scores and kernel matrix for the channels whose
// in-block decay span is too large for the block-start factorisation (hot channels; the MFMA pass gave them zero key
// operands).  Hot channels are rare and usually few per block, so they are taken one at a time: lanes 0..15 hold
// the 16 rows' q, k and gate of the channel and form its in-block cumulative log2 gate b with a DPP row scan, and
// lane L adds the channel's share to the four entries (t, s) = (L / 4, 4 (L % 4) + i):
//   Sc(t, s) += q_t k_s e^{b_t - b_s}  (t >= s),    L(t, s) += beta_t k_t k_s e^{b_t - b_s}  (t > s).
// hot_mask: on lanes with lane % (K / 8) == grp, bit m marks channel 8 grp + m.  `fetch(tc, ch, q, k, g)` is called
// by all 64 lanes (wave-uniform channel ch, tc the clamped token of row lane % 16) and returns that row's q, k and
// gate (natural-log units) for channel ch.
template <int K, bool kDelta, typename T, typename Fetch>
__device__ __forceinline__ void hot_diag_fixup(int chunk_row0, int pw, int len, uint32_t hot_mask, T* sc_tile,
                                               float* lii_tile, const float* beta_rows, const Fetch& fetch) {
  constexpr int LPR = K / 8;
  const int lane = threadIdx.x & 63;
  const int t_seq = chunk_row0 + 16 * pw + (lane & 15);
  const int tc = min(t_seq, len - 1);
  const bool ok = t_seq < len;
  const int tt = lane >> 2, s0 = 4 * (lane & 3);
  float sc_acc[4] = {0.f, 0.f, 0.f, 0.f}, p_acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int grp = 0; grp < LPR; ++grp) {
    uint32_t m = __shfl(hot_mask, grp, kWave);  // wave-uniform
    while (m) {
      const int ch = 8 * grp + __builtin_ctz(m);
      m &= m - 1;
      float q, k, g;
      fetch(tc, ch, q, k, g);
      if (!ok) q = k = g = 0.f;
      const float b = row_scan16(g * kLog2e);
      const float qt = __shfl(q, tt, kWave), kt = __shfl(k, tt, kWave), bt = __shfl(b, tt, kWave);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int sr = s0 + i;
        const float ks = __shfl(k, sr, kWave), bs = __shfl(b, sr, kWave);
        const float d = ks * __builtin_amdgcn_exp2f(fminf(bt - bs, 0.f));
        if (tt >= sr) sc_acc[i] += qt * d;
        if (kDelta && tt > sr) p_acc[i] += kt * d;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int sr = s0 + i;
    if (tt >= sr) {
      T* dst = sc_tile + tt * 16 + sr;
      *dst = cv<T>(f32(*dst) + sc_acc[i]);
    }
    if (kDelta && tt > sr) lii_tile[tt * 16 + sr] += beta_rows[tt] * p_acc[i];
  }
}

}  // namespace chunk
}  // namespace gdr
