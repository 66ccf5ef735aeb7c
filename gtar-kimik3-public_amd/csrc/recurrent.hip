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
#include "gdr_common.h"
#include "gdr_internal.h"

namespace gdr {

// The state is read exactly once: a non-temporal load keeps it from displacing reusable lines in the caches
// (measured on MI355X at batch 256: 6.3 TB/s against 5.1 TB/s with plain loads for the same kernel).
__device__ __forceinline__ float4 load_stream4(const float* p) {
  return make_float4(__builtin_nontemporal_load(p), __builtin_nontemporal_load(p + 1),
                     __builtin_nontemporal_load(p + 2), __builtin_nontemporal_load(p + 3));
}

// q, k and v share one element type InT (bf16 or fp32; the host widens mixed or fp16 inputs to fp32, exactly), so
// every load has a static type and the compiler can track each one's completion precisely.
template <int VARIANT, int K, int VS, int kThreads, typename InT, bool kH0>
__global__ __launch_bounds__(kThreads) void recurrent_fwd_kernel(const gdr_args a, int n_slices) {
  constexpr int kWaves = kThreads / kWave;
  constexpr int NQ = VS / 4;           // float4 column quads per state row slice
  constexpr int RG = kThreads / NQ;    // row groups
  constexpr int RPT = K / RG;          // state rows per thread
  static_assert(NQ <= kWave && RPT >= 1 && K % RG == 0, "bad recurrent tiling");
  constexpr bool kDelta = VARIANT != GDR_GLA;
  constexpr bool kChannelGate = VARIANT == GDR_KDA || VARIANT == GDR_GLA;
  constexpr bool kScalarGate = VARIANT == GDR_GDN;

  const int slice = blockIdx.x % n_slices;
  const int bh = blockIdx.x / n_slices;
  const int H = a.heads, V = a.value_dim, T = a.seq_len;
  const int b = bh / H, h = bh % H;
  const int v0 = slice * VS;
  const int tid = threadIdx.x;
  const int quad = tid % NQ, rg = tid / NQ;
  const int lane = tid % kWave, wave = tid / kWave;
  const int col = v0 + 4 * quad;

  __shared__ float s_q[K], s_k[K], s_eg[K];
  __shared__ float s_v[VS];
  __shared__ float s_red[kWaves][2][VS];
  __shared__ float s_scalar[2];  // beta, scalar decay
  __shared__ float s_qk;

  // Uniform (b, h) base pointers plus a 32-bit per-lane offset: one address register per row, not a 64-bit pair.
  const size_t state_base = size_t(bh) * K * V;
  const float* h0 = a.h0 ? a.h0 + state_base : nullptr;
  float* ht = a.ht ? a.ht + state_base : nullptr;
  const uint32_t lane_off = uint32_t(rg) * V + col;

  const int64_t qb = b * a.q.stride_b + h * a.q.stride_h;
  const int64_t kb = b * a.k.stride_b + h * a.k.stride_h;
  const int64_t vb = b * a.v.stride_b + h * a.v.stride_h;
  const int64_t ob = b * a.out.stride_b + h * a.out.stride_h;
  const int64_t gb = b * a.gate.stride_b + h * a.gate.stride_h;
  const int64_t bb = b * a.beta.stride_b + h * a.beta.stride_h;

  // One token's vectors: fetched into registers, then converted and staged in LDS.
  const InT* qp = static_cast<const InT*>(a.q.ptr);
  const InT* kp = static_cast<const InT*>(a.k.ptr);
  const InT* vp = static_cast<const InT*>(a.v.ptr);
  InT raw_q = InT(0.f), raw_k = InT(0.f), raw_v = InT(0.f);
  float raw_g = 0.f, raw_beta = 0.f, raw_sg = 0.f;
  auto fetch = [&](int t) {
    if (tid < K) {  // kThreads >= K
      raw_q = qp[qb + t * a.q.stride_t + tid];
      raw_k = kp[kb + t * a.k.stride_t + tid];
      if constexpr (kChannelGate) raw_g = static_cast<const float*>(a.gate.ptr)[gb + t * a.gate.stride_t + tid];
    }
    if (tid < VS) raw_v = vp[vb + t * a.v.stride_t + v0 + tid];
    if (tid == 0) {
      if constexpr (kDelta) raw_beta = static_cast<const float*>(a.beta.ptr)[bb + t * a.beta.stride_t];
      if constexpr (kScalarGate) raw_sg = static_cast<const float*>(a.gate.ptr)[gb + t * a.gate.stride_t];
    }
  };
  auto stage = [&]() {  // the fetched token's vectors, as fp32, into LDS
    if (tid < K) {
      s_q[tid] = static_cast<float>(raw_q);
      s_k[tid] = static_cast<float>(raw_k);
      if constexpr (kChannelGate) s_eg[tid] = exp_fast(raw_g);
    }
    if (tid < VS) s_v[tid] = static_cast<float>(raw_v);
    if (tid == 0) {
      if constexpr (kDelta) s_scalar[0] = raw_beta;
      if constexpr (kScalarGate) s_scalar[1] = exp_fast(raw_sg);
    }
  };

  // Token 0's vectors are requested before the state stream and staged in straight-line code, so staging waits
  // for them alone while the state loads stay in flight.
  if (T > 0) fetch(0);
  float4 st[RPT];  // (kH0 is a template argument: a run-time branch here would make the wait below conservative)
#pragma unroll
  for (int i = 0; i < RPT; ++i)
    st[i] = kH0 ? load_stream4(h0 + lane_off + uint32_t(RG * i) * V) : make_float4(0.f, 0.f, 0.f, 0.f);
  if (T > 0) stage();

  for (int t = 0; t < T; ++t) {
    __syncthreads();

    // Decay and the two dk-partial reductions in one pass over the register-resident rows.
    float ak[4] = {0.f, 0.f, 0.f, 0.f}, aq[4] = {0.f, 0.f, 0.f, 0.f};
    const float eg_scalar = kScalarGate ? s_scalar[1] : 1.f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int r = rg + RG * i;
      float e = 1.f;
      if constexpr (kChannelGate) e = s_eg[r];
      if constexpr (kScalarGate) e = eg_scalar;
      if constexpr (kChannelGate || kScalarGate) {
        st[i].x *= e; st[i].y *= e; st[i].z *= e; st[i].w *= e;
      }
      const float kr = s_k[r], qr = s_q[r];
      ak[0] += kr * st[i].x; ak[1] += kr * st[i].y; ak[2] += kr * st[i].z; ak[3] += kr * st[i].w;
      aq[0] += qr * st[i].x; aq[1] += qr * st[i].y; aq[2] += qr * st[i].z; aq[3] += qr * st[i].w;
    }
#pragma unroll
    for (int m = NQ; m < kWave; m *= 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ak[j] += shfl_xor(ak[j], m);
        aq[j] += shfl_xor(aq[j], m);
      }
    }
    if (lane < NQ) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s_red[wave][0][4 * quad + j] = ak[j];
        s_red[wave][1][4 * quad + j] = aq[j];
      }
    }
    if (wave == kWaves - 1) {  // q . k for the readout correction
      float p = 0.f;
      for (int c = lane; c < K; c += kWave) p += s_q[c] * s_k[c];
#pragma unroll
      for (int m = 1; m < kWave; m *= 2) p += shfl_xor(p, m);
      if (lane == 0) s_qk = p;
    }
    __syncthreads();

    float kS[4], qS[4], u[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      kS[j] = 0.f;
      qS[j] = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        kS[j] += s_red[w][0][4 * quad + j];
        qS[j] += s_red[w][1][4 * quad + j];
      }
      const float vj = s_v[4 * quad + j];
      u[j] = kDelta ? s_scalar[0] * (vj - kS[j]) : vj;
    }
    if (rg == 0) {
      const float qk = s_qk;
      const int64_t oi = ob + t * a.out.stride_t + col;
#pragma unroll
      for (int j = 0; j < 4; ++j) store_any(const_cast<void*>(a.out.ptr), oi + j, a.out.dtype, a.scale * (qS[j] + qk * u[j]));
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const float kr = s_k[rg + RG * i];
      st[i].x += kr * u[0]; st[i].y += kr * u[1]; st[i].z += kr * u[2]; st[i].w += kr * u[3];
    }
    if (t + 1 < T) {  // LDS is restaged for the next token
      __syncthreads();
      fetch(t + 1);
      stage();
    }
  }

  if (ht) {
#pragma unroll
    for (int i = 0; i < RPT; ++i) *reinterpret_cast<float4*>(ht + lane_off + uint32_t(RG * i) * V) = st[i];
  }
}

template <int VARIANT, int K, typename InT, bool kH0>
static hipError_t launch_recurrent_k(const gdr_args& a, hipStream_t stream, int vs) {
  const int bh = a.batch * a.heads;
  if (vs == 128) {  // 512 threads: 8 state rows x one float4 per thread (K = 128)
    const int n_slices = a.value_dim / 128;
    hipLaunchKernelGGL((recurrent_fwd_kernel<VARIANT, K, 128, 512, InT, kH0>), dim3(bh * n_slices), dim3(512), 0,
                       stream, a, n_slices);
  } else {
    const int n_slices = a.value_dim / 32;
    hipLaunchKernelGGL((recurrent_fwd_kernel<VARIANT, K, 32, 256, InT, kH0>), dim3(bh * n_slices), dim3(256), 0,
                       stream, a, n_slices);
  }
  return hipGetLastError();
}

template <int VARIANT, typename InT>
static hipError_t launch_recurrent_v(const gdr_args& a, hipStream_t stream, int vs) {
  if (a.h0)
    return a.key_dim == 64 ? launch_recurrent_k<VARIANT, 64, InT, true>(a, stream, vs)
                           : launch_recurrent_k<VARIANT, 128, InT, true>(a, stream, vs);
  return a.key_dim == 64 ? launch_recurrent_k<VARIANT, 64, InT, false>(a, stream, vs)
                         : launch_recurrent_k<VARIANT, 128, InT, false>(a, stream, vs);
}

template <typename InT>
static hipError_t launch_recurrent_t(const gdr_args& a, hipStream_t stream, int vs) {
  switch (a.variant) {
    case GDR_KDA: return launch_recurrent_v<GDR_KDA, InT>(a, stream, vs);
    case GDR_GDN: return launch_recurrent_v<GDR_GDN, InT>(a, stream, vs);
    case GDR_GLA: return launch_recurrent_v<GDR_GLA, InT>(a, stream, vs);
    default: return launch_recurrent_v<GDR_DELTANET, InT>(a, stream, vs);
  }
}

hipError_t launch_recurrent(const gdr_args& a, hipStream_t stream) {
  // Wide slices stream the most bytes per workgroup; narrow slices give small batches enough workgroups.
  const long long wide_blocks = (long long)a.batch * a.heads * (a.value_dim / 128);
  const int vs = (a.value_dim % 128 == 0 && wide_blocks >= 1024) ? 128 : 32;
  return a.q.dtype == GDR_BF16 ? launch_recurrent_t<__bf16>(a, stream, vs) : launch_recurrent_t<float>(a, stream, vs);
}

}  // namespace gdr
