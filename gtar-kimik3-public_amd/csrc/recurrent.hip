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
// so the kernel is HBM-bound at T = 1.  One workgroup of 256 threads owns a [K, VS] column slice of one
// (b, h) state; thread (quad, rg) holds float4 column quad `quad` of rows rg, rg + RG, ... in registers for the
// whole call.  Both dk-reductions (k S and q S) come out of one pass over the registers, are reduced across
// lanes with DPP/shuffles and across the four waves through LDS, and the rank-1 update is applied in place in
// registers before the single store.  Only the tiny per-token vectors go through LDS.
#include "gdr_common.h"
#include "gdr_internal.h"

namespace gdr {

template <int VARIANT, int K, int VS>
__global__ __launch_bounds__(256) void recurrent_fwd_kernel(const gdr_args a, int n_slices) {
  constexpr int kThreads = 256;
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

  const size_t state_base = size_t(bh) * K * V;
  float4 st[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int r = rg + RG * i;
    st[i] = a.h0 ? *reinterpret_cast<const float4*>(a.h0 + state_base + size_t(r) * V + col)
                 : make_float4(0.f, 0.f, 0.f, 0.f);
  }

  const int64_t qb = b * a.q.stride_b + h * a.q.stride_h;
  const int64_t kb = b * a.k.stride_b + h * a.k.stride_h;
  const int64_t vb = b * a.v.stride_b + h * a.v.stride_h;
  const int64_t ob = b * a.out.stride_b + h * a.out.stride_h;
  const int64_t gb = b * a.gate.stride_b + h * a.gate.stride_h;
  const int64_t bb = b * a.beta.stride_b + h * a.beta.stride_h;

  for (int t = 0; t < T; ++t) {
    // Stage the token's vectors (fp32) in LDS.
    if (tid < K) {
      s_q[tid] = load_any(a.q.ptr, qb + t * a.q.stride_t + tid, a.q.dtype);
      s_k[tid] = load_any(a.k.ptr, kb + t * a.k.stride_t + tid, a.k.dtype);
      if constexpr (kChannelGate)
        s_eg[tid] = exp_fast(static_cast<const float*>(a.gate.ptr)[gb + t * a.gate.stride_t + tid]);
    }
    if (tid < VS) s_v[tid] = load_any(a.v.ptr, vb + t * a.v.stride_t + v0 + tid, a.v.dtype);
    if (tid == 0) {
      if constexpr (kDelta) s_scalar[0] = static_cast<const float*>(a.beta.ptr)[bb + t * a.beta.stride_t];
      if constexpr (kScalarGate)
        s_scalar[1] = exp_fast(static_cast<const float*>(a.gate.ptr)[gb + t * a.gate.stride_t]);
    }
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
    if (t + 1 < T) __syncthreads();  // LDS is restaged for the next token
  }

  if (a.ht) {
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int r = rg + RG * i;
      *reinterpret_cast<float4*>(a.ht + state_base + size_t(r) * V + col) = st[i];
    }
  }
}

template <int VARIANT, int K>
static hipError_t launch_recurrent_k(const gdr_args& a, hipStream_t stream, int vs) {
  const int bh = a.batch * a.heads;
  if (vs == 128) {
    const int n_slices = a.value_dim / 128;
    hipLaunchKernelGGL((recurrent_fwd_kernel<VARIANT, K, 128>), dim3(bh * n_slices), dim3(256), 0, stream, a,
                       n_slices);
  } else {
    const int n_slices = a.value_dim / 32;
    hipLaunchKernelGGL((recurrent_fwd_kernel<VARIANT, K, 32>), dim3(bh * n_slices), dim3(256), 0, stream, a,
                       n_slices);
  }
  return hipGetLastError();
}

template <int VARIANT>
static hipError_t launch_recurrent_v(const gdr_args& a, hipStream_t stream, int vs) {
  return a.key_dim == 64 ? launch_recurrent_k<VARIANT, 64>(a, stream, vs)
                         : launch_recurrent_k<VARIANT, 128>(a, stream, vs);
}

hipError_t launch_recurrent(const gdr_args& a, hipStream_t stream) {
  // Wide slices stream the most bytes per workgroup; narrow slices give small batches enough workgroups.
  const long long wide_blocks = (long long)a.batch * a.heads * (a.value_dim / 128);
  const int vs = (a.value_dim % 128 == 0 && wide_blocks >= 1024) ? 128 : 32;
  switch (a.variant) {
    case GDR_KDA: return launch_recurrent_v<GDR_KDA>(a, stream, vs);
    case GDR_GDN: return launch_recurrent_v<GDR_GDN>(a, stream, vs);
    case GDR_GLA: return launch_recurrent_v<GDR_GLA>(a, stream, vs);
    default: return launch_recurrent_v<GDR_DELTANET>(a, stream, vs);
  }
}

}  // namespace gdr
