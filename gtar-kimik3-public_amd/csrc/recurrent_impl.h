// Kernels of the recurrent (decode) family, shared by recurrent.hip (key dims 64 and 128) and recurrent_k.hip (key
// dims 32, 192 and 256): the templates and their launch helpers; see recurrent.hip for the design.
#pragma once

#include "gdr_common.h"
#include "gdr_internal.h"
#include "varlen_index.h"

namespace gdr {

// The state is read exactly once: a non-temporal load keeps it from displacing reusable lines in the caches
// (measured on MI355X at batch 256: 6.3 TB/s against 5.1 TB/s with plain loads for the same kernel).
__device__ __forceinline__ float4 load_stream4(const float* p) {
  return make_float4(__builtin_nontemporal_load(p), __builtin_nontemporal_load(p + 1),
                     __builtin_nontemporal_load(p + 2), __builtin_nontemporal_load(p + 3));
}

// The two state operations the verify and commit kernels must round identically: explicit fma for the rank-1
// update (never left to contraction, which could instead fuse the decay product into the add).
__device__ __forceinline__ void decay4(float4& s, float e) {
  s.x *= e; s.y *= e; s.z *= e; s.w *= e;
}
__device__ __forceinline__ void rank1_update(float4& s, float kr, float u0, float u1, float u2, float u3) {
  s.x = __builtin_fmaf(kr, u0, s.x); s.y = __builtin_fmaf(kr, u1, s.y);
  s.z = __builtin_fmaf(kr, u2, s.z); s.w = __builtin_fmaf(kr, u3, s.w);
}

// q, k and v share one element type InT (bf16 or fp32; the host widens mixed or fp16 inputs to fp32, exactly), so
// every load has a static type and the compiler can track each one's completion precisely.
// The body of the decode kernel and of the verify kernel (kRecord: also store each token's update row).  With
// kCommit it first applies the accepted prefix of the previous verified block (`c`: its k, gate, length, initial
// state h0 and committed-state output ht; `prev_updates`: its update record) to the register-resident state, exactly
// as the commit kernel does, writes that committed state to c.ht, and then verifies the new block from it; kH0 then
// means c.h0 is non-null.
template <int VARIANT, int K, int VS, int kThreads, typename InT, bool kH0, bool kRecord, bool kCommit = false>
__device__ __forceinline__ void recurrent_body(const gdr_args& a, int n_slices, float* updates,
                                               const gdr_args* c = nullptr, const float* prev_updates = nullptr,
                                               const int32_t* accepted = nullptr) {
  constexpr int kWaves = kThreads / kWave;
  constexpr int NQ = VS / 4;           // float4 column quads per state row slice
  constexpr int RG = kThreads / NQ;    // row groups
  constexpr int RPT = K / RG;          // state rows per thread
  static_assert(NQ <= kWave && RPT >= 1 && K % RG == 0 && kThreads >= VS, "bad recurrent tiling");
  constexpr bool kDelta = VARIANT != GDR_GLA;
  constexpr bool kChannelGate = VARIANT == GDR_KDA || VARIANT == GDR_GLA;
  constexpr bool kScalarGate = VARIANT == GDR_GDN;

  const int slice = blockIdx.x % n_slices;
  const int bh = blockIdx.x / n_slices;  // (batch entry or packed sequence) * H + head
  const int H = a.heads, V = a.value_dim;
  const int h = bh % H;
  // With cu_seqlens (the forward only) the workgroup runs packed sequence bh / H over its rows of the batch-1 input.
  int b = bh / H, bos = 0, T = a.seq_len;
  if (a.cu_seqlens) {
    bos = packed_begin(a.cu_seqlens, b, a.seq_len);
    T = packed_end(a.cu_seqlens, b, a.seq_len) - bos;
    b = 0;
  }
  const int v0 = slice * VS;
  const int tid = threadIdx.x;
  const int quad = tid % NQ, rg = tid / NQ;
  const int lane = tid % kWave, wave = tid / kWave;
  const int col = v0 + 4 * quad;

  // Token vectors are staged through LDS kGroup tokens at a time: one memory latency per group of tokens, not one
  // per token, which under a saturated HBM would dominate multi-token calls (speculative verify blocks).  A later
  // group is fetched only when the previous one is done, so no prefetch registers stay live across the token loop.
  constexpr int kGroup = 8;
  constexpr int NK = (kGroup * K + kThreads - 1) / kThreads;    // q / k / gate elements per thread and group
  constexpr int NV = (kGroup * VS + kThreads - 1) / kThreads;   // v elements per thread and group
  // q, k and the decay factors are stored row-group-major: channel r at position (r % RG) * RPT + r / RG, so a
  // thread's RPT rows rg, rg + RG, ... are contiguous and arrive in one or two wide LDS reads.
  __shared__ __align__(16) float s_q[kGroup][K], s_k[kGroup][K], s_eg[kGroup][kChannelGate ? K : 1];
  __shared__ __align__(16) float s_v[kGroup][VS];  // v rows; the previous block's update rows in the commit phase
  __shared__ float s_scalar[kGroup][2];  // beta, scalar decay
  __shared__ float s_qk[kGroup];         // q . k per token
  __shared__ __align__(16) float s_red[kWaves][2][VS];  // per-wave partial k S and q S
  __shared__ __align__(16) float s_u[VS];               // the token's update row

  // Uniform (b, h) base pointers plus a 32-bit per-lane offset: one address register per row, not a 64-bit pair.
  const size_t state_base = size_t(bh) * K * V;
  const float* h0 = a.h0 ? a.h0 + state_base : nullptr;
  float* ht = a.ht ? a.ht + state_base : nullptr;
  const uint32_t lane_off = uint32_t(rg) * V + col;

  const int64_t qb = b * a.q.stride_b + h * a.q.stride_h + bos * a.q.stride_t;
  const int64_t kb = b * a.k.stride_b + h * a.k.stride_h + bos * a.k.stride_t;
  const int64_t vb = b * a.v.stride_b + h * a.v.stride_h + bos * a.v.stride_t;
  const int64_t ob = b * a.out.stride_b + h * a.out.stride_h + bos * a.out.stride_t;
  const int64_t gb = b * a.gate.stride_b + h * a.gate.stride_h + bos * a.gate.stride_t;
  const int64_t bb = b * a.beta.stride_b + h * a.beta.stride_h + bos * a.beta.stride_t;

  // A group's vectors: fetched into registers (element i of a [kGroup][K] or [kGroup][VS] block goes to thread
  // i % kThreads), then converted and staged in LDS.  Elements of tokens at or beyond T are neither loaded nor staged.
  const InT* qp = static_cast<const InT*>(a.q.ptr);
  const InT* kp = static_cast<const InT*>(a.k.ptr);
  const InT* vp = static_cast<const InT*>(a.v.ptr);
  const float* gp = static_cast<const float*>(a.gate.ptr);
  const float* betap = static_cast<const float*>(a.beta.ptr);
  InT raw_q[NK], raw_k[NK], raw_v[NV];
  float raw_g[NK], raw_beta = 0.f, raw_sg = 0.f;
  auto fetch = [&](int t0) {
#pragma unroll
    for (int j = 0; j < NK; ++j) {
      const int i = tid + j * kThreads, tt = i / K, c = i % K;
      if (i < kGroup * K && t0 + tt < T) {
        raw_q[j] = qp[qb + (t0 + tt) * a.q.stride_t + c];
        raw_k[j] = kp[kb + (t0 + tt) * a.k.stride_t + c];
        if constexpr (kChannelGate) raw_g[j] = gp[gb + (t0 + tt) * a.gate.stride_t + c];
      }
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int i = tid + j * kThreads, tt = i / VS, c = i % VS;
      if (i < kGroup * VS && t0 + tt < T) raw_v[j] = vp[vb + (t0 + tt) * a.v.stride_t + v0 + c];
    }
    if (tid < kGroup && t0 + tid < T) {
      if constexpr (kDelta) raw_beta = betap[bb + (t0 + tid) * a.beta.stride_t];
      if constexpr (kScalarGate) raw_sg = gp[gb + (t0 + tid) * a.gate.stride_t];
    }
  };
  auto stage = [&](int t0) {
#pragma unroll
    for (int j = 0; j < NK; ++j) {
      const int i = tid + j * kThreads, tt = i / K, c = i % K, pos = (c % RG) * RPT + c / RG;
      if (i < kGroup * K && t0 + tt < T) {
        s_q[tt][pos] = static_cast<float>(raw_q[j]);
        s_k[tt][pos] = static_cast<float>(raw_k[j]);
        if constexpr (kChannelGate) s_eg[tt][pos] = exp_fast(raw_g[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int i = tid + j * kThreads, tt = i / VS, c = i % VS;
      if (i < kGroup * VS && t0 + tt < T) s_v[tt][c] = static_cast<float>(raw_v[j]);
    }
    if (tid < kGroup && t0 + tid < T) {
      if constexpr (kDelta) s_scalar[tid][0] = raw_beta;
      if constexpr (kScalarGate) s_scalar[tid][1] = exp_fast(raw_sg);
    }
  };

  float4 st[RPT];  // (kH0 is a template argument: a run-time branch here would make the wait below conservative)
  if constexpr (kCommit) {
    // The previous block's accepted prefix, staged kGroup tokens at a time through the same LDS tiles (k and the
    // decay factors row-group-major, the update rows in s_v): per token S <- decay_t S; S <- S + k_t^T u_t, with the
    // commit kernel's operations in its order, so the committed state is bit-identical to gdr_recurrent_commit's.
    const int Tc = c->seq_len;
    const int n = accepted ? min(max(accepted[b], 0), Tc) : Tc;  // uniform over the workgroup
    const InT* ckp = static_cast<const InT*>(c->k.ptr);
    const float* cgp = static_cast<const float*>(c->gate.ptr);
    const int64_t ckb = b * c->k.stride_b + h * c->k.stride_h;
    const int64_t cgb = b * c->gate.stride_b + h * c->gate.stride_h;
    const float* up = prev_updates + size_t(bh) * Tc * V + v0;
    // Its group registers use the verify's element-to-thread mapping (element i of a group to thread i % kThreads).
    constexpr int NU = (kGroup * NQ + kThreads - 1) / kThreads;  // update-row quads per thread and group
    InT ck[NK];
    float cg[NK], csg = 0.f;
    float4 cu[NU];
    auto cfetch = [&](int t0, int cnt) {
#pragma unroll
      for (int j = 0; j < NK; ++j) {
        const int i = tid + j * kThreads, tt = i / K, ch = i % K;
        if (i < kGroup * K && tt < cnt) {
          ck[j] = ckp[ckb + (t0 + tt) * c->k.stride_t + ch];
          if constexpr (kChannelGate) cg[j] = cgp[cgb + (t0 + tt) * c->gate.stride_t + ch];
        }
      }
#pragma unroll
      for (int j = 0; j < NU; ++j) {
        const int i = tid + j * kThreads, tt = i / NQ, qd = i % NQ;
        if (i < kGroup * NQ && tt < cnt) cu[j] = *reinterpret_cast<const float4*>(up + size_t(t0 + tt) * V + 4 * qd);
      }
      if constexpr (kScalarGate) {
        if (tid < cnt) csg = cgp[cgb + (t0 + tid) * c->gate.stride_t];
      }
    };
    auto cstage = [&](int cnt) {
#pragma unroll
      for (int j = 0; j < NK; ++j) {
        const int i = tid + j * kThreads, tt = i / K, ch = i % K, pos = (ch % RG) * RPT + ch / RG;
        if (i < kGroup * K && tt < cnt) {
          s_k[tt][pos] = static_cast<float>(ck[j]);
          if constexpr (kChannelGate) s_eg[tt][pos] = exp_fast(cg[j]);
        }
      }
#pragma unroll
      for (int j = 0; j < NU; ++j) {
        const int i = tid + j * kThreads, tt = i / NQ, qd = i % NQ;
        if (i < kGroup * NQ && tt < cnt) *reinterpret_cast<float4*>(&s_v[tt][4 * qd]) = cu[j];
      }
      if constexpr (kScalarGate) {
        if (tid < cnt) s_scalar[tid][1] = exp_fast(csg);
      }
    };
    // Request order: the first commit group, the state, then the block's first group, so each wait below covers
    // only what it needs (loads complete in order) and the block's vectors arrive during the commit.
    auto capply = [&](int cnt) {
      for (int tt = 0; tt < cnt; ++tt) {
        const float4 u = *reinterpret_cast<const float4*>(&s_v[tt][4 * quad]);
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
          if constexpr (kChannelGate) decay4(st[i], s_eg[tt][rg * RPT + i]);
          if constexpr (kScalarGate) decay4(st[i], s_scalar[tt][1]);
          rank1_update(st[i], s_k[tt][rg * RPT + i], u.x, u.y, u.z, u.w);
        }
      }
    };
    // The first group is straight-line code (a group of 0 tokens loads and stages nothing), so the wait before its
    // staging can count the later loads precisely; later groups (blocks longer than kGroup) loop.
    const int cnt0 = min(kGroup, n);
    cfetch(0, cnt0);
#pragma unroll
    for (int i = 0; i < RPT; ++i)
      st[i] = kH0 ? load_stream4(c->h0 + state_base + lane_off + uint32_t(RG * i) * V) : make_float4(0.f, 0.f, 0.f, 0.f);
    if (T > 0) fetch(0);
    cstage(cnt0);
    __syncthreads();
    capply(cnt0);
    for (int t0 = kGroup; t0 < n; t0 += kGroup) {
      const int cnt = min(kGroup, n - t0);
      __syncthreads();  // the previous group's LDS reads are done
      cfetch(t0, cnt);
      cstage(cnt);
      __syncthreads();
      capply(cnt);
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i)  // each element is read and written by this thread only, so c.ht may be c.h0
      *reinterpret_cast<float4*>(c->ht + state_base + lane_off + uint32_t(RG * i) * V) = st[i];
    __syncthreads();  // the commit's LDS reads are done before the block is staged
    if (T > 0) stage(0);
  } else {
    // The first group's vectors are requested before the state stream and staged in straight-line code, so staging
    // waits for them alone while the state loads stay in flight.
    if (T > 0) fetch(0);
#pragma unroll
    for (int i = 0; i < RPT; ++i)
      st[i] = kH0 ? load_stream4(h0 + lane_off + uint32_t(RG * i) * V) : make_float4(0.f, 0.f, 0.f, 0.f);
    if (T > 0) stage(0);
  }

  // Per token: every wave folds its rows into per-wave partial sums of k S and q S (registers, then LDS); after a
  // barrier one thread per column adds the waves' partials in wave order, forms u and the output; after a second
  // barrier every thread applies the rank-1 update with u.  Only 2 x VS partials per wave cross LDS, not each
  // thread's reads of every wave's.  Around a group boundary two more barriers keep the previous group alive until
  // every wave is done with it and make the new one visible.
  for (int t0 = 0; t0 < T; t0 += kGroup) {
    if (t0 > 0) {
      __syncthreads();
      fetch(t0);
      stage(t0);
    }
    __syncthreads();
    const int n_tok = min(kGroup, T - t0);
    // q . k of the group's tokens (for the readout correction), one wave per token; read after token tt's first
    // barrier, which orders these writes.
    for (int tt = wave; tt < n_tok; tt += kWaves) {
      float p = 0.f;
      for (int c = lane; c < K; c += kWave) p += s_q[tt][c] * s_k[tt][c];
#pragma unroll
      for (int m = 1; m < kWave; m *= 2) p = xor_sum(p, m);
      if (lane == 0) s_qk[tt] = p;
    }
    for (int tt = 0; tt < n_tok; ++tt) {
      const int t = t0 + tt;

      // Decay and the two dk-partial reductions in one pass over the register-resident rows.
      float ak[4] = {0.f, 0.f, 0.f, 0.f}, aq[4] = {0.f, 0.f, 0.f, 0.f};
      const float eg_scalar = kScalarGate ? s_scalar[tt][1] : 1.f;
      float kr[RPT], qr[RPT], er[RPT];  // this thread's rows, contiguous in the row-group-major layout
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        kr[i] = s_k[tt][rg * RPT + i];
        qr[i] = s_q[tt][rg * RPT + i];
        if constexpr (kChannelGate) er[i] = s_eg[tt][rg * RPT + i];
      }
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        float e = 1.f;
        if constexpr (kChannelGate) e = er[i];
        if constexpr (kScalarGate) e = eg_scalar;
        if constexpr (kChannelGate || kScalarGate) decay4(st[i], e);
        ak[0] += kr[i] * st[i].x; ak[1] += kr[i] * st[i].y; ak[2] += kr[i] * st[i].z; ak[3] += kr[i] * st[i].w;
        aq[0] += qr[i] * st[i].x; aq[1] += qr[i] * st[i].y; aq[2] += qr[i] * st[i].z; aq[3] += qr[i] * st[i].w;
      }
#pragma unroll
      for (int m = NQ; m < kWave; m *= 2) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          ak[j] = xor_sum(ak[j], m);  // VALU lane moves for m = 8, 16, 32: no LDS round trip
          aq[j] = xor_sum(aq[j], m);
        }
      }
      if (lane < NQ) {
        *reinterpret_cast<float4*>(&s_red[wave][0][4 * quad]) = make_float4(ak[0], ak[1], ak[2], ak[3]);
        *reinterpret_cast<float4*>(&s_red[wave][1][4 * quad]) = make_float4(aq[0], aq[1], aq[2], aq[3]);
      }
      __syncthreads();

      if (tid < VS) {  // kThreads >= VS: one thread per column
        float kS = 0.f, qS = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          kS += s_red[w][0][tid];
          qS += s_red[w][1][tid];
        }
        const float vj = s_v[tt][tid];
        const float u = kDelta ? s_scalar[tt][0] * (vj - kS) : vj;
        s_u[tid] = u;
        store_any(const_cast<void*>(a.out.ptr), ob + t * a.out.stride_t + v0 + tid, a.out.dtype,
                  a.scale * (qS + s_qk[tt] * u));
        if constexpr (kRecord) updates[(size_t(bh) * T + t) * V + v0 + tid] = u;
      }
      __syncthreads();

      const float4 u = *reinterpret_cast<const float4*>(&s_u[4 * quad]);
#pragma unroll
      for (int i = 0; i < RPT; ++i) rank1_update(st[i], kr[i], u.x, u.y, u.z, u.w);
    }
  }

  if (ht) {
#pragma unroll
    for (int i = 0; i < RPT; ++i) *reinterpret_cast<float4*>(ht + lane_off + uint32_t(RG * i) * V) = st[i];
  }
}

// Two kernels (so profiles tell them apart) over one body.  Occupancy floor of 4 waves per SIMD (at most 128
// VGPRs): two 512-thread workgroups per CU, which the group-staging address arithmetic would otherwise push down to
// one.
template <int VARIANT, int K, int VS, int kThreads, typename InT, bool kH0>
__global__ __launch_bounds__(kThreads, 4) void recurrent_fwd_kernel(const gdr_args a, int n_slices) {
  recurrent_body<VARIANT, K, VS, kThreads, InT, kH0, false>(a, n_slices, nullptr);
}

template <int VARIANT, int K, int VS, int kThreads, typename InT, bool kH0>
__global__ __launch_bounds__(kThreads, 4) void recurrent_verify_kernel(const gdr_args a, int n_slices,
                                                                       float* updates) {
  recurrent_body<VARIANT, K, VS, kThreads, InT, kH0, true>(a, n_slices, updates);
}

// Commit of the previous block, then verify of the next, in one pass over the state (kH0: c.h0 is non-null).
template <int VARIANT, int K, int VS, int kThreads, typename InT, bool kH0>
__global__ __launch_bounds__(kThreads, 4) void recurrent_commit_verify_kernel(const gdr_args a, int n_slices,
                                                                              float* updates, const gdr_args c,
                                                                              const float* prev_updates,
                                                                              const int32_t* accepted) {
  recurrent_body<VARIANT, K, VS, kThreads, InT, kH0, true, true>(a, n_slices, updates, &c, prev_updates, accepted);
}

// State after the first n_b = clamp(accepted[b], 0, T) tokens of a verified block (all T when `accepted` is NULL):
//   S = h0;  for t < n_b:  S <- decay_t S;  S <- S + k_t^T u_t      (u_t from the verify kernel's record)
// Same workgroup tiling as the recurrent kernel (one [K, VS] column slice per workgroup, float4 column quads held in
// registers), so the state is streamed once each way.  Tokens are staged through LDS kGroup at a time.
template <int VARIANT, int K, int VS, int kThreads, typename InT, bool kH0>
__global__ __launch_bounds__(kThreads) void recurrent_commit_kernel(const gdr_args a, int n_slices,
                                                                    const float* __restrict__ updates,
                                                                    const int32_t* __restrict__ accepted) {
  constexpr int NQ = VS / 4, RG = kThreads / NQ, RPT = K / RG;
  static_assert(NQ <= kWave && RPT >= 1 && K % RG == 0, "bad commit tiling");
  constexpr int kGroup = 8;
  constexpr bool kChannelGate = VARIANT == GDR_KDA || VARIANT == GDR_GLA;
  constexpr bool kScalarGate = VARIANT == GDR_GDN;

  const int slice = blockIdx.x % n_slices;
  const int bh = blockIdx.x / n_slices;
  const int H = a.heads, V = a.value_dim, T = a.seq_len;
  const int b = bh / H, h = bh % H;
  const int v0 = slice * VS;
  const int tid = threadIdx.x;
  const int quad = tid % NQ, rg = tid / NQ;
  const int n = accepted ? min(max(accepted[b], 0), T) : T;  // uniform over the workgroup

  __shared__ float s_k[kGroup][K];
  __shared__ float s_eg[kGroup][kChannelGate ? K : 1];
  __shared__ float4 s_u[kGroup][NQ];

  const size_t state_base = size_t(bh) * K * V;
  const uint32_t lane_off = uint32_t(rg) * V + v0 + 4 * quad;
  const int64_t kb = b * a.k.stride_b + h * a.k.stride_h;
  const int64_t gb = b * a.gate.stride_b + h * a.gate.stride_h;
  const InT* kp = static_cast<const InT*>(a.k.ptr);
  const float* gp = static_cast<const float*>(a.gate.ptr);
  const float* up = updates + size_t(bh) * T * V + v0;

  float4 st[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i)
    st[i] = kH0 ? load_stream4(a.h0 + state_base + lane_off + uint32_t(RG * i) * V) : make_float4(0.f, 0.f, 0.f, 0.f);

  for (int t0 = 0; t0 < n; t0 += kGroup) {
    const int cnt = min(kGroup, n - t0);
    __syncthreads();  // the previous group's LDS reads are done
    for (int i = tid; i < cnt * K; i += kThreads) {
      const int tt = i / K, c = i % K;
      s_k[tt][c] = static_cast<float>(kp[kb + (t0 + tt) * a.k.stride_t + c]);
      if constexpr (kChannelGate) s_eg[tt][c] = exp_fast(gp[gb + (t0 + tt) * a.gate.stride_t + c]);
    }
    if constexpr (kScalarGate) {
      if (tid < cnt) s_eg[tid][0] = exp_fast(gp[gb + (t0 + tid) * a.gate.stride_t]);
    }
    for (int i = tid; i < cnt * NQ; i += kThreads) {
      const int tt = i / NQ, c = i % NQ;
      s_u[tt][c] = *reinterpret_cast<const float4*>(up + size_t(t0 + tt) * V + 4 * c);
    }
    __syncthreads();
    for (int tt = 0; tt < cnt; ++tt) {
      const float4 u = s_u[tt][quad];
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const int r = rg + RG * i;
        if constexpr (kChannelGate) decay4(st[i], s_eg[tt][r]);
        if constexpr (kScalarGate) decay4(st[i], s_eg[tt][0]);
        rank1_update(st[i], s_k[tt][r], u.x, u.y, u.z, u.w);
      }
    }
  }

#pragma unroll
  for (int i = 0; i < RPT; ++i)
    *reinterpret_cast<float4*>(a.ht + state_base + lane_off + uint32_t(RG * i) * V) = st[i];
}

// Launch modes of the recurrent family: the forward, the verify forward (with the update record) and the commit.
enum class RecMode { kForward, kVerify, kCommit, kCommitVerify };

struct RecExtra {
  float* record;             // kVerify, kCommitVerify: written
  const float* updates;      // kCommit, kCommitVerify: read (the previous block's record)
  const int32_t* accepted;   // kCommit, kCommitVerify: device [B] or NULL
  const gdr_args* prev;      // kCommitVerify: the previous block's commit arguments
};

template <int VARIANT, int K, int VS, int kThreads, typename InT, bool kH0>
inline void launch_shape(const gdr_args& a, hipStream_t stream, RecMode mode, const RecExtra& x) {
  const int n_slices = a.value_dim / VS;
  const dim3 grid((a.cu_seqlens ? a.n_seqs : a.batch) * a.heads * n_slices), block(kThreads);
  if (mode == RecMode::kCommitVerify)
    hipLaunchKernelGGL((recurrent_commit_verify_kernel<VARIANT, K, VS, kThreads, InT, kH0>), grid, block, 0, stream,
                       a, n_slices, x.record, *x.prev, x.updates, x.accepted);
  else if (mode == RecMode::kCommit)
    hipLaunchKernelGGL((recurrent_commit_kernel<VARIANT, K, VS, kThreads, InT, kH0>), grid, block, 0, stream, a,
                       n_slices, x.updates, x.accepted);
  else if (mode == RecMode::kVerify)
    hipLaunchKernelGGL((recurrent_verify_kernel<VARIANT, K, VS, kThreads, InT, kH0>), grid, block, 0, stream, a,
                       n_slices, x.record);
  else
    hipLaunchKernelGGL((recurrent_fwd_kernel<VARIANT, K, VS, kThreads, InT, kH0>), grid, block, 0, stream, a,
                       n_slices);
}

template <int VARIANT, int K, typename InT, bool kH0>
inline hipError_t launch_recurrent_k(const gdr_args& a, hipStream_t stream, int vs, RecMode mode, const RecExtra& x) {
  // 128-column slices: 512 threads, K / 16 state rows x one float4 per thread (8 at K = 128); key dims above 128
  // take 32-column slices only (256 threads, K / 32 rows per thread), which keeps the state within the registers.
  if constexpr (K <= 128) {
    if (vs == 128) {
      launch_shape<VARIANT, K, 128, 512, InT, kH0>(a, stream, mode, x);
      return hipGetLastError();
    }
  }
  launch_shape<VARIANT, K, 32, 256, InT, kH0>(a, stream, mode, x);
  return hipGetLastError();
}

// The key dims other than 64 and 128 (32, 192 and 256), instantiated in recurrent_k.hip.
hipError_t launch_recurrent_other_k(const gdr_args& a, hipStream_t stream, int vs, RecMode mode, const RecExtra& x,
                                    int dtype);

}  // namespace gdr
