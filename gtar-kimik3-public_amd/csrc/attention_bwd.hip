// Backward of the causal grouped-query attention (gdr_attention_bwd; src/ops/flash_attention_2.py:180-207).
//
//   P = 2^(c S - lse)  (S = Q K^T, c = scale log2 e, lse the forward's row log-sum-exp in log2 units)
//   delta = rowsum(O (x) dO),  dP = dO V^T,  dS = P (x) (dP - delta)
//   dQ = scale dS K,  dK = scale dS^T Q,  dV = P^T dO                  (per (sequence, query head); key/value head
//                                                                       h / (H / Hkv) sums its group's terms)
//
// Two launches of four-wave workgroups on v_mfma_f32_16x16x32_{bf16,f16} with fp32 accumulation; P and dS enter
// their products rounded to the input type, as the reference's probs.to(dtype) and dscores.to(dtype) do:
//   * attention_dq_kernel -- 128 query rows of one (sequence, query head), two 16-row blocks per wave, the q and dO
//     rows held in registers as B operands.  It first forms delta from the out and dO rows (and stores it for the
//     second launch), then streams the 64-row key and value tiles up to the diagonal through double-buffered LDS
//     (LDS DMA).  Per tile S^T = K Q^T and dP^T = V dO^T take the tile rows as A operands, so a lane holds 16
//     entries of one query row; dS^T then feeds dQ^T += K^T dS^T straight from the accumulators, K^T coming from the
//     transposing LDS read.
//   * attention_dkdv_kernel -- 64 keys of one (sequence, key/value head), one 16-key block per wave, the k and v
//     rows held in registers as B operands.  Query and dO tiles of 64 rows, with their lse and delta, stream through
//     double-buffered LDS for every query head of the group, from the tile holding the diagonal on.  Per tile S =
//     Q K^T and dP = dO V^T (a lane holds 16 entries of one key column), then dV^T += dO^T P and dK^T += Q^T dS with
//     the transposing read.
// Only tiles crossing the diagonal or the sequence end are masked.  No atomics: every output element has one
// owning lane, so the result does not depend on scheduling.
#include "attention_common.h"
#include "varlen_index.h"
#include "gdr_internal.h"

namespace gdr {
namespace {

using attn::cat;
using attn::kTile;
using attn::Mma;
using attn::short4;
using chunk::kLog2e;

constexpr int kQB = 128;  // query rows per dq workgroup
constexpr int kKB = 64;   // keys per dk/dv workgroup (one 16-key block per wave)
constexpr int kRB = 2;    // 16-row query blocks per wave in the dq kernel
static_assert(kKB == kTile, "the dk/dv kernel's first query tile is the one holding its diagonal");

// The lse and delta of query rows 16 m + 4 g4 .. + 3 (m = 0..3) of a tile from their LDS rows at byte addresses
// `la` and `da` (this lane's 4 g4 already added), waited for inside.  Inline assembly: the compiler cannot tell these
// reads from the LDS DMA still in flight into the other buffers, and would otherwise wait for that DMA first.
__device__ __forceinline__ void lds_rows4(uint32_t la, uint32_t da, floatx4 (&l)[4], floatx4 (&d)[4]) {
  asm volatile(
      "ds_read_b128 %0, %8\n\t"
      "ds_read_b128 %1, %8 offset:64\n\t"
      "ds_read_b128 %2, %8 offset:128\n\t"
      "ds_read_b128 %3, %8 offset:192\n\t"
      "ds_read_b128 %4, %9\n\t"
      "ds_read_b128 %5, %9 offset:64\n\t"
      "ds_read_b128 %6, %9 offset:128\n\t"
      "ds_read_b128 %7, %9 offset:192\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(l[0]), "=&v"(l[1]), "=&v"(l[2]), "=&v"(l[3]), "=&v"(d[0]), "=&v"(d[1]), "=&v"(d[2]), "=&v"(d[3])
      : "v"(la), "v"(da));
}

template <typename V4, typename V8>
__device__ __forceinline__ V8 tr_pair(const short4 (&r)[4], int s2) {
  return cat<V4, V8>(__builtin_bit_cast(V4, r[2 * s2]), __builtin_bit_cast(V4, r[2 * s2 + 1]));
}

template <int D, typename T>
__global__ __launch_bounds__(attn::kThreads, 2) void attention_dq_kernel(const gdr_attention_args a,
                                                                      const gdr_attention_grads g, int nqb) {
  using M = Mma<T>;
  using V8 = typename M::v8;
  using V4 = typename M::v4;
  constexpr int DS = D / 32;  // 32-wide k steps of the score products
  constexpr int DT = D / 16;  // 16-column tiles of dQ^T
  constexpr int TILE = kTile * D;
  extern __shared__ __align__(16) unsigned char smem[];
  T* ks = reinterpret_cast<T*>(smem);             // [2][kTile][D] swizzled
  T* vs = reinterpret_cast<T*>(smem) + 2 * TILE;  // [2][kTile][D] swizzled

  // ---- workgroup -> (sequence, query block, head), the latest query blocks (the most keys) first ----
  const int H = a.heads;
  const int h = blockIdx.x % H, slot = blockIdx.x / H;
  int n, qb, bos = 0, len = a.seq_len;
  if (a.cu_seqlens) {
    n = packed_slot_seq(a.cu_seqlens, a.n_seqs, a.seq_len, kQB, slot);
    bos = packed_begin(a.cu_seqlens, n, a.seq_len);
    len = packed_end(a.cu_seqlens, n, a.seq_len) - bos;
    const int nb = (len + kQB - 1) / kQB;
    const int r = slot - packed_slot_base(a.cu_seqlens, n, a.seq_len, kQB);
    if (r < 0 || r >= nb) return;  // gap slot: uniform over the workgroup, before any barrier
    qb = nb - 1 - r;
  } else {
    n = slot / nqb;
    qb = nqb - 1 - slot % nqb;
  }
  const int bidx = a.cu_seqlens ? 0 : n;
  const int hk = h / (H / a.kv_heads);
  auto at = [&](const gdr_tensor& t, int head) {
    return static_cast<const T*>(t.ptr) + bidx * t.stride_b + head * t.stride_h + int64_t(bos) * t.stride_t;
  };
  const T* qp = at(a.q, h);
  const T* kp = at(a.k, hk);
  const T* vp = at(a.v, hk);
  const T* op = at(a.out, h);
  const T* dop = at(g.d_out, h);
  T* dqp = const_cast<T*>(at(g.d_q, h));
  const int64_t row0 = (int64_t(bidx) * H + h) * a.seq_len + bos;  // lse / delta index of the sequence's row 0

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l16 = lane & 15, g4 = lane >> 4;
  const int q0 = qb * kQB;

  // This lane's query rows (l16 of each block) as B operands: q and dO columns 32 ds + 8 g4 .. + 7.  delta =
  // rowsum(out (x) dO) from the same fragments, summed over the four lane groups.
  int qpos[kRB];
  V8 qf[kRB][DS], df[kRB][DS];
  float lse[kRB], dlt[kRB];
#pragma unroll
  for (int b = 0; b < kRB; ++b) {
    qpos[b] = q0 + 16 * (kRB * wave + b) + l16;
    const int qrow = min(qpos[b], len - 1);
    float part = 0.f;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      const int col = 32 * ds + 8 * g4;
      qf[b][ds] = *reinterpret_cast<const V8*>(qp + int64_t(qrow) * a.q.stride_t + col);
      df[b][ds] = *reinterpret_cast<const V8*>(dop + int64_t(qrow) * g.d_out.stride_t + col);
      const V8 of = *reinterpret_cast<const V8*>(op + int64_t(qrow) * a.out.stride_t + col);
#pragma unroll
      for (int j = 0; j < 8; ++j) part += static_cast<float>(of[j]) * static_cast<float>(df[b][ds][j]);
    }
    part = xor_sum(part, 16);
    dlt[b] = xor_sum(part, 32);
    lse[b] = a.lse[row0 + qrow];
    if (g4 == 0 && qpos[b] < len) g.delta[row0 + qpos[b]] = dlt[b];
  }

  attn::TileDma<D> dma;
  dma.init(__builtin_amdgcn_readfirstlane(wave), lane);
  const int kend = min(len, q0 + kQB);  // keys this block can see
  const int nkb = (kend + kTile - 1) / kTile;
  int koff[DS], toff[DT];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) koff[ds] = attn::row_frag<D>(ds, l16, g4);
#pragma unroll
  for (int t = 0; t < DT; ++t) toff[t] = attn::tr_frag<D>(t, l16, g4);
  const float c = a.scale * kLog2e;
  const uint32_t klds = attn::lds_addr(ks);

  dma.issue(kp, a.k.stride_t, 0, len, ks);
  dma.issue(vp, a.v.stride_t, 0, len, vs);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  floatx4 dq[kRB][DT];  // dQ^T: lane holds columns 16 t + 4 g4 + i of query row qpos[b]
#pragma unroll
  for (int b = 0; b < kRB; ++b)
#pragma unroll
    for (int t = 0; t < DT; ++t) dq[b][t] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int kb = 0; kb < nkb; ++kb) {
    const int cur = kb & 1;
    if (kb + 1 < nkb) {  // the other buffers were released by the barrier that ended the previous step
      dma.issue(kp, a.k.stride_t, (kb + 1) * kTile, len, ks + (cur ^ 1) * TILE);
      dma.issue(vp, a.v.stride_t, (kb + 1) * kTile, len, vs + (cur ^ 1) * TILE);
    }
    const T* kt = ks + cur * TILE;
    const T* vt = vs + cur * TILE;
    // S^T and dP^T: lane holds key kb kTile + 16 t + 4 g4 + i of query row qpos[b]
    floatx4 s[kRB][4], dp[kRB][4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int b = 0; b < kRB; ++b) s[b][t] = dp[b][t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const V8 kf = *reinterpret_cast<const V8*>(kt + 16 * t * D + koff[ds]);
        const V8 vf = *reinterpret_cast<const V8*>(vt + 16 * t * D + koff[ds]);
#pragma unroll
        for (int b = 0; b < kRB; ++b) {
          s[b][t] = M::run(kf, qf[b][ds], s[b][t]);
          dp[b][t] = M::run(vf, df[b][ds], dp[b][t]);
        }
      }
    }
    // dS^T = P^T (x) (dP^T - delta); only a tile crossing this wave's diagonal or the sequence end is masked
    const bool full = (kb + 1) * kTile - 1 <= q0 + 32 * wave && (kb + 1) * kTile <= len;
    V8 dsf[kRB][2];
#pragma unroll
    for (int b = 0; b < kRB; ++b) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = kb * kTile + 16 * t + 4 * g4 + i;
          float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[b][t][i], c, -lse[b]));
          if (!full && !(key <= qpos[b] && key < len)) p = 0.f;
          s[b][t][i] = p * (dp[b][t][i] - dlt[b]);
        }
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) dsf[b][s2] = cat<V4, V8>(M::pack(s[b][2 * s2]), M::pack(s[b][2 * s2 + 1]));
    }
    // dQ^T += K^T dS^T: K^T of column tile t through the transposing read, one tile ahead of its MFMAs
    const uint32_t kaddr = klds + 2 * cur * TILE;
    short4 x[2][4];
    attn::tr_read4<D>(kaddr + 2 * toff[0], x[0]);
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      short4(&r)[4] = x[t & 1];
      if (t + 1 < DT) {
        attn::tr_read4<D>(kaddr + 2 * toff[t + 1], x[(t + 1) & 1]);
        asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]));
      } else {
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]));
      }
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const V8 kf = tr_pair<V4, V8>(r, s2);
#pragma unroll
        for (int b = 0; b < kRB; ++b) dq[b][t] = M::run(kf, dsf[b][s2], dq[b][t]);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's copies of the next tiles have landed
    __syncthreads();                 // ... everyone's, and every wave is done with this step's buffers
  }

#pragma unroll
  for (int b = 0; b < kRB; ++b) {
    if (qpos[b] < len) {
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        floatx4 y = dq[b][t];
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] *= a.scale;
        *reinterpret_cast<V4*>(dqp + int64_t(qpos[b]) * g.d_q.stride_t + 16 * t + 4 * g4) = M::pack(y);
      }
    }
  }
}

template <int D, typename T>
__global__ __launch_bounds__(attn::kThreads, 2) void attention_dkdv_kernel(const gdr_attention_args a,
                                                                        const gdr_attention_grads g, int nkb) {
  using M = Mma<T>;
  using V8 = typename M::v8;
  using V4 = typename M::v4;
  constexpr int DS = D / 32;
  constexpr int DT = D / 16;  // 16-column tiles of dK^T and dV^T
  constexpr int TILE = kTile * D;
  extern __shared__ __align__(16) unsigned char smem[];
  T* qs = reinterpret_cast<T*>(smem);              // [2][kTile][D] swizzled query rows
  T* dos = reinterpret_cast<T*>(smem) + 2 * TILE;  // [2][kTile][D] swizzled dO rows
  float* lse_s = reinterpret_cast<float*>(smem + 4 * TILE * sizeof(T));  // [2][kTile]
  float* dlt_s = lse_s + 2 * kTile;                                        // [2][kTile]

  // ---- workgroup -> (sequence, key block, key/value head); the first key blocks (the most queries) first ----
  const int H = a.heads, Hk = a.kv_heads, G = H / Hk;
  const int hk = blockIdx.x % Hk, slot = blockIdx.x / Hk;
  int n, kb, bos = 0, len = a.seq_len;
  if (a.cu_seqlens) {
    n = packed_slot_seq(a.cu_seqlens, a.n_seqs, a.seq_len, kKB, slot);
    bos = packed_begin(a.cu_seqlens, n, a.seq_len);
    len = packed_end(a.cu_seqlens, n, a.seq_len) - bos;
    const int nb = (len + kKB - 1) / kKB;
    kb = slot - packed_slot_base(a.cu_seqlens, n, a.seq_len, kKB);
    if (kb < 0 || kb >= nb) return;  // gap slot: uniform over the workgroup, before any barrier
  } else {
    n = slot % a.batch;
    kb = slot / a.batch;
  }
  const int bidx = a.cu_seqlens ? 0 : n;
  auto at = [&](const gdr_tensor& t, int head) {
    return static_cast<const T*>(t.ptr) + bidx * t.stride_b + head * t.stride_h + int64_t(bos) * t.stride_t;
  };
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l16 = lane & 15, g4 = lane >> 4;
  const int uwave = __builtin_amdgcn_readfirstlane(wave);
  const int key0 = kb * kKB, key = key0 + 16 * wave + l16;  // this lane's key (B-operand column)

  // The lane's key row of k and v as B operands: columns 32 ds + 8 g4 .. + 7.
  V8 kf[DS], vf[DS];
  {
    const int krow = min(key, len - 1);
    const T* kp = at(a.k, hk);
    const T* vp = at(a.v, hk);
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      kf[ds] = *reinterpret_cast<const V8*>(kp + int64_t(krow) * a.k.stride_t + 32 * ds + 8 * g4);
      vf[ds] = *reinterpret_cast<const V8*>(vp + int64_t(krow) * a.v.stride_t + 32 * ds + 8 * g4);
    }
  }

  // Iterations over (query head of the group, query tile from the diagonal on), each tile with its lse and delta
  // rows (waves 0 and 1: one 4-byte LDS DMA per lane; rows past the sequence end read its last row).
  const int nqt = (len + kTile - 1) / kTile, per = nqt - kb, total = G * per;
  attn::TileDma<D> dma;
  dma.init(uwave, lane);
  auto issue = [&](int it, int buf) {
    const int hq = hk * G + it / per, qt = kb + it % per;
    dma.issue(at(a.q, hq), a.q.stride_t, qt * kTile, len, qs + buf * TILE);
    dma.issue(at(g.d_out, hq), g.d_out.stride_t, qt * kTile, len, dos + buf * TILE);
    if (uwave < 2) {
      const float* src = (uwave == 0 ? a.lse : g.delta) + (int64_t(bidx) * H + hq) * a.seq_len + bos +
                         min(qt * kTile + lane, len - 1);
      float* dst = (uwave == 0 ? lse_s : dlt_s) + buf * kTile;
      __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)dst, 4, 0, 0);
    }
  };
  int koff[DS], toff[DT];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) koff[ds] = attn::row_frag<D>(ds, l16, g4);
#pragma unroll
  for (int t = 0; t < DT; ++t) toff[t] = attn::tr_frag<D>(t, l16, g4);
  const float c = a.scale * kLog2e;
  const uint32_t qlds = attn::lds_addr(qs), dlds = attn::lds_addr(dos);
  const uint32_t llds = attn::lds_addr(lse_s), dlds_rows = attn::lds_addr(dlt_s);

  if (total > 0) issue(0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  floatx4 dk[DT], dv[DT];  // dK^T, dV^T: lane holds columns 16 t + 4 g4 + i of key `key`
#pragma unroll
  for (int t = 0; t < DT; ++t) dk[t] = dv[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < total; ++it) {
    const int cur = it & 1;
    if (it + 1 < total) issue(it + 1, cur ^ 1);  // the other buffers were released by the last barrier
    const int qbase = (kb + it % per) * kTile;
    const T* qt = qs + cur * TILE;
    const T* dt = dos + cur * TILE;
    // S and dP: lane holds query qbase + 16 t + 4 g4 + i of key `key`
    floatx4 s[4], dp[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      s[t] = dp[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const V8 qa = *reinterpret_cast<const V8*>(qt + 16 * t * D + koff[ds]);
        const V8 da = *reinterpret_cast<const V8*>(dt + 16 * t * D + koff[ds]);
        s[t] = M::run(qa, kf[ds], s[t]);
        dp[t] = M::run(da, vf[ds], dp[t]);
      }
    }
    // P and dS = P (x) (dP - delta); only a tile crossing this wave's diagonal or the sequence end is masked
    const bool full = qbase >= key0 + 16 * wave + 15 && qbase + kTile <= len;
    V8 pf[2], dsf[2];
    floatx4 lr[4], dr[4];
    lds_rows4(llds + 4 * (cur * kTile + 4 * g4), dlds_rows + 4 * (cur * kTile + 4 * g4), lr, dr);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int q = qbase + 16 * t + 4 * g4 + i;
        float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][i], c, -lr[t][i]));
        if (!full && !(key <= q && q < len)) p = 0.f;
        s[t][i] = p;
        dp[t][i] = p * (dp[t][i] - dr[t][i]);
      }
    }
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      pf[s2] = cat<V4, V8>(M::pack(s[2 * s2]), M::pack(s[2 * s2 + 1]));
      dsf[s2] = cat<V4, V8>(M::pack(dp[2 * s2]), M::pack(dp[2 * s2 + 1]));
    }
    // dV^T += dO^T P and dK^T += Q^T dS: column tile t of the dO and Q tiles through the transposing read, one
    // tile ahead of its MFMAs (eight reads in flight: lgkmcnt(8) covers the current tile's)
    const uint32_t qaddr = qlds + 2 * cur * TILE, daddr = dlds + 2 * cur * TILE;
    short4 xd[2][4], xq[2][4];
    attn::tr_read4<D>(daddr + 2 * toff[0], xd[0]);
    attn::tr_read4<D>(qaddr + 2 * toff[0], xq[0]);
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      short4(&rd)[4] = xd[t & 1];
      short4(&rq)[4] = xq[t & 1];
      if (t + 1 < DT) {
        attn::tr_read4<D>(daddr + 2 * toff[t + 1], xd[(t + 1) & 1]);
        attn::tr_read4<D>(qaddr + 2 * toff[t + 1], xq[(t + 1) & 1]);
        asm volatile("s_waitcnt lgkmcnt(8)"
                     : "+v"(rd[0]), "+v"(rd[1]), "+v"(rd[2]), "+v"(rd[3]), "+v"(rq[0]), "+v"(rq[1]), "+v"(rq[2]),
                       "+v"(rq[3]));
      } else {
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(rd[0]), "+v"(rd[1]), "+v"(rd[2]), "+v"(rd[3]), "+v"(rq[0]), "+v"(rq[1]), "+v"(rq[2]),
                       "+v"(rq[3]));
      }
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        dv[t] = M::run(tr_pair<V4, V8>(rd, s2), pf[s2], dv[t]);
        dk[t] = M::run(tr_pair<V4, V8>(rq, s2), dsf[s2], dk[t]);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's copies of the next tiles have landed
    __syncthreads();                 // ... everyone's, and every wave is done with this step's buffers
  }

  if (key < len) {
    T* dkp = const_cast<T*>(at(g.d_k, hk)) + int64_t(key) * g.d_k.stride_t;
    T* dvp = const_cast<T*>(at(g.d_v, hk)) + int64_t(key) * g.d_v.stride_t;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      floatx4 y = dk[t];
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] *= a.scale;
      *reinterpret_cast<V4*>(dkp + 16 * t + 4 * g4) = M::pack(y);
      *reinterpret_cast<V4*>(dvp + 16 * t + 4 * g4) = M::pack(dv[t]);
    }
  }
}

template <int D, typename T>
hipError_t launch_attention_bwd_typed(const gdr_attention_args& a, const gdr_attention_grads& g, hipStream_t stream) {
  constexpr int dq_lds = 4 * kTile * D * int(sizeof(T));                      // K and V, double-buffered
  constexpr int kv_lds = 4 * kTile * D * int(sizeof(T)) + 4 * kTile * 4;      // q and dO, lse and delta, double-buffered
  hipError_t e = configure_lds<&attention_dq_kernel<D, T>>(dq_lds);
  if (e != hipSuccess) return e;
  e = configure_lds<&attention_dkdv_kernel<D, T>>(kv_lds);
  if (e != hipSuccess) return e;
  const int nqb = (a.seq_len + kQB - 1) / kQB, nkb = (a.seq_len + kKB - 1) / kKB;
  const int64_t qslots = a.cu_seqlens ? int64_t(nqb) + a.n_seqs : int64_t(a.batch) * nqb;
  const int64_t kslots = a.cu_seqlens ? int64_t(nkb) + a.n_seqs : int64_t(a.batch) * nkb;
  if (qslots * a.heads > 0)
    hipLaunchKernelGGL((attention_dq_kernel<D, T>), dim3(unsigned(qslots * a.heads)), dim3(attn::kThreads), dq_lds,
                       stream, a, g, nqb);
  if (kslots * a.kv_heads > 0)
    hipLaunchKernelGGL((attention_dkdv_kernel<D, T>), dim3(unsigned(kslots * a.kv_heads)), dim3(attn::kThreads),
                       kv_lds, stream, a, g, nkb);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_attention_bwd(const gdr_attention_args& a, const gdr_attention_grads& g, hipStream_t stream) {
  if (a.q.dtype == GDR_BF16)
    return a.head_dim == 64 ? launch_attention_bwd_typed<64, __bf16>(a, g, stream)
                            : launch_attention_bwd_typed<128, __bf16>(a, g, stream);
  return a.head_dim == 64 ? launch_attention_bwd_typed<64, _Float16>(a, g, stream)
                          : launch_attention_bwd_typed<128, _Float16>(a, g, stream);
}

}  // namespace gdr
