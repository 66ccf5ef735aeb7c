// Chunkwise (prefill) forward of the gated delta-rule family on gfx950: one fused launch.
//
// Reference: the forward of ChunkKimiDeltaAttention (src/ops/kimi_delta_attention.py:535-558), which runs
// chunk_cumsum (utils.py:15-23), two kernel-matrix launches (:71-106), the WY representation (:109-136), the
// sequential state scan (:139-170) and the output kernel (:173-197), materialising gate_cumsum, P, scores, A,
// W, U, u and a [B, H, NC+1, K, V] States tensor in HBM.  Gated DeltaNet, GLA and DeltaNet are the same chunk
// algebra with a scalar gate, no delta rule, or no gate (gated_deltanet.py:62-162, gated_linear_attention.py:
// 59-144, deltanet.py:60-149).
//
// Algebra per chunk of C = 64 tokens with state S entering it (b = in-chunk inclusive cumsum of the log gate):
//   P  = tril(K K^T (x) e^{b_t - b_s}, -1),  L = diag(beta) P,  A = (I + L)^{-1}
//   u  = A diag(beta) (V - (K e^b) S)                  (GLA: u = V)
//   O  = (scale Q e^b) S + tril(scale Q K^T (x) e^{b_t - b_s}) u
//   S' = diag(e^{b_end}) S + (K e^{b_end - b})^T u
// which is the reference's  W = A beta K e^b,  U = A beta V,  u = U - W S  with the product W S regrouped so W
// is never formed.
//
// MI355X design (one launch; one workgroup per (sequence, head) x 64-column value slice; 8 waves):
//   * Waves 4-7 are producers, waves 0-3 consumers, and the two groups run one chunk apart: in step s the
//     producers prepare chunk s while the consumers run the state recurrence of chunk s-1, so the VALU-heavy
//     preparation (gate cumsum, decay factors, operand scaling) overlaps the MFMA-heavy state chain on every
//     SIMD.  The only per-step workgroup barrier sits between steps; operands pass through a double-buffered
//     LDS region, and the producers hand off among themselves through an LDS counter.  Global loads of the
//     next chunk are issued a step ahead.
//   * Producer wave p owns the 16-row block p of a chunk.  Decay factors are anchored per 16-row block so that
//     every factor folded into an off-diagonal operand is <= 1 (the reference's secondary chunking,
//     kimi_delta_attention.py:84-100, with one anchor per query block instead of one per block pair).  Diagonal
//     blocks use the block-start anchor, whose key factor e^{-b} is bounded by the block's own decay span;
//     channels whose span exceeds kHotSpan are evaluated exactly elementwise instead (the reference always
//     evaluates diagonal blocks elementwise, utils.py:48-53).  Gated K K^T and Q K^T strips run on bf16 MFMA
//     (v_mfma_f32_16x16x32_bf16); the producers store the fp32 diagonal blocks of diag(beta) P and the
//     off-diagonal -diag(beta) P blocks as bf16.
//   * At the start of each step consumer wave w inverts the 16x16 unit lower-triangular diagonal block w of
//     (I + diag(beta) P) by fp32 forward substitution (16 lanes, one column each) and publishes it through a
//     second LDS counter, so the latency-bound substitution runs beside the producers' strips.
//   * Consumer wave w owns 16 state columns as an fp32 [K, 16] accumulator tile in registers for the whole
//     sequence (read from h0 once, written to ht once; no per-chunk state touches HBM).  K S and the Q S
//     readout take the state straight from the accumulator registers as the MFMA B operand (two accumulator
//     tiles form one 32-deep k slot set when the A operand is read with the same k permutation); the WY solve
//     is a blocked forward substitution on v_mfma_f32_16x16x16_bf16 from registers; the state update reads
//     (K e^{b_end - b})^T with the gfx950 transposing LDS read (ds_read_b64_tr_b16) from the row-major tile.
#include "chunk_common.h"
#include "varlen_index.h"
#include "gdr_internal.h"

namespace gdr {

using namespace chunk;

namespace {

constexpr int kSlice = 64;      // value columns per workgroup (4 waves x 16)

// LDS map.  Two consumer buffers (one per chunk parity) followed by the producer-private region.  Offsets of
// bf16 arrays are in elements from the buffer base; everything else is in bytes from the LDS base.
template <int K>
struct Lds {
  static constexpr int KP = K + 8;                // row pitch of [64][K] bf16 tiles (16-byte skew per row)
  // consumer buffer, bf16 part (every decay factor folded into these operands is <= 1)
  static constexpr int Lq = 0;                    // [64][KP] q e^{b - a_{blk-1}}   (block-start anchor)
  static constexpr int Lk = Lq + 64 * KP;         // [64][KP] k e^{b - a_{blk-1}}
  static constexpr int Kt = Lk + 64 * KP;         // [64][KP] k e^{b_end - b}       (chunk-end anchor)
  static constexpr int Sc = Kt + 64 * KP;         // 10 tiles [16][16]: gated scores, tile (i, j<=i)
  static constexpr int NegL = Sc + 10 * 256;      // 6 tiles [16][16]: -diag(beta) P, tile (i, j<i)
  static constexpr int Ainv = NegL + 6 * 256;     // 4 tiles [16][16]: (I + diag(beta) P_ii)^{-1}
  static constexpr int BF_END = Ainv + 4 * 256;
  static constexpr int BETA = ((BF_END * 2 + 15) / 16) * 16;  // fp32 [64]
  static constexpr int GAM = BETA + 64 * 4;                    // fp32 [K] e^{b_end}
  static constexpr int ABLK = GAM + K * 4;                     // fp32 [3][K] e^{a_i}, i = 0..2 (block ends)
  static constexpr int LII = ABLK + 3 * K * 4;                 // fp32 [4][16][16] strictly-lower diagonal blocks of L
  static constexpr int BUF = LII + 4 * 256 * 4;                // bytes per consumer buffer
  // producer-private region
  static constexpr int KAP = 2 * BUF;             // bf16 [64][KP] k e^{a_blk - b}  (block-end anchor)
  static constexpr int TOT = KAP + 64 * KP * 2;   // fp32 [2][4][K] per-block log2-gate totals, by chunk parity
  static constexpr int RDS = TOT + 2 * 4 * K * 4; // fp32 [4][K] e^{-T_blk} (0 for hot channels)
  static constexpr int FAR = RDS + 4 * K * 4;     // fp32 [3][K] key scalings of tiles (2,0), (3,0), (3,1)
  static constexpr int CNT = FAR + 3 * K * 4;     // int producer hand-off counter, int consumer hand-off counter
  static constexpr int BYTES = CNT + 16;
  static_assert(BYTES <= 160 * 1024, "LDS budget");
};

// Waves of one role hand off to each other through an LDS counter; every wave of the role arrives at every
// hand-off, so each wait ends.
__device__ __forceinline__ void producer_handoff(int* cnt, int target) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) __builtin_amdgcn_s_sleep(1);
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// ============================== producer: one wave per 16-row block PW of every chunk ==============================
template <int VARIANT, int K, int PW>
__device__ __forceinline__ void producer_loop(const ChunkCtx& x, unsigned char* smem) {
  constexpr bool kDelta = VARIANT != GDR_GLA;
  constexpr int kGate = (VARIANT == GDR_KDA || VARIANT == GDR_GLA) ? 2 : (VARIANT == GDR_GDN ? 1 : 0);
  constexpr int LPR = K / 8;       // producer lanes per row (8 channels each)
  constexpr int RSG = kWave / LPR; // row subgroups per producer wave
  constexpr int RPL = 16 / RSG;    // rows per producer lane
  constexpr int KS = K / 32;       // k-steps of 32 channels
  constexpr int NVEC = 11;         // per-chunk channel vectors: RDS[4], FAR[3], ABLK[3], GAM
  using M = Lds<K>;
  constexpr int KP = M::KP;
  constexpr float kHot = kHotSpan * kLog2e;  // hot threshold on -T in log2 units

  const int lane = threadIdx.x & 63;
  const int ptid = PW * 64 + lane;  // 0..255 over the producer waves
  const int cg = lane % LPR, rs = lane / LPR, c0 = 8 * cg;
  const int l16 = lane & 15, g4 = lane >> 4;
  constexpr int kRow0 = 16 * PW;
  const int row0 = kRow0 + rs * RPL;  // chunk-local row of this lane's first element
  __bf16* kap = reinterpret_cast<__bf16*>(smem + M::KAP);
  float* tot = reinterpret_cast<float*>(smem + M::TOT);
  float* rds = reinterpret_cast<float*>(smem + M::RDS);
  float* far = reinterpret_cast<float*>(smem + M::FAR);
  int* cnt = reinterpret_cast<int*>(smem + M::CNT);
  const int len = x.len, nchunks = x.nchunks;

  uint4 cq[RPL], ck[RPL];
  float bl[RPL][8], cb[RPL];
  // Loads are unconditional from clamped rows (len >= 1 whenever a chunk exists) and only consumed later: the
  // row mask and the log2 scaling are applied where the values are used, so no load is waited on at issue.
  auto load_qk = [&](int chunk) {
#pragma unroll
    for (int j = 0; j < RPL; ++j) {
      const int tc = min(chunk * kChunk + row0 + j, len - 1);
      cq[j] = *reinterpret_cast<const uint4*>(x.qp + tc * x.q_st + c0);
      ck[j] = *reinterpret_cast<const uint4*>(x.kp + tc * x.k_st + c0);
      if constexpr (kDelta) cb[j] = x.betap[tc * x.b_st];
    }
  };
  auto load_g = [&](int chunk, float (*rg)[8]) {  // raw gate rows
#pragma unroll
    for (int j = 0; j < RPL; ++j) {
      const int tc = min(chunk * kChunk + row0 + j, len - 1);
      if constexpr (kGate == 2) {
        const float4 g0 = *reinterpret_cast<const float4*>(x.gp + tc * x.g_st + c0);
        const float4 g1 = *reinterpret_cast<const float4*>(x.gp + tc * x.g_st + c0 + 4);
        rg[j][0] = g0.x; rg[j][1] = g0.y; rg[j][2] = g0.z; rg[j][3] = g0.w;
        rg[j][4] = g1.x; rg[j][5] = g1.y; rg[j][6] = g1.z; rg[j][7] = g1.w;
      } else if constexpr (kGate == 1) {
        const float g = x.gp[tc * x.g_st];
#pragma unroll
        for (int c = 0; c < 8; ++c) rg[j][c] = g;
      } else {
#pragma unroll
        for (int c = 0; c < 8; ++c) rg[j][c] = 0.f;
      }
    }
  };
  // in-block inclusive prefix of the log2 gate; block totals to tot[slot]
  auto scan = [&](int chunk, int slot) {
    if constexpr (kGate) {
#pragma unroll
      for (int j = 0; j < RPL; ++j) {
        const float keep = chunk * kChunk + row0 + j < len ? kLog2e : 0.f;
#pragma unroll
        for (int c = 0; c < 8; ++c) bl[j][c] *= keep;
      }
#pragma unroll
      for (int j = 1; j < RPL; ++j)
#pragma unroll
        for (int c = 0; c < 8; ++c) bl[j][c] += bl[j - 1][c];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const float own = bl[RPL - 1][c];
        float incl = own;
#pragma unroll
        for (int off = LPR; off < kWave; off *= 2) {
          const float y = __shfl_up(incl, off, kWave);
          if (lane >= off) incl += y;
        }
        const float excl = incl - own;
#pragma unroll
        for (int j = 0; j < RPL; ++j) bl[j][c] += excl;
      }
      if (rs == RSG - 1) {
        *reinterpret_cast<float4*>(tot + (slot * 4 + PW) * K + c0) =
            make_float4(bl[RPL - 1][0], bl[RPL - 1][1], bl[RPL - 1][2], bl[RPL - 1][3]);
        *reinterpret_cast<float4*>(tot + (slot * 4 + PW) * K + c0 + 4) =
            make_float4(bl[RPL - 1][4], bl[RPL - 1][5], bl[RPL - 1][6], bl[RPL - 1][7]);
      }
    }
  };

  if (nchunks > 0) {
    load_qk(0);
    load_g(0, bl);
    scan(0, 0);
  }
  __syncthreads();

  for (int s = 0; s <= nchunks; ++s) {
    if (s < nchunks) {
      const int slot = s & 1;
      __bf16* buf = reinterpret_cast<__bf16*>(smem + slot * M::BUF);
      float* bbeta = reinterpret_cast<float*>(smem + slot * M::BUF + M::BETA);
      float* bgam = reinterpret_cast<float*>(smem + slot * M::BUF + M::GAM);
      float* ablk = reinterpret_cast<float*>(smem + slot * M::BUF + M::ABLK);
      const float* ts = tot + slot * 4 * K;

      // ---- per-chunk channel vectors, computed once and spread over the 256 producer lanes ----
      for (int idx = ptid; idx < NVEC * K; idx += 256) {
        const int v = idx / K, c = idx % K;
        float tb[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) tb[m] = kGate ? ts[m * K + c] : 0.f;
        if (v < 4) {         // RDS[m] = e^{-T_m}, 0 for hot channels
          const float t = tb[v];
          rds[v * K + c] = -t > kHot ? 0.f : __builtin_amdgcn_exp2f(-t);
        } else if (v < 7) {  // FAR: tiles (2,0), (3,0), (3,1)
          const float e = v == 4 ? tb[1] : (v == 5 ? tb[1] + tb[2] : tb[2]);
          far[(v - 4) * K + c] = __builtin_amdgcn_exp2f(e);
        } else if (v < 10) {  // ABLK[i] = e^{a_i}
          const int i = v - 7;
          float upto = 0.f;
#pragma unroll
          for (int m = 0; m < 4; ++m) upto += m <= i ? tb[m] : 0.f;
          ablk[i * K + c] = __builtin_amdgcn_exp2f(upto);
        } else {              // GAM = e^{b_end}
          bgam[c] = __builtin_amdgcn_exp2f(tb[0] + tb[1] + tb[2] + tb[3]);
        }
      }
      if constexpr (kDelta) {
        if (cg == 0) {
#pragma unroll
          for (int j = 0; j < RPL; ++j) bbeta[row0 + j] = s * kChunk + row0 + j < len ? cb[j] : 0.f;
        }
      }
      producer_handoff(cnt, 4 * (2 * s + 1));

      // ---- operands of chunk s ----
      float tw[8], eb[8];
      uint32_t hot_mask = 0;
      {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          tw[c] = 0.f;
          eb[c] = 1.f;
        }
        if constexpr (kGate) {
          float tail[8];
#pragma unroll
          for (int c = 0; c < 8; ++c) tail[c] = 0.f;
#pragma unroll
          for (int m = PW; m < 4; ++m) {
            const float4 t0 = *reinterpret_cast<const float4*>(ts + m * K + c0);
            const float4 t1 = *reinterpret_cast<const float4*>(ts + m * K + c0 + 4);
            const float tv[8] = {t0.x, t0.y, t0.z, t0.w, t1.x, t1.y, t1.z, t1.w};
#pragma unroll
            for (int c = 0; c < 8; ++c) {
              if (m == PW) tw[c] = tv[c];
              else tail[c] += tv[c];
            }
          }
#pragma unroll
          for (int c = 0; c < 8; ++c) eb[c] = PW == 3 ? 1.f : __builtin_amdgcn_exp2f(tail[c]);
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) hot_mask |= (kGate && -tw[c] > kHot) ? (1u << c) : 0u;
      }
#pragma unroll
      for (int j = 0; j < RPL; ++j) {
        const int row = row0 + j;
        float qf[8], kf[8];
        const uint32_t keep = s * kChunk + row < len ? 0xffffffffu : 0u;
        unpack8(make_uint4(cq[j].x & keep, cq[j].y & keep, cq[j].z & keep, cq[j].w & keep), qf);
        unpack8(make_uint4(ck[j].x & keep, ck[j].y & keep, ck[j].z & keep, ck[j].w & keep), kf);
        bf16x8 lq, lk, kv, kt;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          float ell = 1.f, rho = 1.f;
          if constexpr (kGate) {
            ell = __builtin_amdgcn_exp2f(bl[j][c]);
            rho = __builtin_amdgcn_exp2f(tw[c] - bl[j][c]);
          }
          const float kapf = kf[c] * rho;
          lq[c] = bf(qf[c] * ell);
          lk[c] = bf(kf[c] * ell);
          kv[c] = bf(kapf);
          kt[c] = bf(kapf * eb[c]);
        }
        *reinterpret_cast<bf16x8*>(buf + M::Lq + row * KP + c0) = lq;
        *reinterpret_cast<bf16x8*>(buf + M::Lk + row * KP + c0) = lk;
        *reinterpret_cast<bf16x8*>(buf + M::Kt + row * KP + c0) = kt;
        *reinterpret_cast<bf16x8*>(kap + row * KP + c0) = kv;
      }
      if (s + 1 < nchunks) {  // raw rows of chunk s + 1 land while the strips run
        load_qk(s + 1);
        load_g(s + 1, bl);
      }
      producer_handoff(cnt, 4 * (2 * s + 2));

      // ---- gated strips: the 10 tiles (i, j <= i) of Sc and P, balanced over the producer waves; each wave
      // owns the diagonal tile of its own block ----
      float* lii = reinterpret_cast<float*>(smem + slot * M::BUF + M::LII) + PW * 256;
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        constexpr int kJobs[4][3][2] = {{{0, 0}, {3, 0}, {2, 1}}, {{1, 1}, {3, 1}, {1, 0}},
                                        {{2, 2}, {2, 0}, {-1, -1}}, {{3, 3}, {3, 2}, {-1, -1}}};
        const int i = kJobs[PW][q][0], j = kJobs[PW][q][1];
        if (i < 0) continue;
        // key operand of tile (i, j): k e^{a_{i-1} - b} = Kap_j scaled by e^{a_{i-1} - a_j} (<= 1) or, on the
        // diagonal, by e^{-T_i} (>= 1, bounded by the block span; 0 for hot channels)
        const bool diag = j == i, adjacent = j + 1 == i;
        const float* kscale = diag ? rds + i * K : far + ((i == 2) ? 0 : (j == 0 ? 1 : 2)) * K;
        floatx4 acc_s = {0.f, 0.f, 0.f, 0.f}, acc_p = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
          const int kc = 32 * kk + 8 * g4;
          bf16x8 bk = *reinterpret_cast<const bf16x8*>(kap + (16 * j + l16) * KP + kc);
          if (!adjacent) {
            const float4 f0 = *reinterpret_cast<const float4*>(kscale + kc);
            const float4 f1 = *reinterpret_cast<const float4*>(kscale + kc + 4);
            const float f[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
#pragma unroll
            for (int c = 0; c < 8; ++c) bk[c] = bf(f32(bk[c]) * f[c]);
          }
          const bf16x8 aq = *reinterpret_cast<const bf16x8*>(buf + M::Lq + (16 * i + l16) * KP + kc);
          acc_s = mfma32(aq, bk, acc_s);
          if constexpr (kDelta) {
            const bf16x8 ak = *reinterpret_cast<const bf16x8*>(buf + M::Lk + (16 * i + l16) * KP + kc);
            acc_p = mfma32(ak, bk, acc_p);
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tloc = 4 * g4 + r, sloc = l16;
          float sv = acc_s[r];
          if (diag && tloc < sloc) sv = 0.f;
          buf[M::Sc + tri_tile(i, j) * 256 + tloc * 16 + sloc] = bf(sv);
          if constexpr (kDelta) {
            const float p = acc_p[r] * bbeta[16 * i + tloc];
            if (!diag) buf[M::NegL + strict_tile(i, j) * 256 + tloc * 16 + sloc] = bf(-p);
            else lii[tloc * 16 + sloc] = tloc > sloc ? p : 0.f;
          }
        }
      }
      // exact elementwise diagonal block for hot channels (rare)
      if constexpr (kGate) {
        if (__any(hot_mask != 0)) {
          __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
          hot_diag_fixup<K, kDelta>(s * kChunk, PW, x.len, hot_mask, buf + M::Sc + tri_tile(PW, PW) * 256, lii,
                                    bbeta + kRow0, InputRows{x, kGate});
        }
      }
      // ---- chunk s + 1 becomes current ----
      if (s + 1 < nchunks) scan(s + 1, (s + 1) & 1);
    }
    __syncthreads();
  }
}

// ============================== consumer: one wave per 16 state columns ==============================
template <int VARIANT, int K, typename OutT>
__device__ __forceinline__ void consumer_loop(const ChunkCtx& x, unsigned char* smem, int cw) {
  constexpr bool kDelta = VARIANT != GDR_GLA;
  constexpr int KT = K / 16;  // 16-channel tiles of the state
  constexpr int KS = K / 32;  // k-steps of 32 channels
  using M = Lds<K>;
  constexpr int KP = M::KP;
  const int lane = threadIdx.x & 63;
  const int l16 = lane & 15, g4 = lane >> 4;
  const int col = x.v0 + 16 * cw + l16;
  const int len = x.len, nchunks = x.nchunks;
  OutT* op = static_cast<OutT*>(x.op);
  int* ccnt = reinterpret_cast<int*>(smem + M::CNT) + 1;  // consumer hand-off counter

  floatx4 st[KT];
#pragma unroll
  for (int m = 0; m < KT; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) st[m][r] = x.h0 ? x.h0[x.sbase + size_t(16 * m + 4 * g4 + r) * x.V + col] : 0.f;
  // value tile of the next chunk in accumulator layout (row 16 i + 4 g4 + r), loaded unconditionally from
  // clamped rows; rows past the end are zeroed when consumed
  uint16_t vn[4][4];
  auto load_v = [&](int chunk) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = min(chunk * kChunk + 16 * i + 4 * g4 + r, len - 1);
        vn[i][r] = reinterpret_cast<const uint16_t*>(x.vp)[t * x.v_st + col];
      }
  };
  if (nchunks > 0) load_v(0);
  __syncthreads();

  for (int s = 0; s <= nchunks; ++s) {
    if (s >= 1) {
      const int c = s - 1, slot = c & 1;
      const __bf16* buf = reinterpret_cast<const __bf16*>(smem + slot * M::BUF);
      const float* bbeta = reinterpret_cast<const float*>(smem + slot * M::BUF + M::BETA);
      const float* bgam = reinterpret_cast<const float*>(smem + slot * M::BUF + M::GAM);
      const float* ablk = reinterpret_cast<const float*>(smem + slot * M::BUF + M::ABLK);
      if constexpr (kDelta) {
        // diagonal block cw of A: column `lane` of (I + L_cw)^{-1} by forward substitution in fp32, shared with
        // the other consumer waves through LDS
        const float* lii = reinterpret_cast<const float*>(smem + slot * M::BUF + M::LII) + cw * 256;
        __bf16* ainv = const_cast<__bf16*>(buf) + M::Ainv + cw * 256;
        if (lane < 16) {
          float xcol[16];
          xcol[0] = lane == 0 ? 1.f : 0.f;
#pragma unroll
          for (int r = 1; r < 16; ++r) {
            float lrow[16];
#pragma unroll
            for (int m4 = 0; m4 < (r + 3) / 4; ++m4) {
              const float4 v = *reinterpret_cast<const float4*>(lii + r * 16 + 4 * m4);
              lrow[4 * m4] = v.x; lrow[4 * m4 + 1] = v.y; lrow[4 * m4 + 2] = v.z; lrow[4 * m4 + 3] = v.w;
            }
            float acc0 = (r == lane) ? 1.f : 0.f, acc1 = 0.f;
#pragma unroll
            for (int m = 0; m < r; m += 2) {
              acc0 -= lrow[m] * xcol[m];
              if (m + 1 < r) acc1 -= lrow[m + 1] * xcol[m + 1];
            }
            xcol[r] = acc0 + acc1;
          }
#pragma unroll
          for (int r = 0; r < 16; ++r) ainv[r * 16 + lane] = bf(xcol[r]);
        }
        producer_handoff(ccnt, 4 * s);
      }
      float vc[4][4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          vc[i][r] = (c * kChunk + 16 * i + 4 * g4 + r < len) ? bf16_bits_to_f32(vn[i][r]) : 0.f;
      if (c + 1 < nchunks) load_v(c + 1);

      floatx4 acc_o[4], yv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // state operand of query block i: diag(e^{a_{i-1}}) S in bf16 (block-start anchor of Lq/Lk)
        bf16x8 sB[KS];
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
          floatx4 lo = st[2 * kk], hi = st[2 * kk + 1];
          if (i > 0) {
            const float4 f0 = *reinterpret_cast<const float4*>(ablk + (i - 1) * K + 32 * kk + 4 * g4);
            const float4 f1 = *reinterpret_cast<const float4*>(ablk + (i - 1) * K + 32 * kk + 16 + 4 * g4);
            lo[0] *= f0.x; lo[1] *= f0.y; lo[2] *= f0.z; lo[3] *= f0.w;
            hi[0] *= f1.x; hi[1] *= f1.y; hi[2] *= f1.z; hi[3] *= f1.w;
          }
          sB[kk] = concat(pack4(lo), pack4(hi));
        }
        floatx4 ax = {0.f, 0.f, 0.f, 0.f}, ao = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
          const int r0 = (16 * i + l16) * KP + 32 * kk + 4 * g4;
          const bf16x8 aq = concat(*reinterpret_cast<const bf16x4*>(buf + M::Lq + r0),
                                   *reinterpret_cast<const bf16x4*>(buf + M::Lq + r0 + 16));
          ao = mfma32(aq, sB[kk], ao);
          if constexpr (kDelta) {
            const bf16x8 ak = concat(*reinterpret_cast<const bf16x4*>(buf + M::Lk + r0),
                                     *reinterpret_cast<const bf16x4*>(buf + M::Lk + r0 + 16));
            ax = mfma32(ak, sB[kk], ax);
          }
        }
        acc_o[i] = ao;
#pragma unroll
        for (int r = 0; r < 4; ++r) yv[i][r] = kDelta ? bbeta[16 * i + 4 * g4 + r] * (vc[i][r] - ax[r]) : vc[i][r];
      }
      bf16x4 ub[4];
      if constexpr (kDelta) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          floatx4 z = yv[i];
#pragma unroll
          for (int j = 0; j < i; ++j) {
            const bf16x4 nl =
                *reinterpret_cast<const bf16x4*>(buf + M::NegL + strict_tile(i, j) * 256 + l16 * 16 + 4 * g4);
            z = mfma16(nl, ub[j], z);
          }
          const bf16x4 ai = *reinterpret_cast<const bf16x4*>(buf + M::Ainv + i * 256 + l16 * 16 + 4 * g4);
          const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
          ub[i] = pack4(mfma16(ai, pack4(z), zero));
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) ub[i] = pack4(yv[i]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j <= i; ++j) {
          const bf16x4 sc = *reinterpret_cast<const bf16x4*>(buf + M::Sc + tri_tile(i, j) * 256 + l16 * 16 + 4 * g4);
          acc_o[i] = mfma16(sc, ub[j], acc_o[i]);
        }
      }
      // S = diag(gamma) S + Kt^T u, Kt^T read transposed from the row-major tile
#pragma unroll
      for (int m = 0; m < KT; ++m) {
        const float4 gm = *reinterpret_cast<const float4*>(bgam + 16 * m + 4 * g4);
        st[m][0] *= gm.x; st[m][1] *= gm.y; st[m][2] *= gm.z; st[m][3] *= gm.w;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const int tok = 32 * kk + 4 * g4 + (l16 >> 2);
          const int chn = 16 * m + 4 * (l16 & 3);
          const int off = (M::Kt + tok * KP + chn) * 2 + slot * M::BUF;
          const bf16x8 ak = concat(lds_read_tr(smem, off), lds_read_tr(smem, off + 16 * KP * 2));
          st[m] = mfma32(ak, concat(ub[2 * kk], ub[2 * kk + 1]), st[m]);
        }
      }
      // output rows of chunk c
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = c * kChunk + 16 * i + 4 * g4 + r;
          if (t < len) op[t * x.o_st + col] = static_cast<OutT>(x.scale * acc_o[i][r]);
        }
    }
    __syncthreads();
  }
  if (x.ht) {
#pragma unroll
    for (int m = 0; m < KT; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) x.ht[x.sbase + size_t(16 * m + 4 * g4 + r) * x.V + col] = st[m][r];
  }
}

}  // namespace

template <int VARIANT, int K, typename OutT>
__global__ __launch_bounds__(512, 1) void chunk_fwd_kernel(const gdr_args a, int n_slices, int xcd_map) {
  constexpr bool kDelta = VARIANT != GDR_GLA;
  constexpr int kGate = (VARIANT == GDR_KDA || VARIANT == GDR_GLA) ? 2 : (VARIANT == GDR_GDN ? 1 : 0);
  using M = Lds<K>;
  extern __shared__ __align__(16) unsigned char smem[];

  // ---- workgroup -> (sequence, head, value slice); XCD-aware so the slices of one head share an L2 ----
  const int xb = blockIdx.x;
  int bh, slice;
  if (xcd_map) {
    const int xcd = xb & 7, local = xb >> 3;
    slice = local % n_slices;
    bh = (local / n_slices) * 8 + xcd;
  } else {
    slice = xb % n_slices;
    bh = xb / n_slices;
  }
  const int H = a.heads;
  const int n = bh / H, h = bh % H;
  int bos = 0, len = a.seq_len, bidx = n;
  if (a.cu_seqlens) {
    bos = packed_begin(a.cu_seqlens, n, a.seq_len);
    len = packed_end(a.cu_seqlens, n, a.seq_len) - bos;
    bidx = 0;
  }
  ChunkCtx x;
  x.q_st = a.q.stride_t; x.k_st = a.k.stride_t; x.v_st = a.v.stride_t; x.o_st = a.out.stride_t;
  x.g_st = a.gate.stride_t; x.b_st = a.beta.stride_t;
  x.qp = static_cast<const __bf16*>(a.q.ptr) + bidx * a.q.stride_b + h * a.q.stride_h + bos * x.q_st;
  x.kp = static_cast<const __bf16*>(a.k.ptr) + bidx * a.k.stride_b + h * a.k.stride_h + bos * x.k_st;
  x.vp = static_cast<const __bf16*>(a.v.ptr) + bidx * a.v.stride_b + h * a.v.stride_h + bos * x.v_st;
  x.gp = kGate ? static_cast<const float*>(a.gate.ptr) + bidx * a.gate.stride_b + h * a.gate.stride_h + bos * x.g_st
               : nullptr;
  x.betap = kDelta ? static_cast<const float*>(a.beta.ptr) + bidx * a.beta.stride_b + h * a.beta.stride_h +
                         bos * x.b_st
                   : nullptr;
  x.op = static_cast<OutT*>(const_cast<void*>(a.out.ptr)) + bidx * a.out.stride_b + h * a.out.stride_h +
         bos * x.o_st;
  x.len = len;
  x.nchunks = (len + kChunk - 1) / kChunk;
  x.v0 = slice * kSlice;
  x.V = a.value_dim;
  x.sbase = size_t(n * H + h) * K * a.value_dim;
  x.h0 = a.h0;
  x.ht = a.ht;
  x.scale = a.scale;

  const int wave = threadIdx.x >> 6;
  if (threadIdx.x == 0) {
    reinterpret_cast<int*>(smem + M::CNT)[0] = 0;
    reinterpret_cast<int*>(smem + M::CNT)[1] = 0;
  }
  switch (wave) {
    case 4: producer_loop<VARIANT, K, 0>(x, smem); break;
    case 5: producer_loop<VARIANT, K, 1>(x, smem); break;
    case 6: producer_loop<VARIANT, K, 2>(x, smem); break;
    case 7: producer_loop<VARIANT, K, 3>(x, smem); break;
    default: consumer_loop<VARIANT, K, OutT>(x, smem, wave); break;
  }
}

namespace {

template <int VARIANT, int K, typename OutT>
hipError_t launch_typed(const gdr_args& a, hipStream_t stream) {
  const int n_seq = a.cu_seqlens ? a.n_seqs : a.batch;
  const int bh = n_seq * a.heads;
  const int n_slices = a.value_dim / kSlice;
  const int xcd_map = (bh % 8 == 0) ? 1 : 0;
  constexpr int bytes = Lds<K>::BYTES;
  const hipError_t e = configure_lds<&chunk_fwd_kernel<VARIANT, K, OutT>>(bytes);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((chunk_fwd_kernel<VARIANT, K, OutT>), dim3(bh * n_slices), dim3(512), bytes, stream, a,
                     n_slices, xcd_map);
  return hipGetLastError();
}

template <int VARIANT, int K>
hipError_t launch_k(const gdr_args& a, hipStream_t stream) {
  switch (a.out.dtype) {
    case GDR_BF16: return launch_typed<VARIANT, K, __bf16>(a, stream);
    case GDR_F16: return launch_typed<VARIANT, K, _Float16>(a, stream);
    default: return launch_typed<VARIANT, K, float>(a, stream);
  }
}

template <int VARIANT>
hipError_t launch_v(const gdr_args& a, hipStream_t stream) {
  return a.key_dim == 64 ? launch_k<VARIANT, 64>(a, stream) : launch_k<VARIANT, 128>(a, stream);
}

}  // namespace

hipError_t launch_chunk(const gdr_args& a, hipStream_t stream) {
  if (a.q.dtype != GDR_BF16) return hipErrorInvalidValue;  // the Python layer converts q, k, v to bf16
  switch (a.variant) {
    case GDR_KDA: return launch_v<GDR_KDA>(a, stream);
    case GDR_GDN: return launch_v<GDR_GDN>(a, stream);
    case GDR_GLA: return launch_v<GDR_GLA>(a, stream);
    default: return launch_v<GDR_DELTANET>(a, stream);
  }
}

}  // namespace gdr
