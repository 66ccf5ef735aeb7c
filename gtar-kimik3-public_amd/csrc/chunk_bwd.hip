// Chunkwise backward of the gated delta-rule family on gfx950.
//
// Reference: ChunkKimiDeltaAttention.backward (src/ops/kimi_delta_attention.py:560-622) and its kernels
// _chunk_intra_backward, _chunk_state_backward, _chunk_backward_dq, _chunk_backward_dk,
// _chunk_backward_wy_representation, _chunk_backward_kernel_matrix and _chunk_gate_gradient (:200-492); the
// Gated DeltaNet, GLA and DeltaNet twins (gated_deltanet.py:419, gated_linear_attention.py:387, deltanet.py:350).
//
// Forward per chunk (S entering it, B the in-chunk cumsum of the log gate, E_ts = e^{B_t - B_s} per channel):
//   P = tril(K K^T (x) E, -1),  A = (I + diag(beta) P)^{-1},  W = A diag(beta) K e^B,  U = A diag(beta) V
//   u = U - W S,  O = (scale Q e^B) S + Sc u with Sc = scale tril(Q K^T (x) E),  S' = diag(e^{B_end}) S + Kt^T u,
//   Kt = K e^{B_end - B}.
// Backward, given dO and dS' (the gradient of the state leaving the chunk):
//   du = Sc^T dO + Kt dS',   dS = (scale Q e^B)^T dO + diag(e^{B_end}) dS' - W^T du            (reverse scan)
//   dQd = dO S^T,  dW = -du S^T,  dKt = u dS'^T,  dSc = tril(dO u^T),  rowsum(S' (x) dS')         (state products)
//   dA = dW (beta K e^B)^T + du (beta V)^T,  dL = -A^T dA A^T (strictly lower),  dP = diag(beta) dL,
//   dbeta = rowsum(dL (x) P) + rowsum(A^T dW (x) K e^B) + rowsum(A^T du (x) V),
//   dk += beta e^B (x) A^T dW,  dv = beta (x) A^T du,
//   the four gated products  dq += scale dSc (K..E),  dk += scale dSc^T (Q..E) + dP (K..E) + dP^T (K..E),
//   dq += scale dQd (x) e^B,  dk += dKt (x) e^{B_end - B},
//   dg = reverse cumsum over the chunk of (q dq + k dk_{e^{+B} roles} - k dk_{e^{-B} roles}) + rowsum(S' (x) dS')
//      (the reference's form, :480-492), evaluated as reverse cumsum of the terms other than the Kt role
//      + e^{B_end} rowsum(S (x) dS') + exclusive forward cumsum of k dKt e^{B_end - B}: the two agree exactly because
//      S' = e^{B_end} S + Kt^T u, and this one has no cancellation between a large boundary term and the Kt-role sum.
// (GLA: no beta, W = 0, dv = du.  GDN: the gate gradient sums over channels.  DeltaNet: no gate.)
//
// Launches: the forward record and a state recompute (chunk_split.hip, states mode), then here
//   chunk_dscan_kernel   reverse scan over chunks with dS in registers; writes dS' per chunk and du
//   chunk_sprod_kernel   per (chunk, head): the products with S, S' and dS' (MFMA, k = value dim)
//   chunk_grad_kernel    per (chunk, head): everything chunk-local
#include "chunk_common.h"
#include "gdr_internal.h"
#include "split_common.h"

namespace gdr {

using namespace chunk;

namespace {

constexpr int kDScanThreads = 512;  // 4 compute waves of 16 value columns + 4 DMA loader waves

// Position of the 4-channel block [c, c + 4) (c % 4 == 0) in a row of the permuted W / Q e^B record layout:
// within a 32-channel group, channel 4 g + j sits at 8 g + j and channel 16 + 4 g + j at 8 g + 4 + j.
__device__ __forceinline__ int perm_pos(int c) { return (c & ~31) + 8 * ((c & 15) >> 2) + 4 * ((c >> 4) & 1); }

__device__ __forceinline__ bf16x8 ld8(const __bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ bf16x4 ld4(const __bf16* p) { return *reinterpret_cast<const bf16x4*>(p); }

// ============================ reverse state scan: one workgroup per (sequence, head) x 64 columns ============================
// Per chunk c (last to first), each compute wave holds dS' = dS_{c+1} for 16 value columns in registers:
//   du = Sc^T dO + Kt dS'  (row blocks i: Kt rows on 16x16x32 MFMAs with dS' as the two-tile B operand, Sc^T tiles
//   and dO blocks through the transposing LDS read on 16x16x16 MFMAs), then
//   dS = diag(gamma) dS' + Qd^T dO - W^T du  (Qd^T, W^T read transposed from the permuted record rows).
// The loader waves stream the next record (W, Q e^B, Kt, Sc, gamma) and the dO slice into the other LDS buffer.
template <int VARIANT, int K>
__global__ __launch_bounds__(kDScanThreads, 1) void chunk_dscan_kernel(const gdr_args a, const gdr_grads g, int n_slices,
                                                                       int xcd_map, int nc, int64_t rec_bytes,
                                                                       const unsigned char* __restrict__ rec_ws,
                                                                       float* __restrict__ dstates,
                                                                       __bf16* __restrict__ dubuf) {
  constexpr bool kDelta = VARIANT != GDR_GLA;
  constexpr int KT = K / 16, KS = K / 32;
  using R = Rec<K>;
  constexpr int DO = R::FIX;                           // dO slice: bf16 [64][64], 16-byte chunks swizzled by row
  constexpr int SB = R::FIX + kChunk * kScanSlice * 2;  // LDS bytes per buffer
  constexpr int NF = R::FIX / 16, NDO = kChunk * kScanSlice * 2 / 16;
  constexpr int NG = ((NF + NDO + 63) / 64 + 3) / 4;   // 64-piece groups per loader wave
  extern __shared__ __align__(16) unsigned char smem[];

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
  const int H = a.heads, V = a.value_dim, len = a.seq_len;
  const int n = bh / H, h = bh % H;
  const int v0 = slice * kScanSlice;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;

  if (wave >= 4) {
    // ---------------- loader waves ----------------
    const int lw = wave - 4;
    const unsigned char* rec0 = rec_ws + (int64_t(n) * nc * H + h) * rec_bytes;
    const int64_t rec_stride = int64_t(H) * rec_bytes;
    const __bf16* dop = static_cast<const __bf16*>(g.d_out.ptr) + n * g.d_out.stride_b + h * g.d_out.stride_h;
    auto copy = [&](int c, int buf) {
      const unsigned char* src = rec0 + c * rec_stride;
      unsigned char* dst = smem + buf * SB;
#pragma unroll
      for (int k = 0; k < NG; ++k) {
        const int grp = lw + 4 * k;
        const int idx = 64 * grp + lane;
        if (idx < NF + NDO) {
          const void* from;
          if (idx < NF) {
            from = src + idx * 16;
          } else {
            const int p = idx - NF, row = p >> 3, q = (p & 7) ^ (row & 7);  // stored slot p & 7 holds chunk q
            const int t = min(c * kChunk + row, len - 1);                   // clamped rows meet zero Qd/Sc rows
            from = dop + int64_t(t) * g.d_out.stride_t + v0 + 8 * q;
          }
          __builtin_amdgcn_global_load_lds(from, (__attribute__((address_space(3))) void*)(dst + 1024 * grp), 16, 0, 0);
        }
      }
    };
    if (nc > 0) copy(nc - 1, 0);
    __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
    for (int q = 0; q < nc; ++q) {
      if (q + 1 < nc) copy(nc - 2 - q, (q + 1) & 1);
      __builtin_amdgcn_s_waitcnt(0);
      lds_barrier();
    }
    return;
  }

  // ---------------- compute waves ----------------
  const int l16 = lane & 15, g4 = lane >> 4;
  const int lc0 = 16 * wave, c0 = v0 + lc0;
  const size_t kv = size_t(K) * V;
  floatx4 st[KT];
#pragma unroll
  for (int m = 0; m < KT; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      st[m][r] = g.d_final ? g.d_final[bh * kv + size_t(16 * m + 4 * g4 + r) * V + c0 + l16] : 0.f;
  lds_barrier();

  for (int q = 0; q < nc; ++q) {
    const int c = nc - 1 - q;
    const int boff = (q & 1) * SB;
    const __bf16* bb = reinterpret_cast<const __bf16*>(smem + boff);
    const float* gam = reinterpret_cast<const float*>(smem + boff + R::GAM);

    // dS' of this chunk, kept for the chunk-local kernels
    float* dsp = dstates + (size_t(bh) * (nc + 1) + c + 1) * kv;
#pragma unroll
    for (int m = 0; m < KT; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) dsp[size_t(16 * m + 4 * g4 + r) * V + c0 + l16] = st[m][r];

    bf16x8 sB[KS];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) sB[kk] = concat(pack4(st[2 * kk]), pack4(st[2 * kk + 1]));
    // dO blocks as 16x16x16 B operands: lane (column l16, k = 4 g4 + r) holds dO[16 i + 4 g4 + r][lc0 + l16]
    bf16x4 dob[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * i + 4 * g4 + (l16 >> 2), col = lc0 + 4 * (l16 & 3);
      dob[i] = lds_read_tr(smem, boff + DO + 2 * (row * kScanSlice + (((col >> 3) ^ (row & 7)) << 3) + (col & 7)));
    }

    // du_i = Kt_i dS' + sum_{i' >= i} Sc_{i'i}^T dO_{i'}
    floatx4 du[4];
    bf16x4 ndub[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const __bf16* kt = bb + R::KT / 2;
        const bf16x8 ak = concat(ld4(kt + R::rk(16 * i + l16, 32 * kk + 4 * g4)),
                                 ld4(kt + R::rk(16 * i + l16, 32 * kk + 16 + 4 * g4)));
        acc = mfma32(ak, sB[kk], acc);
      }
#pragma unroll
      for (int ip = i; ip < 4; ++ip) {
        const int off = R::SC + 2 * (tri_tile(ip, i) * 256 + (4 * g4 + (l16 >> 2)) * 16 + 4 * (l16 & 3));
        acc = mfma16(lds_read_tr(smem, boff + off), dob[ip], acc);
      }
      du[i] = acc;
      floatx4 neg;
#pragma unroll
      for (int r = 0; r < 4; ++r) neg[r] = -acc[r];
      ndub[i] = pack4(neg);
      __bf16* dup = dubuf + (size_t(bh) * nc * kChunk + c * kChunk + 16 * i + 4 * g4) * V + c0 + l16;
#pragma unroll
      for (int r = 0; r < 4; ++r) dup[size_t(r) * V] = bf(acc[r]);
    }

    // dS = diag(gamma) dS' + Qd^T dO - W^T du; Qd^T and W^T as A operands with the pair k order of the B operands
#pragma unroll
    for (int m = 0; m < KT; ++m) {
      const float4 gm = *reinterpret_cast<const float4*>(gam + 16 * m + 4 * g4);
      st[m][0] *= gm.x; st[m][1] *= gm.y; st[m][2] *= gm.z; st[m][3] *= gm.w;
      const int pos = perm_pos(16 * m + 4 * (l16 & 3));
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int tok = 32 * kk + 4 * g4 + (l16 >> 2);
        const bf16x8 aq = concat(lds_read_tr(smem, boff + R::QD + 2 * R::rk(tok, pos)),
                                 lds_read_tr(smem, boff + R::QD + 2 * R::rk(tok + 16, pos)));
        st[m] = mfma32(aq, concat(dob[2 * kk], dob[2 * kk + 1]), st[m]);
        if constexpr (kDelta) {
          const bf16x8 aw = concat(lds_read_tr(smem, boff + R::W + 2 * R::rk(tok, pos)),
                                   lds_read_tr(smem, boff + R::W + 2 * R::rk(tok + 16, pos)));
          st[m] = mfma32(aw, concat(ndub[2 * kk], ndub[2 * kk + 1]), st[m]);
        }
      }
    }
    (void)du;
    lds_barrier();
  }
  if (g.d_initial) {
#pragma unroll
    for (int m = 0; m < KT; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) g.d_initial[bh * kv + size_t(16 * m + 4 * g4 + r) * V + c0 + l16] = st[m][r];
  }
}

// ================================ state-side products: one workgroup per (chunk, head) ================================
// Products over the value dimension, wave w owning token rows 16 w .. 16 w + 15 of the chunk:
//   dqd = dO S^T,  dw = -du S^T,  dkt = u dS'^T  [64][K];   dsc = tril(dO u^T) [64][64];   bnd = rowsum(S (x) dS')
// S (entering the chunk) and dS' (leaving it) are fp32 in the workspace; 128 value columns at a time are staged
// once per workgroup into LDS as bf16 MFMA operands, and the fp32 row sums of S (x) dS' are taken on the way.
// The dO, du and u rows (A operands) come straight from global memory as 16-byte fragments.
constexpr int kSprodCols = 128;  // value columns staged per pass
template <int K>
struct SprodLds {
  static constexpr int CP = kSprodCols + 8;  // bf16 row pitch
  static constexpr int SL = 0, DS = K * CP * 2, BYTES = 2 * K * CP * 2;
};

template <int VARIANT, int K>
__global__ __launch_bounds__(256) void chunk_sprod_kernel(const gdr_args a, const gdr_grads g, int nc,
                                                          const float* __restrict__ states,
                                                          const float* __restrict__ dstates,
                                                          const __bf16* __restrict__ ubuf,
                                                          const __bf16* __restrict__ dubuf, float* __restrict__ dqd,
                                                          float* __restrict__ dw, float* __restrict__ dkt,
                                                          float* __restrict__ dsc, float* __restrict__ bnd) {
  constexpr bool kDelta = VARIANT != GDR_GLA;
  constexpr int NT = K / 16;
  using L = SprodLds<K>;
  constexpr int CP = L::CP;
  extern __shared__ __align__(16) unsigned char smem[];
  __bf16* SL = reinterpret_cast<__bf16*>(smem + L::SL);
  __bf16* DS = reinterpret_cast<__bf16*>(smem + L::DS);
  const int H = a.heads, V = a.value_dim, len = a.seq_len;
  const int BH = a.batch * H;
  const int bh = blockIdx.x % BH, c = blockIdx.x / BH;
  const int n = bh / H, h = bh % H;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, l16 = lane & 15, g4 = lane >> 4;
  const size_t kv = size_t(K) * V;
  const float* S = states + (size_t(bh) * (nc + 1) + c) * kv;
  const float* dSn = dstates + (size_t(bh) * (nc + 1) + c + 1) * kv;
  const size_t row0 = size_t(bh) * nc * kChunk + c * kChunk;  // first chunk row in ubuf / dubuf / dqd / dw / dkt
  const int t_loc = 16 * wave + l16;
  const int t_glob = c * kChunk + t_loc;
  const bool valid = t_glob < len;
  const __bf16* dor = static_cast<const __bf16*>(g.d_out.ptr) + n * g.d_out.stride_b + h * g.d_out.stride_h +
                      int64_t(min(t_glob, len - 1)) * g.d_out.stride_t;
  const __bf16* ur = ubuf + (row0 + t_loc) * V;
  const __bf16* dur = dubuf + (row0 + t_loc) * V;
  const bf16x8 zero8 = {};
  // staging assignment: thread -> row d = tid / TPR, a 128 / TPR column run
  constexpr int TPR = 256 / K, RUN = kSprodCols / TPR;
  const int sd = tid / TPR, sc0 = (tid % TPR) * RUN;
  float brow = 0.f;  // partial rowsum(S (x) dS') of row sd

  floatx4 aq[NT], aw[NT], ak[NT], as[4];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) aq[nt] = aw[nt] = ak[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) as[j] = floatx4{0.f, 0.f, 0.f, 0.f};

  for (int vc = 0; vc < V; vc += kSprodCols) {
    const int cols = min(kSprodCols, V - vc);
    // stage S and dS' columns [vc, vc + cols) as bf16; fp32 row sums of S (x) dS'
    for (int x = 0; x < RUN; x += 4) {
      const int col = sc0 + x;
      if (col < cols) {
        const float4 sv = *reinterpret_cast<const float4*>(S + size_t(sd) * V + vc + col);
        const float4 dv = *reinterpret_cast<const float4*>(dSn + size_t(sd) * V + vc + col);
        brow += sv.x * dv.x + sv.y * dv.y + sv.z * dv.z + sv.w * dv.w;
        *reinterpret_cast<bf16x4*>(SL + sd * CP + col) = bf16x4{bf(sv.x), bf(sv.y), bf(sv.z), bf(sv.w)};
        *reinterpret_cast<bf16x4*>(DS + sd * CP + col) = bf16x4{bf(dv.x), bf(dv.y), bf(dv.z), bf(dv.w)};
      }
    }
    lds_barrier();
    for (int j0 = 0; j0 < cols; j0 += 32) {
      const int jj = vc + j0 + 8 * g4;
      const bf16x8 ado = valid ? ld8(dor + jj) : zero8;
      const bf16x8 adu = ld8(dur + jj);
      const bf16x8 au = ld8(ur + jj);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const bf16x8 bs = ld8(SL + (16 * nt + l16) * CP + j0 + 8 * g4);
        aq[nt] = mfma32(ado, bs, aq[nt]);
        if constexpr (kDelta) aw[nt] = mfma32(adu, bs, aw[nt]);
        ak[nt] = mfma32(au, ld8(DS + (16 * nt + l16) * CP + j0 + 8 * g4), ak[nt]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)  // every tile of tril(dO u^T) (the upper ones are discarded): no MFMA under a branch
        as[j] = mfma32(ado, ld8(ubuf + (row0 + 16 * j + l16) * V + jj), as[j]);
    }
    lds_barrier();
  }

  auto store_rows = [&](float* dst, const floatx4* acc, float sign) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[(row0 + 16 * wave + 4 * g4 + r) * K + 16 * nt + l16] = sign * acc[nt][r];
  };
  store_rows(dqd, aq, 1.f);
  if constexpr (kDelta) store_rows(dw, aw, -1.f);
  store_rows(dkt, ak, 1.f);
  float* d = dsc + (size_t(bh) * nc + c) * kChunk * kChunk;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 16 * wave + 4 * g4 + r, s = 16 * j + l16;
      d[t * kChunk + s] = s <= t ? as[j][r] : 0.f;
    }
  if constexpr (VARIANT != GDR_DELTANET) {
#pragma unroll
    for (int m = 1; m < TPR; m <<= 1) brow += __shfl_xor(brow, m);
    if (tid % TPR == 0) bnd[(size_t(bh) * nc + c) * K + sd] = brow;
  }
}

// =============================== chunk-local gradients: one workgroup per (chunk, head) ===============================
// LDS (bytes).  Row pitches keep 16-byte alignment and stagger banks.
template <int K>
struct GradLds {
  static constexpr int BP = K + 4;    // fp32 pitch of BB
  static constexpr int KP = K + 8;    // bf16 pitch of QQ, KK, KAP
  static constexpr int MP = 68;       // fp32 pitch of the 64 x 64 matrices
  static constexpr int MAT = 64 * MP * 4;
  static constexpr int BB = 0;                    // fp32 [64][BP]  in-chunk cumsum of the log2 gate
  static constexpr int QQ = BB + 64 * BP * 4;     // bf16 [64][KP]  q (rows past the sequence end zeroed)
  static constexpr int KK = QQ + 64 * KP * 2;     // bf16 [64][KP]  k
  static constexpr int KAP = KK + 64 * KP * 2;    // bf16 [64][KP]  k e^{a_j - B} (a_j: end of the row's own block)
  static constexpr int PP = KAP + 64 * KP * 2;    // fp32 [64][MP]  P (strictly lower); later gate terms [64][K]
  static constexpr int AA = PP + MAT;             // fp32 [64][MP]  A = (I + diag(beta) P)^{-1}
  static constexpr int DL = AA + MAT;             // fp32 [64][MP]  scratch of the inverse, then dA, then dP
  static constexpr int DSC = DL + MAT;            // fp32 [64][MP]  tril(dO u^T)
  static constexpr int TOT = DSC + MAT;           // fp32 [4][K]    block totals of the log2 gate, then FAR [3][K]
  static constexpr int BETA = TOT + 4 * K * 4;    // fp32 [64]
  static constexpr int DBETA = BETA + 256;        // fp32 [64]      accumulated dbeta
  static constexpr int END = DBETA + 256;
  static constexpr bool kZAlias = MAT <= 64 * KP * 2;  // Z of dL = -A^T (dA A^T) reuses KAP when it fits
  static constexpr int ZZ = kZAlias ? KAP : END;
  static constexpr int BYTES = kZAlias ? END : END + MAT;
  static_assert(64 * K * 4 <= 2 * MAT, "gate terms alias PP + AA");
};

// log2-gate span of a 16-row block beyond which a channel's diagonal tile is summed exactly in fp32: the forward's
// hot-channel threshold.  Strong decay makes the diagonal tiles dominate the gradients, and the gate gradient sums
// terms of both signs, so those channels get fp32 terms rather than bf16 operands (the mid-block anchor alone would
// be safe from overflow up to about 220).
constexpr float kDiagSpan = kHotSpan * kLog2e;

__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

// fp32 16x16x4 MFMA: lane l holds A[l % 16][l / 16] and B[l / 16][l % 16]; D as for the bf16 shapes
__device__ __forceinline__ floatx4 mfma_f32(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void store_grad(const gdr_tensor& t, int64_t off, float v) {
  if (t.dtype == GDR_F32) static_cast<float*>(const_cast<void*>(t.ptr))[off] = v;
  else static_cast<__bf16*>(const_cast<void*>(t.ptr))[off] = bf(v);
}

template <int VARIANT, int K>
__global__ __launch_bounds__(256, 1) void chunk_grad_kernel(const gdr_args a, const gdr_grads g, int nc,
                                                            const float* __restrict__ dqd, const float* __restrict__ dwt,
                                                            const float* __restrict__ dkt, const float* __restrict__ dsc,
                                                            const float* __restrict__ bnd,
                                                            const __bf16* __restrict__ dubuf) {
  constexpr bool kDelta = VARIANT != GDR_GLA;
  constexpr int kGate = (VARIANT == GDR_KDA || VARIANT == GDR_GLA) ? 2 : (VARIANT == GDR_GDN ? 1 : 0);
  constexpr int KS = K / 32, NT = K / 16;
  using L = GradLds<K>;
  constexpr int BP = L::BP, KP = L::KP, MP = L::MP;
  extern __shared__ __align__(16) unsigned char smem[];
  float* BB = reinterpret_cast<float*>(smem + L::BB);
  __bf16* QQ = reinterpret_cast<__bf16*>(smem + L::QQ);
  __bf16* KK = reinterpret_cast<__bf16*>(smem + L::KK);
  __bf16* KAP = reinterpret_cast<__bf16*>(smem + L::KAP);
  float* PP = reinterpret_cast<float*>(smem + L::PP);
  float* AA = reinterpret_cast<float*>(smem + L::AA);
  float* DL = reinterpret_cast<float*>(smem + L::DL);
  float* DSC = reinterpret_cast<float*>(smem + L::DSC);
  float* TOT = reinterpret_cast<float*>(smem + L::TOT);
  float* FAR = TOT;
  float* BETA = reinterpret_cast<float*>(smem + L::BETA);
  float* DBETA = reinterpret_cast<float*>(smem + L::DBETA);
  float* ZZ = reinterpret_cast<float*>(smem + L::ZZ);
  float* GT = PP;

  const int H = a.heads, V = a.value_dim, len = a.seq_len, BH = a.batch * H;
  const int bh = blockIdx.x % BH, c = blockIdx.x / BH;
  const int n = bh / H, h = bh % H;
  const int tid = threadIdx.x;
  const int p = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, l16 = lane & 15, g4 = lane >> 4;
  const float scale = a.scale;
  const int t0 = c * kChunk;
  const size_t row0 = size_t(bh) * nc * kChunk + t0;  // chunk rows in dqd / dwt / dkt / dubuf
  const __bf16* qp = static_cast<const __bf16*>(a.q.ptr) + n * a.q.stride_b + h * a.q.stride_h;
  const __bf16* kp = static_cast<const __bf16*>(a.k.ptr) + n * a.k.stride_b + h * a.k.stride_h;
  const __bf16* vp = static_cast<const __bf16*>(a.v.ptr) + n * a.v.stride_b + h * a.v.stride_h;
  const float* gp = kGate ? static_cast<const float*>(a.gate.ptr) + n * a.gate.stride_b + h * a.gate.stride_h : nullptr;
  const float* betap = kDelta ? static_cast<const float*>(a.beta.ptr) + n * a.beta.stride_b + h * a.beta.stride_h
                              : nullptr;

  // ---- 1. q, k, gate rows in the A-operand layout (lane: row 16 p + l16, channels 32 kk + 8 g4 + j) ----
  const int trow = 16 * p + l16, tg = t0 + trow;
  const bool valid = tg < len;
  const int tc = min(tg, len - 1);
  const uint32_t keep = valid ? 0xffffffffu : 0u;
  float bl[KS][8];
  bf16x8 kraw8[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    const int ch = 32 * kk + 8 * g4;
    uint4 qr = *reinterpret_cast<const uint4*>(qp + int64_t(tc) * a.q.stride_t + ch);
    uint4 kr = *reinterpret_cast<const uint4*>(kp + int64_t(tc) * a.k.stride_t + ch);
    qr = make_uint4(qr.x & keep, qr.y & keep, qr.z & keep, qr.w & keep);
    kr = make_uint4(kr.x & keep, kr.y & keep, kr.z & keep, kr.w & keep);
    *reinterpret_cast<uint4*>(QQ + trow * KP + ch) = qr;
    *reinterpret_cast<uint4*>(KK + trow * KP + ch) = kr;
    kraw8[kk] = __builtin_bit_cast(bf16x8, kr);
    if constexpr (kGate == 2) {
      const float4 g0 = *reinterpret_cast<const float4*>(gp + int64_t(tc) * a.gate.stride_t + ch);
      const float4 g1 = *reinterpret_cast<const float4*>(gp + int64_t(tc) * a.gate.stride_t + ch + 4);
      bl[kk][0] = g0.x; bl[kk][1] = g0.y; bl[kk][2] = g0.z; bl[kk][3] = g0.w;
      bl[kk][4] = g1.x; bl[kk][5] = g1.y; bl[kk][6] = g1.z; bl[kk][7] = g1.w;
    } else {
      const float gs = kGate == 1 ? gp[int64_t(tc) * a.gate.stride_t] : 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) bl[kk][j] = gs;
    }
  }
  if (g4 == 0) BETA[trow] = (kDelta && valid) ? betap[int64_t(tc) * a.beta.stride_t] : 0.f;
  {  // tril(dO u^T) into LDS now (its region is free until phase 5) so the load overlaps phases 1-4
    const float4* src = reinterpret_cast<const float4*>(dsc + (size_t(bh) * nc + c) * kChunk * kChunk);
    for (int idx = tid; idx < kChunk * kChunk / 4; idx += 256)
      *reinterpret_cast<float4*>(DSC + (idx >> 4) * MP + 4 * (idx & 15)) = src[idx];
  }
  if (tid < 64) DBETA[tid] = 0.f;
  {
    const float kf = valid ? kLog2e : 0.f;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
#pragma unroll
      for (int j = 0; j < 8; ++j) bl[kk][j] = row_scan16(bl[kk][j] * kf);
    if (l16 == 15) {
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        float* dst = TOT + p * K + 32 * kk + 8 * g4;
        *reinterpret_cast<float4*>(dst) = make_float4(bl[kk][0], bl[kk][1], bl[kk][2], bl[kk][3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(bl[kk][4], bl[kk][5], bl[kk][6], bl[kk][7]);
      }
    }
  }
  lds_barrier();
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    const int ch = 32 * kk + 8 * g4;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float pre = 0.f;
      for (int pb = 0; pb < p; ++pb) pre += TOT[pb * K + ch + j];
      bl[kk][j] += pre;
    }
    *reinterpret_cast<float4*>(BB + trow * BP + ch) = make_float4(bl[kk][0], bl[kk][1], bl[kk][2], bl[kk][3]);
    *reinterpret_cast<float4*>(BB + trow * BP + ch + 4) = make_float4(bl[kk][4], bl[kk][5], bl[kk][6], bl[kk][7]);
  }
  lds_barrier();

  // ---- 2. factors: FAR[(2,0), (3,0), (3,1)] = e^{a_{i-1} - a_j}; KAP = k e^{a_p - B}; Lk = k e^{B - a_{p-1}} ----
  auto anchor = [&](int blk, int ch) -> float { return blk < 0 ? 0.f : BB[(16 * blk + 15) * BP + ch]; };
  for (int idx = tid; idx < 3 * K; idx += 256) {
    const int v = idx / K, ch = idx % K;
    const float a0 = anchor(0, ch), a1 = anchor(1, ch), a2 = anchor(2, ch);
    FAR[v * K + ch] = ex2(v == 0 ? a1 - a0 : (v == 1 ? a2 - a0 : a2 - a1));
  }
  auto build_kap = [&]() {
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int ch = 32 * kk + 8 * g4;
      const bf16x8 kr = *reinterpret_cast<const bf16x8*>(KK + trow * KP + ch);
      bf16x8 o;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = bf(f32(kr[j]) * ex2(anchor(p, ch + j) - BB[trow * BP + ch + j]));
      *reinterpret_cast<bf16x8*>(KAP + trow * KP + ch) = o;
    }
  };
  build_kap();
  bf16x8 lk[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    const int ch = 32 * kk + 8 * g4;
#pragma unroll
    for (int j = 0; j < 8; ++j) lk[kk][j] = bf(f32(kraw8[kk][j]) * ex2(bl[kk][j] - anchor(p - 1, ch + j)));
  }
  auto far_of = [&](int i, int j) -> const float* {  // e^{a_{i-1} - a_j} for j < i - 1, else nullptr (factor 1)
    return j < i - 1 ? FAR + ((i == 2) ? 0 : (j == 0 ? 1 : 2)) * K : nullptr;
  };
  lds_barrier();

  if constexpr (kDelta) {
    // ---- 3. P: off-diagonal tiles (p, j < p) on MFMA; the diagonal tile exactly in fp32 ----
#pragma unroll
    for (int j = 0; j < 3; ++j) {  // tiles j >= p are computed and dropped: no MFMA under a branch
      const float* far = far_of(p, j);
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const int ch = 32 * kk + 8 * g4;
        bf16x8 bk = *reinterpret_cast<const bf16x8*>(KAP + (16 * j + l16) * KP + ch);
        if (far) {
#pragma unroll
          for (int e = 0; e < 8; ++e) bk[e] = bf(f32(bk[e]) * far[ch + e]);
        }
        acc = mfma32(lk[kk], bk, acc);
      }
      if (j < p) {
#pragma unroll
        for (int r = 0; r < 4; ++r) PP[(16 * p + 4 * g4 + r) * MP + 16 * j + l16] = acc[r];
      }
    }
    {  // diagonal tile: (k e^{B - m}) (k e^{m - B})^T with m the middle of the block's gate range, so every factor
       // is within 2^{+-span/2}; channels whose span exceeds kDiagSpan take a zero operand and an exact fp32 sum
      bf16x8 ae[KS], af[KS];
      bool any_hot = false;
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const int ch = 32 * kk + 8 * g4;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float top = BB[(16 * p) * BP + ch + j], bot = BB[(16 * p + 15) * BP + ch + j];
          const bool hot = top - bot > kDiagSpan;
          any_hot |= hot;
          const float mid = 0.5f * (top + bot), kv = f32(kraw8[kk][j]);
          ae[kk][j] = bf(hot ? 0.f : kv * ex2(bl[kk][j] - mid));
          af[kk][j] = bf(hot ? 0.f : kv * ex2(mid - bl[kk][j]));
        }
      }
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) acc = mfma32(ae[kk], af[kk], acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 4 * g4 + r;
        if (l16 < t) PP[(16 * p + t) * MP + 16 * p + l16] = acc[r];
      }
      if (__any(any_hot)) {
        for (int q = lane; q < 120; q += 64) {  // pair (t, s), s < t: add the hot channels' exact terms
          int t = 1;
          while (t * (t + 1) / 2 <= q) ++t;
          const int s2 = q - t * (t - 1) / 2;
          const int rt = 16 * p + t, rs = 16 * p + s2;
          float add = 0.f;
          for (int d = 0; d < K; ++d) {
            if (!(BB[(16 * p) * BP + d] - BB[(16 * p + 15) * BP + d] > kDiagSpan)) continue;
            add += f32(KK[rt * KP + d]) * f32(KK[rs * KP + d]) * ex2(BB[rt * BP + d] - BB[rs * BP + d]);
          }
          PP[rt * MP + rs] += add;
        }
      }
    }
    for (int idx = lane; idx < 16 * 64; idx += 64) {  // diagonal and everything right of it in this row block
      const int x = idx >> 6, col = idx & 63;
      if (col >= 16 * p + x) PP[(16 * p + x) * MP + col] = 0.f;
    }
    lds_barrier();

    // ---- 4. A = (I + diag(beta) P)^{-1}: diagonal blocks by forward substitution, then block rows 1..3 ----
    if (lane < 16) {
      float x[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float acc = r == lane ? 1.f : 0.f;
        const float br = BETA[16 * p + r];
#pragma unroll
        for (int m = 0; m < r; ++m) acc -= br * PP[(16 * p + r) * MP + 16 * p + m] * x[m];
        x[r] = acc;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) AA[(16 * p + r) * MP + 16 * p + lane] = x[r];
    }
    for (int idx = lane; idx < 16 * 64; idx += 64) {
      const int x = idx >> 6, col = idx & 63;
      if (col >= 16 * (p + 1) || col < 16 * p) AA[(16 * p + x) * MP + col] = 0.f;
    }
    lds_barrier();
    // Block rows 1..3 in turn on fp32 MFMA; wave p owns tile column p:  Y = diag(beta) P[block i, :16i] A[:16i, p],
    // A_ip = -A_ii Y (zero for p >= i, since A is lower triangular).  Y passes through wave-private scratch in DL.
#pragma unroll
    for (int i = 1; i < 4; ++i) {
      const int ta = 16 * i + l16;
      const float bt = BETA[ta];
      floatx4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q0 = 0; q0 < 16 * i; q0 += 4)
        y = mfma_f32(bt * PP[ta * MP + q0 + g4], AA[(q0 + g4) * MP + 16 * p + l16], y);
#pragma unroll
      for (int r = 0; r < 4; ++r) DL[(16 * p + 4 * g4 + r) * MP + l16] = y[r];
      floatx4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q0 = 0; q0 < 16; q0 += 4)
        z = mfma_f32(AA[ta * MP + 16 * i + q0 + g4], DL[(16 * p + q0 + g4) * MP + l16], z);
      if (p < i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) AA[(16 * i + 4 * g4 + r) * MP + 16 * p + l16] = -z[r];
      }
      lds_barrier();
    }
  }

  // ---- 5. dA = dW (beta K e^B)^T + du (beta V)^T, tiles (p, j <= p) ----
  if constexpr (kDelta) {
    // beta k e^B of this lane's row into the KAP region (free here; KAP is rebuilt after phase 6)
    {
      const float bt = BETA[trow];
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        bf16x8 o;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = bf(f32(kraw8[kk][j]) * bt * ex2(bl[kk][j]));
        *reinterpret_cast<bf16x8*>(KAP + trow * KP + 32 * kk + 8 * g4) = o;
      }
    }
    lds_barrier();
    floatx4 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int ch = 32 * kk + 8 * g4;
      const float* wr = dwt + (row0 + trow) * K + ch;
      const float4 w0 = *reinterpret_cast<const float4*>(wr), w1 = *reinterpret_cast<const float4*>(wr + 4);
      const bf16x8 aw = {bf(w0.x), bf(w0.y), bf(w0.z), bf(w0.w), bf(w1.x), bf(w1.y), bf(w1.z), bf(w1.w)};
#pragma unroll
      for (int j = 0; j < 4; ++j)  // all four tiles (those right of the diagonal are dropped)
        acc[j] = mfma32(aw, *reinterpret_cast<const bf16x8*>(KAP + (16 * j + l16) * KP + ch), acc[j]);
    }
    // The value-dimension part accumulates separately and is added after the loop: an MFMA accumulator carried
    // from straight-line code into a loop of runtime trip count came out wrong for K = 64.
    floatx4 acv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acv[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int j0 = 0; j0 < V; j0 += 32) {
      const bf16x8 au = ld8(dubuf + (row0 + trow) * V + j0 + 8 * g4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int rs = 16 * j + l16;
        const bf16x8 vr = ld8(vp + int64_t(min(t0 + rs, len - 1)) * a.v.stride_t + j0 + 8 * g4);
        const float bs = BETA[rs];
        bf16x8 bv;
#pragma unroll
        for (int e = 0; e < 8; ++e) bv[e] = bf(f32(vr[e]) * bs);
        acv[j] = mfma32(au, bv, acv[j]);
      }
    }
    lds_barrier();  // the inverse's scratch in DL is dead
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) DL[(16 * p + 4 * g4 + r) * MP + 16 * j + l16] = j <= p ? acc[j][r] + acv[j][r] : 0.f;
  }
  lds_barrier();

  // ---- 6. dL = -A^T (dA A^T) on the strict lower triangle; dP = diag(beta) dL; dbeta += rowsum(dL (x) P) ----
  if constexpr (kDelta) {
    // fp32 MFMA (the reference evaluates this product in fp32 too, kimi_delta_attention.py:385).  Z = dA A^T for row block p, tile columns
    // si (k over q < 16 (si + 1): A[s][q] = 0 beyond); only Z's strictly lower part reaches dL.
#pragma unroll
    for (int si = 0; si < 4; ++si) {
      floatx4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q0 = 0; q0 < 16 * (si + 1); q0 += 4)
        z = mfma_f32(DL[(16 * p + l16) * MP + q0 + g4], AA[(16 * si + l16) * MP + q0 + g4], z);
#pragma unroll
      for (int r = 0; r < 4; ++r) ZZ[(16 * p + 4 * g4 + r) * MP + 16 * si + l16] = z[r];
    }
    lds_barrier();
    // dL = -A^T Z for row block p (k over all r: A[r][t] = 0 for r < t), kept strictly lower; dP = diag(beta) dL
    float dbr[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int si = 0; si < 4; ++si) {
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r0 = 0; r0 < kChunk; r0 += 4)
        acc = mfma_f32(AA[(r0 + g4) * MP + 16 * p + l16], ZZ[(r0 + g4) * MP + 16 * si + l16], acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * p + 4 * g4 + r, s = 16 * si + l16;
        const float dl = t > s ? -acc[r] : 0.f;
        dbr[r] += dl * PP[t * MP + s];
        DL[t * MP + s] = BETA[t] * dl;
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = dbr[r];
      v += __shfl_xor(v, 1, 16);
      v += __shfl_xor(v, 2, 16);
      v += __shfl_xor(v, 4, 16);
      v += __shfl_xor(v, 8, 16);
      if (l16 == 0) atomicAdd(DBETA + 16 * p + 4 * g4 + r, v);
    }
    lds_barrier();
  }

  // ---- 7. X1 = A^T dW, X2 = A^T du (rows s of block p): dk += beta e^B X1, dv = beta X2, dbeta ----
  floatx4 dkpos[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) dkpos[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int srow = 16 * p + 4 * g4;  // this lane's accumulator rows srow + r
  auto tr_off = [&](int base, int row, int col) { return base + 2 * (row * KP + col); };
  if constexpr (kDelta) {
    bf16x4 at[4];  // (A^T)[16 p + l16][16 kb + 4 g4 + r]; zero for kb < p (A is lower triangular)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      floatx4 v;
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = AA[(16 * kb + 4 * g4 + r) * MP + 16 * p + l16];
      at[kb] = pack4(v);
    }
    lds_barrier();  // A lives in registers now; P is dead: AA and PP take staged operands
    // dW as bf16 [64][KP] in PP, read by the transposing LDS read as the B operand of X1 = A^T dW
    __bf16* WS = reinterpret_cast<__bf16*>(smem + L::PP);
    __bf16* US = reinterpret_cast<__bf16*>(smem + L::KAP);  // du columns of one pass (KAP is rebuilt afterwards)
    __bf16* VS = reinterpret_cast<__bf16*>(smem + L::AA);   // v columns of one pass
    for (int idx = tid; idx < kChunk * K / 4; idx += 256) {
      const int row = idx / (K / 4), col = 4 * (idx % (K / 4));
      const float4 w = *reinterpret_cast<const float4*>(dwt + (row0 + row) * K + col);
      *reinterpret_cast<bf16x4*>(WS + row * KP + col) = bf16x4{bf(w.x), bf(w.y), bf(w.z), bf(w.w)};
    }
    lds_barrier();
    float dbp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int d = 16 * nt + l16;
      floatx4 x1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
        x1 = mfma16(at[kb], lds_read_tr(smem, tr_off(L::PP, 16 * kb + 4 * g4 + (l16 >> 2), 16 * nt + 4 * (l16 & 3))),
                    x1);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rs = srow + r;
        const float eb = ex2(BB[rs * BP + d]);
        dkpos[nt][r] = BETA[rs] * eb * x1[r];
        dbp[r] += x1[r] * f32(KK[rs * KP + d]) * eb;
      }
    }
    // X2 = A^T du in passes of K value columns: du and v staged as bf16 (16-byte global loads)
    for (int vc = 0; vc < V; vc += K) {
      const int cols = min(K, V - vc);
      for (int idx = tid; idx < kChunk * cols / 8; idx += 256) {
        const int row = idx / (cols / 8), col = 8 * (idx % (cols / 8));
        *reinterpret_cast<bf16x8*>(US + row * KP + col) = ld8(dubuf + (row0 + row) * V + vc + col);
        *reinterpret_cast<bf16x8*>(VS + row * KP + col) =
            ld8(vp + int64_t(min(t0 + row, len - 1)) * a.v.stride_t + vc + col);
      }
      lds_barrier();
      for (int j0 = 0; j0 < cols; j0 += 16) {
        const int jc = vc + j0 + l16;
        floatx4 x2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
          x2 = mfma16(at[kb], lds_read_tr(smem, tr_off(L::KAP, 16 * kb + 4 * g4 + (l16 >> 2), j0 + 4 * (l16 & 3))),
                      x2);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int rs = srow + r;
          if (t0 + rs < len) {
            const int64_t tt = t0 + rs;
            store_grad(g.d_value, n * g.d_value.stride_b + h * g.d_value.stride_h + tt * g.d_value.stride_t + jc,
                       BETA[rs] * x2[r]);
            dbp[r] += x2[r] * f32(VS[rs * KP + j0 + l16]);
          }
        }
      }
      lds_barrier();
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = dbp[r];
      v += __shfl_xor(v, 1, 16);
      v += __shfl_xor(v, 2, 16);
      v += __shfl_xor(v, 4, 16);
      v += __shfl_xor(v, 8, 16);
      if (l16 == 0) atomicAdd(DBETA + srow + r, v);
    }
    build_kap();  // phases 5-7 reused the KAP region
    lds_barrier();
  } else {
    for (int idx = tid; idx < kChunk * V; idx += 256) {  // GLA: U = V, so dv = du
      const int rr = idx / V, jc = idx % V;
      if (t0 + rr < len)
        store_grad(g.d_value,
                   n * g.d_value.stride_b + h * g.d_value.stride_h + int64_t(t0 + rr) * g.d_value.stride_t + jc,
                   f32(dubuf[(row0 + rr) * V + jc]));
    }
  }

  // ---- 8. the four gated products off the diagonal (block-anchored factors, every one <= 1) ----
  //   left  (rows t of block p, tiles j < p):  e^{B_t - a_{p-1}} sum_j D_pj (k_j e^{a_j - B}) e^{a_{p-1} - a_j}
  //   key   (rows s of block p, tiles i > p):  e^{a_p - B_s} sum_i D_ip^T (x_i e^{B - a_{i-1}}) e^{a_{i-1} - a_p}
  // with D = tril(dO u^T) (dq, and dk with x = q) and D = dP (dk twice, x = k).
  float pre_qd[NT][4], pre_kt[NT][4];  // assembly operands, loaded here so their latency hides behind phases 8-9
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pre_qd[nt][r] = dqd[(row0 + srow + r) * K + 16 * nt + l16];
      pre_kt[nt][r] = dkt[(row0 + srow + r) * K + 16 * nt + l16];
    }
  floatx4 aq[NT], al[NT], ks[NT], kq[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) aq[nt] = al[nt] = ks[nt] = kq[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
  // Both loops run over every tile with zero operands outside the range: no MFMA sits under a branch.
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const float* far = far_of(p, j);
    const float keepj = j < p ? 1.f : 0.f;
    const float4 s4 = *reinterpret_cast<const float4*>(DSC + (16 * p + l16) * MP + 16 * j + 4 * g4);
    const float4 p4 = *reinterpret_cast<const float4*>(DL + (16 * p + l16) * MP + 16 * j + 4 * g4);
    const bf16x4 a1 = {bf(keepj * s4.x), bf(keepj * s4.y), bf(keepj * s4.z), bf(keepj * s4.w)};
    const bf16x4 a2 = {bf(keepj * p4.x), bf(keepj * p4.y), bf(keepj * p4.z), bf(keepj * p4.w)};
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      bf16x4 b = lds_read_tr(smem, tr_off(L::KAP, 16 * j + 4 * g4 + (l16 >> 2), 16 * nt + 4 * (l16 & 3)));
      if (far) {
        const float f = far[16 * nt + l16];
#pragma unroll
        for (int r = 0; r < 4; ++r) b[r] = bf(f32(b[r]) * f);
      }
      aq[nt] = mfma16(a1, b, aq[nt]);
      if constexpr (kDelta) al[nt] = mfma16(a2, b, al[nt]);
    }
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int d = 16 * nt + l16;
    const float ap = anchor(p - 1, d);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float lt = ex2(BB[(srow + r) * BP + d] - ap);
      aq[nt][r] *= lt;
      al[nt][r] *= lt;
    }
  }
#pragma unroll
  for (int i = 1; i < 4; ++i) {
    const float* far = far_of(i, p);
    const float keepi = i > p ? 1.f : 0.f;
    floatx4 s4, p4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s4[r] = keepi * DSC[(16 * i + 4 * g4 + r) * MP + 16 * p + l16];
      p4[r] = keepi * DL[(16 * i + 4 * g4 + r) * MP + 16 * p + l16];
    }
    const bf16x4 a1 = pack4(s4), a2 = pack4(p4);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int d = 16 * nt + l16;
      const int row = 16 * i + 4 * g4 + (l16 >> 2), col = 16 * nt + 4 * (l16 & 3);
      const bf16x4 qr = lds_read_tr(smem, tr_off(L::QQ, row, col));
      const bf16x4 kr = lds_read_tr(smem, tr_off(L::KK, row, col));
      const float ai = anchor(i - 1, d), f = far ? far[d] : 1.f;
      bf16x4 bq, bk;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float fac = ex2(BB[(16 * i + 4 * g4 + r) * BP + d] - ai) * f;
        bq[r] = bf(f32(qr[r]) * fac);
        bk[r] = bf(f32(kr[r]) * fac);
      }
      ks[nt] = mfma16(a1, bq, ks[nt]);
      if constexpr (kDelta) kq[nt] = mfma16(a2, bk, kq[nt]);
    }
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int d = 16 * nt + l16;
    const float ap = anchor(p, d);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float rs = ex2(ap - BB[(srow + r) * BP + d]);
      ks[nt][r] *= rs;
      kq[nt][r] *= rs;
    }
  }

  // ---- 9. diagonal tiles: anchored at the middle of the block's gate range (factors within 2^{+-span/2}); a
  // channel whose span exceeds kDiagSpan gets a zero operand there and its exact elementwise sum instead ----
  {
    bf16x4 a1, a2, a1t, a2t;
    {
      const float4 s4 = *reinterpret_cast<const float4*>(DSC + (16 * p + l16) * MP + 16 * p + 4 * g4);
      const float4 p4 = *reinterpret_cast<const float4*>(DL + (16 * p + l16) * MP + 16 * p + 4 * g4);
      a1 = bf16x4{bf(s4.x), bf(s4.y), bf(s4.z), bf(s4.w)};
      a2 = bf16x4{bf(p4.x), bf(p4.y), bf(p4.z), bf(p4.w)};
      floatx4 s4t, p4t;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s4t[r] = DSC[(16 * p + 4 * g4 + r) * MP + 16 * p + l16];
        p4t[r] = DL[(16 * p + 4 * g4 + r) * MP + 16 * p + l16];
      }
      a1t = pack4(s4t);
      a2t = pack4(p4t);
    }
    bool any_hot = false;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int d = 16 * nt + l16;
      const float top = BB[(16 * p) * BP + d], bot = BB[(16 * p + 15) * BP + d];
      const bool hot = top - bot > kDiagSpan;
      any_hot |= hot;
      const float mid = 0.5f * (top + bot);
      const int row = 16 * p + 4 * g4 + (l16 >> 2), col = 16 * nt + 4 * (l16 & 3);
      const bf16x4 qr = lds_read_tr(smem, tr_off(L::QQ, row, col));
      const bf16x4 kr = lds_read_tr(smem, tr_off(L::KK, row, col));
      bf16x4 bkf, bqe, bke;  // k f, q e, k e at rows srow + r (this lane's k slots)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float bx = BB[(srow + r) * BP + d];
        const float e = hot ? 0.f : ex2(bx - mid), f = hot ? 0.f : ex2(mid - bx);
        bkf[r] = bf(f32(kr[r]) * f);
        bqe[r] = bf(f32(qr[r]) * e);
        bke[r] = bf(f32(kr[r]) * e);
      }
      const floatx4 z = {0.f, 0.f, 0.f, 0.f};
      const floatx4 lq = mfma16(a1, bkf, z), ls = mfma16(a1t, bqe, z);
      floatx4 ll = z, lk2 = z;
      if constexpr (kDelta) {
        ll = mfma16(a2, bkf, z);
        lk2 = mfma16(a2t, bke, z);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float bx = BB[(srow + r) * BP + d];
        const float e = hot ? 0.f : ex2(bx - mid), f = hot ? 0.f : ex2(mid - bx);
        aq[nt][r] += e * lq[r];
        al[nt][r] += e * ll[r];
        ks[nt][r] += f * ls[r];
        kq[nt][r] += f * lk2[r];
      }
    }
    if (__any(any_hot)) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int d = 16 * nt + l16;
        const float top = BB[(16 * p) * BP + d], bot = BB[(16 * p + 15) * BP + d];
        if (!(top - bot > kDiagSpan)) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 4 * g4 + r, rt = 16 * p + t;
          const float bt = BB[rt * BP + d];
          float sq = 0.f, sl = 0.f, sk = 0.f, sp = 0.f;
#pragma unroll 1
          for (int x = 0; x < 16; ++x) {
            const int rx = 16 * p + x;
            const float bx = BB[rx * BP + d];
            if (x <= t) {  // left: (t, s = x)
              const float e = ex2(bt - bx) * f32(KK[rx * KP + d]);
              sq += DSC[rt * MP + rx] * e;
              if constexpr (kDelta) sl += DL[rt * MP + rx] * e;
            }
            if (x >= t) {  // key: (t' = x, s = t)
              const float e = ex2(bx - bt);
              sk += DSC[rx * MP + rt] * f32(QQ[rx * KP + d]) * e;
              if constexpr (kDelta) sp += DL[rx * MP + rt] * f32(KK[rx * KP + d]) * e;
            }
          }
          aq[nt][r] += sq;
          al[nt][r] += sl;
          ks[nt][r] += sk;
          kq[nt][r] += sp;
        }
      }
    }
  }
  lds_barrier();  // every wave is past its last read of PP / AA: the gate terms reuse them

  // ---- 10. assembly: dq, dk; gate terms q dq + k dk_{e^{+B}} - k dk_{e^{-B}} without the Kt role (GT) and the Kt
  // role's k dKt e^{B_end - B} (KTT) ----
  const float* bend = BB + 63 * BP;
  float* KTT = DL;  // DL + DSC, free after phase 9
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int d = 16 * nt + l16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int rs = srow + r;
      const float bx = BB[rs * BP + d];
      const float dq = scale * (pre_qd[nt][r] * ex2(bx) + aq[nt][r]);
      const float dkp = dkpos[nt][r] + al[nt][r];
      const float dkn = scale * ks[nt][r] + kq[nt][r];
      const float dkt_role = pre_kt[nt][r] * ex2(bend[d] - bx);
      const float qv = f32(QQ[rs * KP + d]), kv = f32(KK[rs * KP + d]);
      GT[rs * K + d] = qv * dq + kv * (dkp - dkn);
      KTT[rs * K + d] = kv * dkt_role;
      if (t0 + rs < len) {
        const int64_t tt = t0 + rs;
        store_grad(g.d_query, n * g.d_query.stride_b + h * g.d_query.stride_h + tt * g.d_query.stride_t + d, dq);
        store_grad(g.d_key, n * g.d_key.stride_b + h * g.d_key.stride_h + tt * g.d_key.stride_t + d,
                   dkp + dkn + dkt_role);
      }
    }
  }
  lds_barrier();

  // ---- 11. gate gradient: reverse cumsum of GT + e^{B_end} rowsum(S (x) dS') + exclusive forward cumsum of KTT ----
  float* dgp = kGate ? static_cast<float*>(const_cast<void*>(g.d_gate.ptr)) + n * g.d_gate.stride_b +
                           h * g.d_gate.stride_h
                     : nullptr;
  const float* bndc = bnd + (size_t(bh) * nc + c) * K;
  if constexpr (kGate == 2) {
    // thread (channel d, half h) scans rows [32 h, 32 h + 32); the halves meet through TOT (free)
    const int d = tid % K, hh = tid / K;  // K = 128: halves 0, 1; K = 64: quarters 0..3 of 16 rows
    constexpr int NPART = 256 / K, RP = kChunk / NPART;
    float gtv[RP], ktv[RP];
#pragma unroll
    for (int x = 0; x < RP; ++x) {
      gtv[x] = GT[(RP * hh + x) * K + d];
      ktv[x] = KTT[(RP * hh + x) * K + d];
    }
    float gsum = 0.f, ksum = 0.f;
#pragma unroll
    for (int x = 0; x < RP; ++x) gsum += gtv[x], ksum += ktv[x];
    TOT[hh * K + d] = gsum;  // TOT holds 4 K floats: part sums of GT, then of KTT in the second half
    lds_barrier();
    float gafter = bndc[d] * ex2(bend[d]), kbefore = 0.f;  // GT after this part, KTT before it
    for (int o = hh + 1; o < NPART; ++o) gafter += TOT[o * K + d];
    lds_barrier();
    TOT[hh * K + d] = ksum;
    lds_barrier();
    for (int o = 0; o < hh; ++o) kbefore += TOT[o * K + d];
    float suf = gafter, pre = kbefore;
    float kex[RP];
#pragma unroll
    for (int x = 0; x < RP; ++x) {
      kex[x] = pre;
      pre += ktv[x];
    }
#pragma unroll
    for (int x = RP - 1; x >= 0; --x) {
      suf += gtv[x];
      const int t = RP * hh + x;
      if (t0 + t < len) dgp[int64_t(t0 + t) * g.d_gate.stride_t + d] = suf + kex[x];
    }
  } else if constexpr (kGate == 1) {
    // per-row sums over the channels into TOT (free): [0, 64) of GT, [64, 128) of KTT; wave w sums rows
    // 16 w .. 16 w + 15 with lanes over channels
    for (int x = 0; x < 16; ++x) {
      const int t = 16 * p + x;
      float a = 0.f, b = 0.f;
      for (int d = lane; d < K; d += 64) a += GT[t * K + d], b += KTT[t * K + d];
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) a += __shfl_xor(a, m), b += __shfl_xor(b, m);
      if (lane == 0) {
        TOT[t] = a;
        TOT[kChunk + t] = b;
      }
    }
    lds_barrier();
    if (tid == 0) {
      float total = 0.f, pre = 0.f;
      for (int d = 0; d < K; ++d) total += bndc[d] * ex2(bend[d]);
      for (int t = 0; t < kChunk; ++t) {  // exclusive prefix of the Kt-role row sums
        const float x = TOT[kChunk + t];
        TOT[kChunk + t] = pre;
        pre += x;
      }
      for (int t = kChunk - 1; t >= 0; --t) {
        total += TOT[t];
        if (t0 + t < len) dgp[int64_t(t0 + t) * g.d_gate.stride_t] = total + TOT[kChunk + t];
      }
    }
  }
  if constexpr (kDelta) {
    if (tid < kChunk && t0 + tid < len) {
      float* dbp = static_cast<float*>(const_cast<void*>(g.d_beta.ptr)) + n * g.d_beta.stride_b + h * g.d_beta.stride_h;
      dbp[int64_t(t0 + tid) * g.d_beta.stride_t] = DBETA[tid];
    }
  }
}

// =============================================== launchers ===============================================
int64_t round256(int64_t x) { return (x + 255) / 256 * 256; }

template <int VARIANT, int K>
hipError_t launch_bwd_typed(const gdr_args& a, const gdr_grads& g, const BwdLayout& Lw, unsigned char* ws,
                            hipStream_t stream) {
  const int nc = (a.seq_len + kChunk - 1) / kChunk;
  const int bh = a.batch * a.heads;
  const int64_t rec = Rec<K>::bytes(a.value_dim);
  constexpr int dscan_lds = 2 * (Rec<K>::FIX + kChunk * kScanSlice * 2);
  constexpr int grad_lds = GradLds<K>::BYTES;
  hipError_t e = configure_lds<&chunk_dscan_kernel<VARIANT, K>>(dscan_lds);
  if (e == hipSuccess) e = configure_lds<&chunk_grad_kernel<VARIANT, K>>(grad_lds);
  if (e == hipSuccess) e = configure_lds<&chunk_sprod_kernel<VARIANT, K>>(SprodLds<K>::BYTES);
  if (e != hipSuccess) return e;
  if (nc == 0) return hipSuccess;
  float* states = reinterpret_cast<float*>(ws + Lw.states);
  float* dstates = reinterpret_cast<float*>(ws + Lw.dstates);
  __bf16* ubuf = reinterpret_cast<__bf16*>(ws + Lw.ubuf);
  __bf16* dubuf = reinterpret_cast<__bf16*>(ws + Lw.dubuf);
  float* dqd = reinterpret_cast<float*>(ws + Lw.dqd);
  float* dw = reinterpret_cast<float*>(ws + Lw.dw);
  float* dkt = reinterpret_cast<float*>(ws + Lw.dkt);
  float* dsc = reinterpret_cast<float*>(ws + Lw.dsc);
  float* bnd = reinterpret_cast<float*>(ws + Lw.bnd);
  const int n_slices = a.value_dim / kScanSlice;
  const int xcd_map = (bh % 8 == 0) ? 1 : 0;
  hipLaunchKernelGGL((chunk_dscan_kernel<VARIANT, K>), dim3(bh * n_slices), dim3(kDScanThreads), dscan_lds, stream,
                     a, g, n_slices, xcd_map, nc, rec, ws + Lw.rec, dstates, dubuf);
  hipLaunchKernelGGL((chunk_sprod_kernel<VARIANT, K>), dim3(bh * nc), dim3(256), SprodLds<K>::BYTES, stream, a, g,
                     nc, states, dstates, ubuf, dubuf, dqd, dw, dkt, dsc, bnd);
  hipLaunchKernelGGL((chunk_grad_kernel<VARIANT, K>), dim3(bh * nc), dim3(256), grad_lds, stream, a, g, nc, dqd, dw,
                     dkt, dsc, bnd, dubuf);
  return hipGetLastError();
}

template <int VARIANT>
hipError_t launch_bwd_v(const gdr_args& a, const gdr_grads& g, const BwdLayout& L, unsigned char* ws,
                        hipStream_t stream) {
  return a.key_dim == 64 ? launch_bwd_typed<VARIANT, 64>(a, g, L, ws, stream)
                         : launch_bwd_typed<VARIANT, 128>(a, g, L, ws, stream);
}

}  // namespace

BwdLayout chunk_bwd_layout(const gdr_args& a) {
  BwdLayout L{};
  const int64_t nc = (a.seq_len + kChunk - 1) / kChunk;
  const int64_t bh = int64_t(a.batch) * a.heads, K = a.key_dim, V = a.value_dim;
  int64_t off = 0;
  auto take = [&](int64_t bytes) { const int64_t o = off; off += round256(bytes); return o; };
  L.rec = take(chunk_workspace_bytes(a));
  L.states = take(bh * (nc + 1) * K * V * 4);
  L.dstates = take(bh * (nc + 1) * K * V * 4);
  L.ubuf = take(bh * nc * kChunk * V * 2);
  L.dubuf = take(bh * nc * kChunk * V * 2);
  L.dqd = take(bh * nc * kChunk * K * 4);
  L.dw = take(bh * nc * kChunk * K * 4);
  L.dkt = take(bh * nc * kChunk * K * 4);
  L.dsc = take(bh * nc * kChunk * kChunk * 4);
  L.bnd = take(bh * nc * K * 4);
  L.total = off;
  return L;
}

hipError_t launch_chunk_bwd(const gdr_args& a, const gdr_grads& g, const BwdLayout& L, unsigned char* ws,
                            hipStream_t stream) {
  switch (a.variant) {
    case GDR_KDA: return launch_bwd_v<GDR_KDA>(a, g, L, ws, stream);
    case GDR_GDN: return launch_bwd_v<GDR_GDN>(a, g, L, ws, stream);
    case GDR_GLA: return launch_bwd_v<GDR_GLA>(a, g, L, ws, stream);
    default: return launch_bwd_v<GDR_DELTANET>(a, g, L, ws, stream);
  }
}

}  // namespace gdr
