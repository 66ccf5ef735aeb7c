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
//   chunk_dscan_kernel   reverse scan over chunks with dS in registers; writes dS' (bf16) per chunk and du^T
//   chunk_dlocal_kernel  per (chunk, head): everything chunk-local, including the products with S and dS'
#include <type_traits>

#include "chunk_common.h"
#include "gdr_internal.h"
#include "split_common.h"

namespace gdr {

using namespace chunk;

namespace {

// Threads of a reverse-scan workgroup of SL value columns: SL / 16 compute waves of 16 columns + 4 DMA loader waves.
template <int SL>
constexpr int dscan_threads() { return 64 * (SL / 16 + 4); }

// Position of the 4-channel block [c, c + 4) (c % 4 == 0) in a row of the permuted W / Q e^B record layout:
// within a 32-channel group, channel 4 g + j sits at 8 g + j and channel 16 + 4 g + j at 8 g + 4 + j.
__device__ __forceinline__ int perm_pos(int c) { return (c & ~31) + 8 * ((c & 15) >> 2) + 4 * ((c >> 4) & 1); }

__device__ __forceinline__ bf16x8 ld8(const __bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ bf16x4 ld4(const __bf16* p) { return *reinterpret_cast<const bf16x4*>(p); }

// ============================ reverse state scan: one workgroup per (sequence, head) x SL columns ============================
// Per chunk c (last to first), each compute wave holds dS' = dS_{c+1} for 16 value columns in registers:
//   du = Sc^T dO + Kt dS'  (row blocks i: Kt rows on 16x16x32 MFMAs with dS' as the two-tile B operand, Sc^T tiles
//   and dO blocks through the transposing LDS read on 16x16x16 MFMAs), then
//   dS = diag(gamma) dS' + Qd^T dO - W^T du  (Qd^T, W^T read transposed from the permuted record rows).
// The loader waves stream the next record (W, Q e^B, Kt, Sc, gamma) and the dO slice into the other LDS buffer.
// SL (64, 32 or 16 columns) is chosen per launch as for the forward scan: every compute wave reads the whole record
// from LDS each step, so narrower slices mean fewer waves per CU sharing its LDS bandwidth and more CUs at work.
template <int VARIANT, int K, int SL>
__global__ __launch_bounds__(dscan_threads<SL>(), 1) void chunk_dscan_kernel(const gdr_args a, const gdr_grads g,
                                                                             int n_slices, int xcd_map, int nc,
                                                                             int64_t rec_bytes,
                                                                             const unsigned char* __restrict__ rec_ws,
                                                                             __bf16* __restrict__ dstates,
                                                                             __bf16* __restrict__ dubt) {
  constexpr bool kDelta = VARIANT != GDR_GLA;
  constexpr int KT = K / 16, KS = K / 32;
  using R = Rec<K>;
  constexpr int kComp = SL / 16;                // compute waves
  constexpr int CPR = SL / 8;                   // 16-byte chunks per dO row
  constexpr int DO = R::FIX;                    // dO slice: bf16 [64][SL], chunk q of row r at slot q ^ (r % CPR)
  constexpr int SB = R::FIX + kChunk * SL * 2;  // LDS bytes per buffer
  constexpr int NF = R::FIX / 16, NDO = kChunk * SL * 2 / 16;
  constexpr int G0 = kDelta ? 0 : R::QD / 1024;        // GLA reads no W: its copies start at Q e^B
  constexpr int NG = ((NF + NDO + 63) / 64 - G0 + 3) / 4;  // 64-piece groups per loader wave
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
  const int v0 = slice * SL;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;

  if (wave >= kComp) {
    // ---------------- loader waves ----------------
    const int lw = wave - kComp;
    const unsigned char* rec0 = rec_ws + (int64_t(n) * nc * H + h) * rec_bytes;
    const int64_t rec_stride = int64_t(H) * rec_bytes;
    const __bf16* dop = static_cast<const __bf16*>(g.d_out.ptr) + n * g.d_out.stride_b + h * g.d_out.stride_h;
    // Each slice workgroup of a head starts its copy at its own offset into the record, so that the slices do not
    // request the same missing lines of the shared record at the same moment.
    constexpr int kGroups = (NF + NDO + 63) / 64 - G0;
    const int rot = (slice * kGroups) / n_slices;
    auto copy = [&](int c, int buf) {
      const unsigned char* src = rec0 + c * rec_stride;
      unsigned char* dst = smem + buf * SB;
#pragma unroll
      for (int k = 0; k < NG; ++k) {
        const int j = lw + 4 * k;  // past the record: no copy
        const int grp = j < kGroups ? G0 + (j + rot) % kGroups : 1 << 20;
        const int idx = 64 * grp + lane;
        if (idx < NF + NDO) {
          const void* from;
          if (idx < NF) {
            from = src + idx * 16;
          } else {
            const int p = idx - NF, row = p / CPR, q = (p % CPR) ^ (row % CPR);  // slot p % CPR holds chunk q
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

    // dS' of this chunk (bf16, the chunk-local kernel's MFMA operand)
    __bf16* dsp = dstates + (size_t(bh) * nc + c) * kv;
#pragma unroll
    for (int m = 0; m < KT; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) dsp[size_t(16 * m + 4 * g4 + r) * V + c0 + l16] = bf(st[m][r]);

    bf16x8 sB[KS];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) sB[kk] = concat(pack4(st[2 * kk]), pack4(st[2 * kk + 1]));
    // dO blocks as 16x16x16 B operands: lane (column l16, k = 4 g4 + r) holds dO[16 i + 4 g4 + r][lc0 + l16]
    bf16x4 dob[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * i + 4 * g4 + (l16 >> 2), col = lc0 + 4 * (l16 & 3);
      dob[i] = lds_read_tr(smem, boff + DO + 2 * (row * SL + (((col >> 3) ^ (row % CPR)) << 3) + (col & 7)));
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
      // du transposed ([V][64] per chunk): the four tokens of this lane in one 8-byte store
      *reinterpret_cast<bf16x4*>(dubt + ((size_t(bh) * nc + c) * V + c0 + l16) * kChunk + 16 * i + 4 * g4) = pack4(acc);
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

// ================================ chunk-local gradients: one workgroup per (chunk, head) ================================
// Given S (the state entering the chunk), dS' (the gradient of the state leaving it), u and du (bf16, from the state
// replay and the reverse scan), everything of the chunk's backward that is local to it:
//   X2 = A^T du  (dv = beta (x) X2),   X1 = -X2 S^T,   dQd = dO S^T,   dKt = u dS'^T,
//   dSc = tril(dO u^T),   dL = -X2 u^T (strictly lower),   dP = diag(beta) dL,
//   dbeta = rowsum(X2 (x) V) + rowsum(X1 (x) K e^B) + rowsum(dL (x) P),
//   the four gated products, dq, dk and the gate gradient.
// With Y = diag(beta)(V - K e^B S) the forward has u = A Y, so dA = du Y^T and dL = -A^T dA A^T = -(A^T du)(A Y)^T
// = -X2 u^T; likewise A^T dW = -A^T du S^T = -X2 S^T.  Neither dW, dA nor a product with A^T on both sides is formed.
// Work split over K / 16 waves: the row-owned part (the block-local log2-gate cumsum, P = tril(K K^T (x) E, -1)
// and A = (I + diag(beta) P)^{-1}) runs on waves 0..3, one 16-row block each.  Everything after has wave w owning the
// 16-channel column tile w: X1, dQd, dKt, the gated products and the assembly for all 64 rows of its channels, so
// the gate gradient's cumulative sums over rows stay inside the wave.  X2 and dSc / dL are split by 16-token block.
// The value dimension is consumed in passes of 64 columns: dO, u and X2 go through swizzled LDS buffers, and the
// S and dS' rows of the wave's channels come straight from global memory as 16-byte B operands.
template <int K>
struct DLocalLds {
  static constexpr int NW = K / 16;       // waves
  static constexpr int KP = K + 8;        // bf16 pitch of the q / k rows
  static constexpr int MP = 68;           // fp32 pitch of P and A
  static constexpr int DP = 68;           // bf16 pitch of dSc and dP
  static constexpr int PB = 64 * 64 * 2;  // one swizzled bf16 [64][64] pass buffer
  static constexpr int RB0 = 64 * KP * 2 > 64 * MP * 4 ? 64 * KP * 2 : 64 * MP * 4;
  static constexpr int RB = RB0 > 2 * PB ? RB0 : 2 * PB;
  static constexpr int R1 = 0;            // q rows (bf16 [64][KP]), then P (fp32 [64][MP]), then 2 X2 pass buffers
  static constexpr int R2 = RB;           // k rows, then A, then 2 dO pass buffers
  static constexpr int R3 = 2 * RB;       // k e^{a_p - B} rows, then the inverse's scratch, then 2 u pass buffers
  static constexpr int R4 = 3 * RB;       // dSc, dP (bf16 [64][DP] each)
  static constexpr int TOT = 4 * RB;            // fp32 [4][K] block totals of the block-local log2-gate cumsum
  static constexpr int BETA = TOT + 4 * K * 4;  // fp32 [64]
  static constexpr int HOT = BETA + 256;        // u8 [4][K] channels whose block span exceeds kDiagSpan
  static constexpr int DB = HOT + 4 * K;        // fp32 [3][NW][64] per-wave dbeta partials, one slot per term
  static constexpr int BP = K + 4;              // fp32 pitch of BB
  static constexpr int BB = DB + 3 * NW * 256;  // fp32 [64][BP] block-local log2-gate cumsum (row-owned scan)
  static constexpr int kPre = 2;                // value passes whose dO, u and du^T are fetched at the start
  static constexpr int DOU = BB + 64 * BP * 4;  // [kPre][dO, u, du^T] swizzled pass buffers, filled by LDS DMA
  static constexpr int BYTES = DOU + kPre * 3 * PB;
  static_assert(2 * 64 * DP * 2 <= RB, "dSc and dP fit R4");
  static_assert((2 * NW * 64 + NW) * 4 <= RB, "the GDN row sums fit R1");
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

// Four consecutive elements of a gradient row (the last dimension is contiguous): one 16-byte (fp32) or 8-byte (bf16)
// store where the address is aligned for it, else four element stores.
__device__ __forceinline__ void store_grad4(const gdr_tensor& t, int64_t off, floatx4 v) {
  if (t.dtype == GDR_F32) {
    float* p = static_cast<float*>(const_cast<void*>(t.ptr)) + off;
    if ((reinterpret_cast<uintptr_t>(p) & 15) == 0) {
      *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
      return;
    }
  } else {
    __bf16* p = static_cast<__bf16*>(const_cast<void*>(t.ptr)) + off;
    if ((reinterpret_cast<uintptr_t>(p) & 7) == 0) {
      *reinterpret_cast<bf16x4*>(p) = pack4(v);
      return;
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) store_grad(t, off + r, v[r]);
}

// Element off + r * stride of a gradient tensor for the rows r < min(4, rows) (rows may be <= 0): the dtype test once.
__device__ __forceinline__ void store_rows4(const gdr_tensor& t, int64_t off, int64_t stride, const float (&v)[4],
                                            int rows) {
  if (t.dtype == GDR_F32) {
    float* p = static_cast<float*>(const_cast<void*>(t.ptr)) + off;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (r < rows) p[r * stride] = v[r];
  } else {
    __bf16* p = static_cast<__bf16*>(const_cast<void*>(t.ptr)) + off;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (r < rows) p[r * stride] = bf(v[r]);
  }
}

// Byte offset of (row, col) in a swizzled bf16 [64][64] pass buffer: 16-byte chunk q of row r sits at chunk q ^ (r % 8).
__device__ __forceinline__ int pb_off(int row, int col) {
  return row * 128 + (((col >> 3) ^ (row & 7)) << 4) + (col & 7) * 2;
}

__device__ __forceinline__ float pick4(const float (&x)[4], int r) {
  return r == 0 ? x[0] : (r == 1 ? x[1] : (r == 2 ? x[2] : x[3]));
}
__device__ __forceinline__ float pick4(bf16x4 x, int r) {
  return f32(r == 0 ? x[0] : (r == 1 ? x[1] : (r == 2 ? x[2] : x[3])));
}

// Sums of the 16-lane rows (width 16) and of the four 16-lane groups (over lanes l, l + 16, l + 32, l + 48).
__device__ __forceinline__ float sum16(float v) { return row_sum16(v); }  // its lanes' associations differ
__device__ __forceinline__ float sum_groups(float v) {                    // the same sum in every lane
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

template <int VARIANT, int K>
__global__ __launch_bounds__(64 * (K / 16)) void chunk_dlocal_kernel(const gdr_args a, const gdr_grads g, int nc,
                                                                     const __bf16* __restrict__ states,
                                                                     const __bf16* __restrict__ dstates,
                                                                     const __bf16* __restrict__ ubuf,
                                                                     const __bf16* __restrict__ dubt) {
  constexpr bool kDelta = VARIANT != GDR_GLA;
  constexpr int kGate = (VARIANT == GDR_KDA || VARIANT == GDR_GLA) ? 2 : (VARIANT == GDR_GDN ? 1 : 0);
  constexpr int KS = K / 32;
  using L = DLocalLds<K>;
  constexpr int NW = L::NW, NRT = 16 / NW, KP = L::KP, MP = L::MP, DP = L::DP, BP = L::BP;
  extern __shared__ __align__(16) unsigned char smem[];
  float* TOT = reinterpret_cast<float*>(smem + L::TOT);
  float* BETA = reinterpret_cast<float*>(smem + L::BETA);
  unsigned char* HOTF = smem + L::HOT;
  float* BB = reinterpret_cast<float*>(smem + L::BB);

  const int H = a.heads, V = a.value_dim, len = a.seq_len, BH = a.batch * H;
  const int bh = blockIdx.x % BH, c = blockIdx.x / BH;
  const int n = bh / H, h = bh % H;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, l16 = lane & 15, g4 = lane >> 4;
  const float scale = a.scale;
  const int t0 = c * kChunk, nvalid = min(kChunk, len - t0);
  const int d = 16 * w + l16;     // this lane's channel in the column-owned phases
  const int tb = w & 3;           // 16-token block of this wave in X2 (its tokens) and dSc / dL (its columns)
  const int rb = (w >> 2) * NRT;  // first of this wave's NRT row tiles of dSc / dL and value tiles of X2
  const __bf16* qp = static_cast<const __bf16*>(a.q.ptr) + n * a.q.stride_b + h * a.q.stride_h;
  const __bf16* kp = static_cast<const __bf16*>(a.k.ptr) + n * a.k.stride_b + h * a.k.stride_h;
  const __bf16* vp = static_cast<const __bf16*>(a.v.ptr) + n * a.v.stride_b + h * a.v.stride_h;
  const float* gp = kGate ? static_cast<const float*>(a.gate.ptr) + n * a.gate.stride_b + h * a.gate.stride_h : nullptr;
  const float* betap = kDelta ? static_cast<const float*>(a.beta.ptr) + n * a.beta.stride_b + h * a.beta.stride_h
                              : nullptr;
  auto gate_at = [&](int row, int ch) -> float {  // natural-log gate of chunk row `row` (< nvalid), channel ch
    const int64_t tt = t0 + row;
    return kGate == 2 ? gp[tt * a.gate.stride_t + ch] : gp[tt * a.gate.stride_t];
  };
  const floatx4 z4 = {0.f, 0.f, 0.f, 0.f};
  const size_t cidx = size_t(bh) * nc + c;
  const __bf16* ug = ubuf + cidx * kChunk * V;  // u [64][V]
  const __bf16* dop = static_cast<const __bf16*>(g.d_out.ptr) + n * g.d_out.stride_b + h * g.d_out.stride_h;

  // dO and u columns of the first kPre value passes (token rows) and du^T rows of those columns, copied into their
  // swizzled LDS buffers (global_load_lds_dwordx4: lane i lands at the wave's base + 16 i, i.e. row 8 (m mod 8) + i / 8
  // of the buffer, slot i % 8, which holds chunk (i % 8) ^ (row % 8) of the row) by `nw` waves from wave w0 of them.
  // dO rows past the sequence end read its last row; they and the u rows there are zeroed once the copies have landed,
  // and du^T's columns there are masked where they are used.  The compiler orders every LDS read that follows a
  // global_load_lds in the same wave behind the whole copy, so with eight waves (and a delta rule) the copies are
  // issued by waves 4..7 after the P tiles, which then have no LDS reads until after the inverse (that waves 0..3
  // compute meanwhile); otherwise they go out behind the row loads.
  constexpr bool kLateCopies = NW >= 8 && kDelta;
  auto copy_pass_buffers = [&](int w0, int nw) {
    const int npre = min(V / 64, L::kPre);
#pragma unroll
    for (int k = 0; k < 3 * L::kPre * 8 / (kLateCopies ? NW / 2 : NW); ++k) {
      const int m = w0 + nw * k, ps = m / 24, tn = (m >> 3) % 3, row = 8 * (m & 7) + (lane >> 3);
      const int chunk8 = 8 * ((lane & 7) ^ (row & 7)), col = 64 * ps + chunk8;
      const __bf16* src = tn == 0   ? dop + (t0 + min(row, nvalid - 1)) * int64_t(g.d_out.stride_t) + col
                          : tn == 1 ? ug + size_t(row) * V + col
                                    : dubt + (cidx * V + 64 * ps + row) * kChunk + chunk8;
      if (ps < npre)
        __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(smem + L::DOU + m * 1024),
                                         16, 0, 0);
    }
  };
  // The workgroup barriers of the P tiles and the inverse, which the late copies are in flight across: the
  // compiler's LDS release fence would wait for them (it counts the copies as LDS writes, on vmcnt), so this one
  // waits for the wave's own LDS operations only.  The copies are waited for before the passes read them.
  auto copy_barrier = [&]() {
    if constexpr (kLateCopies) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else lds_barrier();
  };
  auto zero_past_end = [&]() {  // the prefetched dO and u rows past the sequence end become zeros
    if (nvalid < kChunk) {
      for (int idx = tid; idx < L::kPre * 2 * 64 * 8; idx += 64 * NW) {
        const int ps = idx >> 10, tn = (idx >> 9) & 1, row = (idx >> 3) & 63;
        if (row >= nvalid)
          *reinterpret_cast<uint4*>(smem + L::DOU + (3 * ps + tn) * L::PB + 16 * (idx & 511)) = make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };

  // ---- 1. row-owned (block p = w mod 4; lane: row 16 p + l16, channels 32 kk + 8 g4 + j for this wave's KH channel
  // groups kk0 .. kk0 + KH - 1; with eight waves, waves p and p + 4 take the two halves of the channels): q, k rows
  // into LDS; the log2-gate cumsum within the block (b); P's operands k e^{b} (A), k e^{b_15 - b} (B, via LDS) and
  // the diagonal tile's k e^{+-(b - mid)}; block totals and hot-channel flags ----
  constexpr int KH = NW >= 8 ? KS / 2 : KS;  // 32-channel groups per wave in the row-owned phases
  const int kk0 = NW >= 8 ? (w >> 2) * KH : 0;
  bf16x8 lk[KH], ae[KH], af[KH];
  {
    const int p = w & 3, trow = 16 * p + l16;
    const bool valid = trow < nvalid;
    const int64_t tc = t0 + min(trow, nvalid - 1);
    const uint32_t keep = valid ? 0xffffffffu : 0u;
    __bf16* QL = reinterpret_cast<__bf16*>(smem + L::R1);
    __bf16* KL = reinterpret_cast<__bf16*>(smem + L::R2);
    __bf16* KAPL = reinterpret_cast<__bf16*>(smem + L::R3);
    float bl[KH][8];
    bf16x8 kr8[KH];
#pragma unroll
    for (int x = 0; x < KH; ++x) {
      const int ch = 32 * (kk0 + x) + 8 * g4;
      uint4 qr = *reinterpret_cast<const uint4*>(qp + tc * a.q.stride_t + ch);
      uint4 kr = *reinterpret_cast<const uint4*>(kp + tc * a.k.stride_t + ch);
      qr = make_uint4(qr.x & keep, qr.y & keep, qr.z & keep, qr.w & keep);
      kr = make_uint4(kr.x & keep, kr.y & keep, kr.z & keep, kr.w & keep);
      *reinterpret_cast<uint4*>(QL + trow * KP + ch) = qr;
      *reinterpret_cast<uint4*>(KL + trow * KP + ch) = kr;
      kr8[x] = __builtin_bit_cast(bf16x8, kr);
      if constexpr (kGate == 2) {
        const float4 g0 = *reinterpret_cast<const float4*>(gp + tc * a.gate.stride_t + ch);
        const float4 g1 = *reinterpret_cast<const float4*>(gp + tc * a.gate.stride_t + ch + 4);
        bl[x][0] = g0.x; bl[x][1] = g0.y; bl[x][2] = g0.z; bl[x][3] = g0.w;
        bl[x][4] = g1.x; bl[x][5] = g1.y; bl[x][6] = g1.z; bl[x][7] = g1.w;
      } else {
        const float gs = kGate == 1 ? gp[tc * a.gate.stride_t] : 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) bl[x][j] = gs;
      }
    }
    if constexpr (!kLateCopies) copy_pass_buffers(w, NW);
    if (kDelta && kk0 == 0 && g4 == 0) BETA[trow] = valid ? betap[tc * a.beta.stride_t] : 0.f;
    const float kf = valid ? kLog2e : 0.f;
#pragma unroll
    for (int x = 0; x < KH; ++x)
#pragma unroll
      for (int j = 0; j < 8; ++j) bl[x][j] = row_scan16(bl[x][j] * kf);
#pragma unroll
    for (int x = 0; x < KH; ++x) {
      const int ch = 32 * (kk0 + x) + 8 * g4;
      bf16x8 kap;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float b = bl[x][j];
        const float top = row_lane<0>(b), bot = row_lane<15>(b);
        const bool hot = top - bot > kDiagSpan;
        const float mid = 0.5f * (top + bot), kv = f32(kr8[x][j]);
        kap[j] = bf(kv * ex2(bot - b));
        lk[x][j] = bf(kv * ex2(b));
        ae[x][j] = bf(hot ? 0.f : kv * ex2(b - mid));
        af[x][j] = bf(hot ? 0.f : kv * ex2(mid - b));
        if (l16 == 0) HOTF[p * K + ch + j] = hot ? 1 : 0;
      }
      *reinterpret_cast<bf16x8*>(KAPL + trow * KP + ch) = kap;
      if constexpr (kGate != 0) {
        *reinterpret_cast<float4*>(BB + trow * BP + ch) = make_float4(bl[x][0], bl[x][1], bl[x][2], bl[x][3]);
        *reinterpret_cast<float4*>(BB + trow * BP + ch + 4) = make_float4(bl[x][4], bl[x][5], bl[x][6], bl[x][7]);
      }
      if (l16 == 15) {
        *reinterpret_cast<float4*>(TOT + p * K + ch) = make_float4(bl[x][0], bl[x][1], bl[x][2], bl[x][3]);
        *reinterpret_cast<float4*>(TOT + p * K + ch + 4) = make_float4(bl[x][4], bl[x][5], bl[x][6], bl[x][7]);
      }
    }
  }

  if constexpr (!kLateCopies) __builtin_amdgcn_s_waitcnt(0);  // this wave's pass-buffer copies have landed
  lds_barrier();

  // ---- 1b. column-owned (every wave, channel d): the in-chunk log2-gate cumsum B at rows 16 j + 4 g4 + r, the
  // block-local cumsum plus the totals of the blocks before ----
  if constexpr (!kLateCopies) zero_past_end();
  float bc[4][4];
  {
    float pre = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int r = 0; r < 4; ++r) bc[j][r] = kGate ? BB[(16 * j + 4 * g4 + r) * BP + d] + pre : 0.f;
      if (kGate && j < 3) pre += TOT[j * K + d];
    }
  }

  // ---- 2. q, k of channel d at rows 16 j + 4 g4 + r (the 16x16x16 B-operand layout); P's tiles of row block
  // w mod 4 over this wave's channel groups ----
  bf16x4 qc[4], kc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 16 * j + 4 * g4 + (l16 >> 2), col = 16 * w + 4 * (l16 & 3);
    qc[j] = lds_read_tr(smem, L::R1 + 2 * (row * KP + col));
    kc[j] = lds_read_tr(smem, L::R2 + 2 * (row * KP + col));
  }
  floatx4 pacc[3] = {z4, z4, z4}, pdiag = z4;
  if constexpr (kDelta) {
    // P_pj = (k e^{b}) (k e^{b_15 - b})^T e^{a_{p-1} - a_j}: the last factor is 1 for j = p - 1, else the block
    // totals in between.  Tiles j >= p are computed and dropped: no MFMA under a branch.
    const __bf16* KAPL = reinterpret_cast<const __bf16*>(smem + L::R3);
    const int p = w & 3;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      floatx4 acc = z4;
#pragma unroll
      for (int x = 0; x < KH; ++x) {
        const int ch = 32 * (kk0 + x) + 8 * g4;
        bf16x8 bk = *reinterpret_cast<const bf16x8*>(KAPL + (16 * j + l16) * KP + ch);
        if (j < p - 1) {
          float4 f0 = make_float4(0.f, 0.f, 0.f, 0.f), f1 = f0;
          for (int q = j + 1; q < p; ++q) {
            const float4 u0 = *reinterpret_cast<const float4*>(TOT + q * K + ch);
            const float4 u1 = *reinterpret_cast<const float4*>(TOT + q * K + ch + 4);
            f0.x += u0.x; f0.y += u0.y; f0.z += u0.z; f0.w += u0.w;
            f1.x += u1.x; f1.y += u1.y; f1.z += u1.z; f1.w += u1.w;
          }
          const float fs[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) bk[e] = bf(f32(bk[e]) * ex2(fs[e]));
        }
        acc = mfma32(lk[x], bk, acc);
      }
      pacc[j] = acc;
    }
    // diagonal tile: (k e^{b - mid}) (k e^{mid - b})^T with mid the middle of the block's gate range
#pragma unroll
    for (int x = 0; x < KH; ++x) pdiag = mfma32(ae[x], af[x], pdiag);
    if (NW >= 8 && w >= 4) {  // the second channel half's partial tiles, to R4 (unused until step 5)
      floatx4* part = reinterpret_cast<floatx4*>(smem + L::R4) + p * 4 * 64 + lane;
#pragma unroll
      for (int j = 0; j < 3; ++j) part[64 * j] = pacc[j];
      part[64 * 3] = pdiag;
    }
  }
  lds_barrier();  // the q and k rows are read: R1 takes P, R2 takes A
  if constexpr (kLateCopies) {
    if (w >= NW / 2) copy_pass_buffers(w - NW / 2, NW / 2);
  }

  // v rows for rowsum(X2 (x) V), loaded one value pass ahead of their use (the first pass's before the inverse)
  auto load_vv = [&](int v0, bf16x4 (&dst)[NRT]) {
#pragma unroll
    for (int x = 0; x < NRT; ++x)
      dst[x] = ld4(vp + int64_t(t0 + min(16 * tb + l16, nvalid - 1)) * a.v.stride_t + v0 + 16 * (rb + x) + 4 * g4);
  };
  bf16x4 vnext[NRT];
  if constexpr (kDelta) load_vv(0, vnext);

  bf16x8 aB[2];        // A[32 kb + 8 g4 + e][16 tb + l16]: B operand of X2^T = du^T A
  float pv[NRT][4];    // P at this wave's dL positions (16 (rb + ii) + 4 g4 + r, 16 tb + l16)
  if constexpr (kDelta) {
    float* PL = reinterpret_cast<float*>(smem + L::R1);
    float* AL = reinterpret_cast<float*>(smem + L::R2);
    float* YS = reinterpret_cast<float*>(smem + L::R3);
    if (w < 4) {
      const int p = w;
      if constexpr (NW >= 8) {  // plus the other channel half's partial tiles
        const floatx4* part = reinterpret_cast<const floatx4*>(smem + L::R4) + p * 4 * 64 + lane;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const floatx4 o = part[64 * j];
#pragma unroll
          for (int r = 0; r < 4; ++r) pacc[j][r] += o[r];
        }
        const floatx4 o = part[64 * 3];
#pragma unroll
        for (int r = 0; r < 4; ++r) pdiag[r] += o[r];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 4 * g4 + r;
          const float off = j < 3 ? pacc[j < 3 ? j : 0][r] : 0.f;
          PL[(16 * p + t) * MP + 16 * j + l16] = j < p ? off : ((j == p && l16 < t) ? pdiag[r] : 0.f);
        }
      bool hot = false;  // any hot channel in this block
      for (int ch = lane; ch < K; ch += 64) hot |= HOTF[p * K + ch] != 0;
      if (__any(hot)) {
        // exact terms of the hot channels of the diagonal tile, pair (t, s < t) of the block, from the gates
        const __bf16* KL = reinterpret_cast<const __bf16*>(smem + L::R2);
        for (int q = lane; q < 120; q += 64) {
          int t = 1;
          while (t * (t + 1) / 2 <= q) ++t;
          const int s2 = q - t * (t - 1) / 2;
          const int rt = 16 * p + t, rs = 16 * p + s2;
          if (rt >= nvalid) continue;  // rows past the sequence end have k = 0
          float add = 0.f;
          for (int dd = 0; dd < K; ++dd) {
            if (!HOTF[p * K + dd]) continue;
            float e = 0.f;
            for (int x = rs + 1; x <= rt; ++x) e += gate_at(x, dd);
            add += f32(KL[rt * KP + dd]) * f32(KL[rs * KP + dd]) * ex2(e * kLog2e);
          }
          PL[rt * MP + rs] += add;
        }
      }
    }
    copy_barrier();

    // ---- 3. A = (I + diag(beta) P)^{-1} (waves 0..3): diagonal blocks by forward substitution, then block rows
    // 1..3 on fp32 MFMA with wave p owning tile column p ----
    if (w < 4) {
      const int p = w;
      if (lane < 16) {
        float x[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float acc = r == lane ? 1.f : 0.f;
          const float br = BETA[16 * p + r];
#pragma unroll
          for (int m = 0; m < r; ++m) acc -= br * PL[(16 * p + r) * MP + 16 * p + m] * x[m];
          x[r] = acc;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) AL[(16 * p + r) * MP + 16 * p + lane] = x[r];
      }
      for (int idx = lane; idx < 16 * 64; idx += 64) {
        const int x = idx >> 6, col = idx & 63;
        if (col >= 16 * (p + 1) || col < 16 * p) AL[(16 * p + x) * MP + col] = 0.f;
      }
    }
    copy_barrier();
    // Y = diag(beta) P[block i, :16 i] A[:16 i, block p] (wave-private scratch), A_ip = -A_ii Y (zero for p >= i).
    // Wave p reads only column block p of A (its own writes, and the zeros and diagonal blocks in place before the
    // barrier above), A_ii and its own scratch, so the block rows need no barrier between them: a wave's LDS
    // accesses complete in order.
#pragma unroll
    for (int i = 1; i < 4; ++i) {
      if (w < 4) {
        const int p = w, ta = 16 * i + l16;
        const float bt = BETA[ta];
        floatx4 y = z4;
#pragma unroll
        for (int q0 = 0; q0 < 16 * i; q0 += 4)
          y = mfma_f32(bt * PL[ta * MP + q0 + g4], AL[(q0 + g4) * MP + 16 * p + l16], y);
#pragma unroll
        for (int r = 0; r < 4; ++r) YS[(16 * p + 4 * g4 + r) * MP + l16] = y[r];
        floatx4 zz = z4;
#pragma unroll
        for (int q0 = 0; q0 < 16; q0 += 4)
          zz = mfma_f32(AL[ta * MP + 16 * i + q0 + g4], YS[(16 * p + q0 + g4) * MP + l16], zz);
        if (p < i) {
#pragma unroll
          for (int r = 0; r < 4; ++r) AL[(16 * i + 4 * g4 + r) * MP + 16 * p + l16] = -zz[r];
        }
      }
    }
    copy_barrier();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 8; ++e) aB[kb][e] = bf(AL[(32 * kb + 8 * g4 + e) * MP + 16 * tb + l16]);
#pragma unroll
    for (int ii = 0; ii < NRT; ++ii)
#pragma unroll
      for (int r = 0; r < 4; ++r) pv[ii][r] = PL[(16 * (rb + ii) + 4 * g4 + r) * MP + 16 * tb + l16];
  } else {
    // GLA: A = I, X2 = du
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 8; ++e) aB[kb][e] = bf(32 * kb + 8 * g4 + e == 16 * tb + l16 ? 1.f : 0.f);
  }
  if constexpr (kLateCopies) __builtin_amdgcn_s_waitcnt(0);  // this wave's pass-buffer copies have landed
  lds_barrier();  // P and A are read: R1 .. R3 take the pass buffers
  if constexpr (kLateCopies) {
    zero_past_end();
    if (nvalid < kChunk) lds_barrier();
  }

  // ---- 4. passes over 64 value columns: X2 (dv, dbeta), then X1, dQd, dKt (channel tile w, all rows) and dSc,
  // dL (columns of block tb, this wave's row tiles), and bnd = rowsum(S (x) dS') of channel d ----
  const __bf16* Sg = states + (cidx * K + d) * V;     // row d of S
  const __bf16* dSg = dstates + (cidx * K + d) * V;   // row d of dS'
  const __bf16* dutg = dubt + cidx * V * kChunk;      // du^T [V][64]
  floatx4 x1[4], qd[4], kt[4], sc[NRT], dl[NRT];
#pragma unroll
  for (int i = 0; i < 4; ++i) x1[i] = qd[i] = kt[i] = z4;
#pragma unroll
  for (int ii = 0; ii < NRT; ++ii) sc[ii] = dl[ii] = z4;
  float bnd = 0.f, dbv = 0.f;
  for (int v0 = 0; v0 < V; v0 += 64) {
    const int buf = (v0 >> 6) & 1, ps = v0 >> 6;
    const bool pre = ps < L::kPre;  // dO and u already in their LDS buffers
    unsigned char* X2B = smem + L::R1 + buf * L::PB;
    unsigned char* DOB = pre ? smem + L::DOU + 3 * ps * L::PB : smem + L::R2 + buf * L::PB;
    unsigned char* UB = pre ? smem + L::DOU + (3 * ps + 1) * L::PB : smem + L::R3 + buf * L::PB;
    const unsigned char* DUB = smem + L::DOU + (3 * ps + 2) * L::PB;  // du^T rows of the pass (pre only)
    // this pass's global operands first, so their latency overlaps the staging below: du^T for X2, v for
    // rowsum(X2 (x) V), and the S / dS' rows of channel d
    bf16x8 adu[NRT][2], sfr[2], dsfr[2];
    bf16x4 vv[NRT];
    if constexpr (kDelta) {
#pragma unroll
      for (int x = 0; x < NRT; ++x) vv[x] = vnext[x];
      if (v0 + 64 < V) load_vv(v0 + 64, vnext);
    }
#pragma unroll
    for (int x = 0; x < NRT; ++x) {
      const int v = v0 + 16 * (rb + x);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
        adu[x][kb] = pre ? *reinterpret_cast<const bf16x8*>(DUB + pb_off(16 * (rb + x) + l16, 32 * kb + 8 * g4))
                         : ld8(dutg + size_t(v + l16) * kChunk + 32 * kb + 8 * g4);
    }
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      sfr[kv] = ld8(Sg + v0 + 32 * kv + 8 * g4);
      dsfr[kv] = ld8(dSg + v0 + 32 * kv + 8 * g4);
    }
    // later passes: dO and u columns [v0, v0 + 64), rows past the sequence end as zeros (the buffers written here
    // were last read two passes ago, before the previous pass's barrier)
    for (int idx = pre ? 64 * 8 : tid; idx < 64 * 8; idx += 64 * NW) {
      const int row = idx >> 3, q = idx & 7;
      uint4 dv = make_uint4(0u, 0u, 0u, 0u), uv = make_uint4(0u, 0u, 0u, 0u);
      if (row < nvalid) {
        dv = *reinterpret_cast<const uint4*>(dop + int64_t(t0 + row) * g.d_out.stride_t + v0 + 8 * q);
        uv = *reinterpret_cast<const uint4*>(ug + size_t(row) * V + v0 + 8 * q);
      }
      *reinterpret_cast<uint4*>(DOB + pb_off(row, 8 * q)) = dv;
      *reinterpret_cast<uint4*>(UB + pb_off(row, 8 * q)) = uv;
    }
    // X2^T tiles (value tile rb + x of the pass, tokens of block tb): lane holds X2[16 tb + l16][v + 4 g4 + r]
#pragma unroll
    for (int x = 0; x < NRT; ++x) {
      const int vl = 16 * (rb + x), v = v0 + vl;
      floatx4 acc = z4;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int s0 = 32 * kb + 8 * g4;
        bf16x8 du8 = adu[x][kb];
        if (s0 + 8 > nvalid) {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (s0 + e >= nvalid) du8[e] = bf(0.f);
        }
        acc = mfma32(du8, aB[kb], acc);
      }
      const int t = 16 * tb + l16;
      const float bt = kDelta ? BETA[t] : 1.f;
      if (t < nvalid) {
        const int64_t off =
            n * g.d_value.stride_b + h * g.d_value.stride_h + int64_t(t0 + t) * g.d_value.stride_t + v + 4 * g4;
        store_grad4(g.d_value, off, floatx4{bt * acc[0], bt * acc[1], bt * acc[2], bt * acc[3]});
      }
      if constexpr (kDelta) {
#pragma unroll
        for (int r = 0; r < 4; ++r) dbv += acc[r] * f32(vv[x][r]);
        *reinterpret_cast<bf16x4*>(X2B + pb_off(t, vl + 4 * g4)) = pack4(acc);
      }
    }
    lds_barrier();
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      const int lc = 32 * kv + 8 * g4;
#pragma unroll
      for (int e = 0; e < 8; ++e) bnd += f32(sfr[kv][e]) * f32(dsfr[kv][e]);
      const bf16x8 us = *reinterpret_cast<const bf16x8*>(UB + pb_off(16 * tb + l16, lc));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * i + l16;
        qd[i] = mfma32(*reinterpret_cast<const bf16x8*>(DOB + pb_off(row, lc)), sfr[kv], qd[i]);
        kt[i] = mfma32(*reinterpret_cast<const bf16x8*>(UB + pb_off(row, lc)), dsfr[kv], kt[i]);
        if constexpr (kDelta)
          x1[i] = mfma32(*reinterpret_cast<const bf16x8*>(X2B + pb_off(row, lc)), sfr[kv], x1[i]);
      }
#pragma unroll
      for (int ii = 0; ii < NRT; ++ii) {
        const int row = 16 * (rb + ii) + l16;
        sc[ii] = mfma32(*reinterpret_cast<const bf16x8*>(DOB + pb_off(row, lc)), us, sc[ii]);
        if constexpr (kDelta) dl[ii] = mfma32(*reinterpret_cast<const bf16x8*>(X2B + pb_off(row, lc)), us, dl[ii]);
      }
    }
  }

  // ---- 5. dSc = tril(dO u^T) and dP = diag(beta) dL (bf16) into R4; dbeta partials into this wave's DB row ----
  __bf16* DSCL = reinterpret_cast<__bf16*>(smem + L::R4);
  __bf16* DPL = DSCL + 64 * DP;
  // dbeta partials of this wave, each row written once per term: rowsum(dL (x) P) at DB[t], rowsum(X2 (x) V) at
  // DB[64 NW + t], rowsum(X1 (x) K e^B) at DB[128 NW + t] (rows this wave does not reach stay zero)
  float* DB = reinterpret_cast<float*>(smem + L::DB) + 64 * w;
  DB[lane] = 0.f;
  DB[64 * NW + lane] = 0.f;
#pragma unroll
  for (int ii = 0; ii < NRT; ++ii)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 16 * (rb + ii) + 4 * g4 + r, s = 16 * tb + l16;
      DSCL[t * DP + s] = bf(t >= s ? sc[ii][r] : 0.f);
      if constexpr (kDelta) {
        const float dlv = t > s ? -dl[ii][r] : 0.f;
        DPL[t * DP + s] = bf(BETA[t] * dlv);
        const float v = sum16(dlv * pv[ii][r]);  // rowsum(dL (x) P) over this wave's 16 columns
        if (l16 == 0) DB[t] = v;
      }
    }
  if constexpr (kDelta) {
    const float v = sum_groups(dbv);  // rowsum(X2 (x) V) over this wave's value tiles
    if (g4 == 0) DB[64 * NW + 16 * tb + l16] = v;
  }
  bnd = sum_groups(bnd);
  lds_barrier();

  // ---- 6. per 16-row tile i of channel d: the gated products off the diagonal (block-anchored factors, each <= 1)
  // and on it (anchored at the middle of the block's gate range; hot channels exactly), then dq, dk and the gate
  // terms.  left: rows t of tile i, sources s <= t;  key: rows s of tile i, sources t >= s. ----
  float anc[4], mid[4];
  bool hot[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    anc[j] = from_row<3>(bc[j][3]);  // a_j = B at row 16 j + 15
    const float top = from_row<0>(bc[j][0]);
    mid[j] = 0.5f * (top + anc[j]);
    hot[j] = top - anc[j] > kDiagSpan;
  }
  const float bend = anc[3];
  float gtv[4][4], ktv[4][4];
  const int64_t qrow0 = n * g.d_query.stride_b + h * g.d_query.stride_h + d;
  const int64_t krow0 = n * g.d_key.stride_b + h * g.d_key.stride_h + d;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    floatx4 lq = z4, lp = z4, kq = z4, kp2 = z4;
#pragma unroll
    for (int j = 0; j < i; ++j) {  // left, sources in blocks j < i: (k e^{a_{i-1} - B_s}) then e^{B_t - a_{i-1}}
      bf16x4 bop;
#pragma unroll
      for (int r = 0; r < 4; ++r) bop[r] = bf(f32(kc[j][r]) * ex2(anc[i - 1] - bc[j][r]));
      lq = mfma16(ld4(DSCL + (16 * i + l16) * DP + 16 * j + 4 * g4), bop, lq);
      if constexpr (kDelta) lp = mfma16(ld4(DPL + (16 * i + l16) * DP + 16 * j + 4 * g4), bop, lp);
    }
    if (i > 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float f = ex2(bc[i][r] - anc[i - 1]);
        lq[r] *= f;
        lp[r] *= f;
      }
    }
#pragma unroll
    for (int j = i + 1; j < 4; ++j) {  // key, sources in blocks j > i: (x e^{B_t - a_i}) then e^{a_i - B_s}
      bf16x4 bq, bk;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float f = ex2(bc[j][r] - anc[i]);
        bq[r] = bf(f32(qc[j][r]) * f);
        bk[r] = bf(f32(kc[j][r]) * f);
      }
      const int off = 2 * ((16 * j + 4 * g4 + (l16 >> 2)) * DP + 16 * i + 4 * (l16 & 3));
      kq = mfma16(lds_read_tr(smem, L::R4 + off), bq, kq);
      if constexpr (kDelta) kp2 = mfma16(lds_read_tr(smem, L::R4 + 64 * DP * 2 + off), bk, kp2);
    }
    if (i < 3) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float f = ex2(anc[i] - bc[i][r]);
        kq[r] *= f;
        kp2[r] *= f;
      }
    }
    {  // diagonal tile (i, i)
      bf16x4 bkf, bqe, bke;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = hot[i] ? 0.f : ex2(bc[i][r] - mid[i]), f = hot[i] ? 0.f : ex2(mid[i] - bc[i][r]);
        bkf[r] = bf(f32(kc[i][r]) * f);
        bqe[r] = bf(f32(qc[i][r]) * e);
        bke[r] = bf(f32(kc[i][r]) * e);
      }
      const int off = 2 * ((16 * i + 4 * g4 + (l16 >> 2)) * DP + 16 * i + 4 * (l16 & 3));
      const floatx4 lqd = mfma16(ld4(DSCL + (16 * i + l16) * DP + 16 * i + 4 * g4), bkf, z4);
      const floatx4 kqd = mfma16(lds_read_tr(smem, L::R4 + off), bqe, z4);
      floatx4 lpd = z4, kpd = z4;
      if constexpr (kDelta) {
        lpd = mfma16(ld4(DPL + (16 * i + l16) * DP + 16 * i + 4 * g4), bkf, z4);
        kpd = mfma16(lds_read_tr(smem, L::R4 + 64 * DP * 2 + off), bke, z4);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = hot[i] ? 0.f : ex2(bc[i][r] - mid[i]), f = hot[i] ? 0.f : ex2(mid[i] - bc[i][r]);
        lq[r] += e * lqd[r];
        lp[r] += e * lpd[r];
        kq[r] += f * kqd[r];
        kp2[r] += f * kpd[r];
      }
    }
    if (__any(hot[i])) {
      // hot channels of block i: exact fp32 sums; row 16 i + x of channel d lives in lane l16 + 16 (x / 4), slot x % 4
      float sq[4] = {0.f, 0.f, 0.f, 0.f}, sl[4] = {0.f, 0.f, 0.f, 0.f};
      float sk[4] = {0.f, 0.f, 0.f, 0.f}, sp[4] = {0.f, 0.f, 0.f, 0.f};
      for (int x = 0; x < 16; ++x) {
        const int src = l16 + 16 * (x >> 2), rr = x & 3;
        const float bx = __shfl(pick4(bc[i], rr), src);
        const float kx = __shfl(pick4(kc[i], rr), src), qx = __shfl(pick4(qc[i], rr), src);
        if (hot[i]) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int tl = 4 * g4 + r, rt = 16 * i + tl, rx = 16 * i + x;
            if (x <= tl) {  // left: (t, s = x)
              const float e = ex2(bc[i][r] - bx) * kx;
              sq[r] += f32(DSCL[rt * DP + rx]) * e;
              if constexpr (kDelta) sl[r] += f32(DPL[rt * DP + rx]) * e;
            }
            if (x >= tl) {  // key: (t' = x, s = t)
              const float e = ex2(bx - bc[i][r]);
              sk[r] += f32(DSCL[rx * DP + rt]) * qx * e;
              if constexpr (kDelta) sp[r] += f32(DPL[rx * DP + rt]) * kx * e;
            }
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        lq[r] += sq[r];
        lp[r] += sl[r];
        kq[r] += sk[r];
        kp2[r] += sp[r];
      }
    }
    // assembly of row tile i
    float dq4[4], dk4[4];
    const float4 b4 = kDelta ? *reinterpret_cast<const float4*>(BETA + 16 * i + 4 * g4) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 16 * i + 4 * g4 + r;
      const float eb = ex2(bc[i][r]);
      const float qv = f32(qc[i][r]), kv = f32(kc[i][r]);
      const float dqv = scale * (qd[i][r] * eb + lq[r]);
      const float x1v = kDelta ? -x1[i][r] : 0.f;  // X1 = -X2 S^T
      const float bt = r == 0 ? b4.x : r == 1 ? b4.y : r == 2 ? b4.z : b4.w;
      const float dkp = bt * eb * x1v + lp[r];       // the e^{+B} roles
      const float dkn = scale * kq[r] + kp2[r];      // the e^{-B} roles
      const float dktr = kt[i][r] * ex2(bend - bc[i][r]);
      gtv[i][r] = qv * dqv + kv * (dkp - dkn);
      ktv[i][r] = kv * dktr;
      if constexpr (kDelta) {
        const float v = sum16(x1v * kv * eb);  // rowsum(X1 (x) K e^B) over this wave's channels
        if (l16 == 0) DB[128 * NW + t] = v;
      }
      dq4[r] = dqv;
      dk4[r] = dkp + dkn + dktr;
    }
    const int t4 = 16 * i + 4 * g4;  // the lane's four rows t4 .. t4 + 3, one dtype branch per tensor
    store_rows4(g.d_query, qrow0 + int64_t(t0 + t4) * g.d_query.stride_t, g.d_query.stride_t, dq4, nvalid - t4);
    store_rows4(g.d_key, krow0 + int64_t(t0 + t4) * g.d_key.stride_t, g.d_key.stride_t, dk4, nvalid - t4);
  }

  // ---- 7. gate gradient: inclusive suffix over rows of the non-Kt terms + e^{B_end} rowsum(S (x) dS') + exclusive
  // prefix of the Kt-role terms ----
  if constexpr (kGate == 2) {
    float* dgp = static_cast<float*>(const_cast<void*>(g.d_gate.ptr)) + n * g.d_gate.stride_b + h * g.d_gate.stride_h;
    float kex[4][4];
    float carry = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float s = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        kex[i][r] = s;
        s += ktv[i][r];
      }
      float total;
      const float incl = rows_scan(s, false, total);  // over the groups g4' <= g4
      const float before = carry + (incl - s);
#pragma unroll
      for (int r = 0; r < 4; ++r) kex[i][r] += before;
      carry += total;
    }
    carry = ex2(bend) * bnd;
#pragma unroll
    for (int i = 3; i >= 0; --i) {
      float s = 0.f, suf[4];
#pragma unroll
      for (int r = 3; r >= 0; --r) {
        s += gtv[i][r];
        suf[r] = s;
      }
      float total;
      const float incl = rows_scan(s, true, total);  // over the groups g4' >= g4
      const float after = carry + (incl - s);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * i + 4 * g4 + r;
        if (t < nvalid) dgp[int64_t(t0 + t) * g.d_gate.stride_t + d] = after + suf[r] + kex[i][r];
      }
      carry += total;
    }
  } else if constexpr (kGate == 1) {
    float* GPS = reinterpret_cast<float*>(smem + L::R1);  // [NW][64] row sums of GT, [NW][64] of the Kt role, [NW] bnd
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float a1 = sum16(gtv[i][r]), a2 = sum16(ktv[i][r]);
        if (l16 == 0) {
          GPS[w * 64 + 16 * i + 4 * g4 + r] = a1;
          GPS[(NW + w) * 64 + 16 * i + 4 * g4 + r] = a2;
        }
      }
    const float bs = sum16(bnd);
    if (lane == 0) GPS[2 * NW * 64 + w] = bs;
  }
  if constexpr (kDelta || kGate == 1) lds_barrier();
  if constexpr (kDelta) {
    if (tid < nvalid) {
      const float* DBA = reinterpret_cast<const float*>(smem + L::DB);
      float v = 0.f;
#pragma unroll
      for (int q = 0; q < NW; ++q) v += DBA[q * 64 + tid] + DBA[(NW + q) * 64 + tid] + DBA[(2 * NW + q) * 64 + tid];
      float* dbp = static_cast<float*>(const_cast<void*>(g.d_beta.ptr)) + n * g.d_beta.stride_b + h * g.d_beta.stride_h;
      dbp[int64_t(t0 + tid) * g.d_beta.stride_t] = v;
    }
  }
  if constexpr (kGate == 1) {
    if (w == 0) {  // lane = row t
      const float* GPS = reinterpret_cast<const float*>(smem + L::R1);
      float gt = 0.f, ktr = 0.f, bs = 0.f;
#pragma unroll
      for (int q = 0; q < NW; ++q) {
        gt += GPS[q * 64 + lane];
        ktr += GPS[(NW + q) * 64 + lane];
        bs += GPS[2 * NW * 64 + q];
      }
      float pre = ktr, suf = gt;  // inclusive prefix of the Kt role, inclusive suffix of the rest
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const float yp = __shfl(pre, (lane - o) & 63), ys = __shfl(suf, (lane + o) & 63);
        if (lane >= o) pre += yp;
        if (lane + o < 64) suf += ys;
      }
      if (lane < nvalid) {
        float* dgp = static_cast<float*>(const_cast<void*>(g.d_gate.ptr)) + n * g.d_gate.stride_b + h * g.d_gate.stride_h;
        dgp[int64_t(t0 + lane) * g.d_gate.stride_t] = suf + ex2(bend) * bs + (pre - ktr);
      }
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
  constexpr int dlocal_lds = DLocalLds<K>::BYTES;
  hipError_t e = configure_lds<&chunk_dlocal_kernel<VARIANT, K>>(dlocal_lds);
  if (e != hipSuccess) return e;
  if (nc == 0) return hipSuccess;
  const __bf16* states = reinterpret_cast<const __bf16*>(ws + Lw.states);
  __bf16* dstates = reinterpret_cast<__bf16*>(ws + Lw.dstates);
  const __bf16* ubuf = reinterpret_cast<const __bf16*>(ws + Lw.ubuf);
  __bf16* dubt = reinterpret_cast<__bf16*>(ws + Lw.dubt);
  const int xcd_map = (bh % 8 == 0) ? 1 : 0;
  auto dscan = [&](auto sl_c) -> hipError_t {
    constexpr int SL = decltype(sl_c)::value;
    constexpr int lds = 2 * (Rec<K>::FIX + kChunk * SL * 2);
    constexpr auto kernel = &chunk_dscan_kernel<VARIANT, K, SL>;
    const hipError_t err = configure_lds<kernel>(lds);
    if (err != hipSuccess) return err;
    const int n_slices = a.value_dim / SL;
    hipLaunchKernelGGL(kernel, dim3(bh * n_slices), dim3(dscan_threads<SL>()), lds, stream, a, g, n_slices, xcd_map,
                       nc, rec, ws + Lw.rec, dstates, dubt);
    return hipSuccess;
  };
  const int sl = scan_slice(bh, a.value_dim);
  e = sl == 64 ? dscan(std::integral_constant<int, 64>{})
               : sl == 32 ? dscan(std::integral_constant<int, 32>{}) : dscan(std::integral_constant<int, 16>{});
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((chunk_dlocal_kernel<VARIANT, K>), dim3(bh * nc), dim3(64 * DLocalLds<K>::NW), dlocal_lds,
                     stream, a, g, nc, states, dstates, ubuf, dubt);
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
  const int64_t chunks = int64_t(a.batch) * a.heads * nc, K = a.key_dim, V = a.value_dim;
  int64_t off = 0;
  auto take = [&](int64_t bytes) { const int64_t o = off; off += round256(bytes); return o; };
  L.rec = take(chunk_workspace_bytes(a));
  L.states = take(chunks * K * V * 2);
  L.dstates = take(chunks * K * V * 2);
  L.ubuf = take(chunks * kChunk * V * 2);
  L.dubt = take(chunks * kChunk * V * 2);
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
