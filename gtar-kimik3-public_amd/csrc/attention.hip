// Causal softmax attention (grouped-query, optional packed variable-length input) on gfx950 -- the attention layer
// of the hybrid stack (src/layers/attention.py:82-117, src/ops/flash_attention_2.py:24-151, forward only).
//
//   O[t] = sum_{s <= t} softmax_s(scale q_t . k_s) v_s       per (sequence, query head); key/value head h / (H / Hkv)
//
// One 256-thread workgroup owns 128 query rows of one (sequence, query head); wave w owns the two 16-row blocks
// 32 w + 16 b .. + 15 (b = 0, 1), so each K and V fragment it reads from LDS feeds both blocks' MFMAs (half the LDS
// traffic per FLOP of one block per wave).  Key/value tiles of 64 rows stream through double-buffered LDS (K and V
// rows XOR-swizzled by 16-byte chunk), loaded straight into LDS (no registers) while the current tile is used; two
// workgroups share a CU.  Per tile, wave and row block, on v_mfma_f32_16x16x32_{bf16,f16}:
//   * S^T = K Q^T  -- K rows from LDS as A, the wave's Q rows (registers for the whole call) as B, so each lane holds
//     16 scores of one query row (lane % 16) and the online-softmax statistics stay per lane;
//   * O^T += V^T P^T -- V^T through the transposing LDS read (ds_read_b64_tr_b16) as A, the bf16/f16 probabilities
//     straight from the score registers as B (the key order inside a 32-key step is the one the score tiles give;
//     the V^T read follows it), so O^T lands in the same per-query-row lane layout.
// Scores are exponentiated with v_exp_f32 in log2 units (the scale folded into one FMA); only tiles crossing the
// diagonal or the sequence end are masked.  The exponent base of a row moves only when a tile's max exceeds it by
// more than 2^8 (probabilities stay below 256, exact in bf16/f16 range), so the accumulators are rescaled on a few
// tiles only, and the row sums come out of the MFMA (all-ones A operand) from the same rounded probabilities as
// P V (uniform branches around VALU work; no MFMA sits under a data-dependent branch).  K tiles run one ahead of V
// tiles, so each tile's exponentials interleave with the next tile's score MFMAs in one basic block.
#include "attention_common.h"
#include "varlen_index.h"
#include "gdr_internal.h"

namespace gdr {
namespace {

using attn::cat;
using attn::Mma;
using attn::short4;
using chunk::kLog2e;
using chunk::lds_dma16;

constexpr int kBM = 128;  // query rows per workgroup
constexpr int kBN = attn::kTile;  // keys per LDS tile
constexpr int kAttnThreads = attn::kThreads;
constexpr int kRB = 2;  // 16-row query blocks per wave
constexpr float kNegInf = -__builtin_inff();
constexpr float kLazy = 8.f;  // log2 of the largest probability before the accumulators are rebased

template <int D, typename T>
__global__ __launch_bounds__(kAttnThreads, 2) void attention_fwd_kernel(const gdr_attention_args a, int nqb) {
  using M = Mma<T>;
  using V8 = typename M::v8;
  using V4 = typename M::v4;
  constexpr int DC = D / 8;         // 16-byte chunks per row
  constexpr int DS = D / 32;        // 32-wide k steps of S^T = K Q^T
  constexpr int DT = D / 16;        // 16-column tiles of O^T
  constexpr int TILE = kBN * D;     // elements per K or V tile
  constexpr int LOADS = kBN * DC / kAttnThreads;  // 16-byte pieces per thread per tile
  static_assert(LOADS >= 1 && kBN * DC % kAttnThreads == 0, "tile load split");
  extern __shared__ __align__(16) unsigned char smem[];
  T* ks = reinterpret_cast<T*>(smem);              // [2][kBN][D] swizzled
  T* vs = reinterpret_cast<T*>(smem) + 2 * TILE;   // [2][kBN][D] swizzled

  // ---- workgroup -> (sequence, query block, head); the latest query blocks (the most keys) are dispatched first ----
  const int H = a.heads;
  const int h = blockIdx.x % H, slot = blockIdx.x / H;
  int n, qb, bos = 0, len = a.seq_len;
  if (a.cu_seqlens) {  // query-block slots: floor(bos / kBM) + n is the first of sequence n (clamped offsets)
    n = packed_slot_seq(a.cu_seqlens, a.n_seqs, a.seq_len, kBM, slot);
    bos = packed_begin(a.cu_seqlens, n, a.seq_len);
    len = packed_end(a.cu_seqlens, n, a.seq_len) - bos;
    const int nb = (len + kBM - 1) / kBM;
    const int r = slot - packed_slot_base(a.cu_seqlens, n, a.seq_len, kBM);
    if (r < 0 || r >= nb) return;  // gap slot: uniform over the workgroup, before any barrier
    qb = nb - 1 - r;
  } else {
    n = slot / nqb;
    qb = nqb - 1 - slot % nqb;
  }
  const int bidx = a.cu_seqlens ? 0 : n;
  const int hk = h / (H / a.kv_heads);
  const T* qp = static_cast<const T*>(a.q.ptr) + bidx * a.q.stride_b + h * a.q.stride_h + int64_t(bos) * a.q.stride_t;
  const T* kp = static_cast<const T*>(a.k.ptr) + bidx * a.k.stride_b + hk * a.k.stride_h + int64_t(bos) * a.k.stride_t;
  const T* vp = static_cast<const T*>(a.v.ptr) + bidx * a.v.stride_b + hk * a.v.stride_h + int64_t(bos) * a.v.stride_t;
  T* op = static_cast<T*>(const_cast<void*>(a.out.ptr)) + bidx * a.out.stride_b + h * a.out.stride_h +
          int64_t(bos) * a.out.stride_t;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l16 = lane & 15, g4 = lane >> 4;
  const int q0 = qb * kBM;
  int qpos[kRB];  // this lane's query row of each block (position in the sequence)
  // Q rows as the B operand of S^T = K Q^T: lane (l16, g4) holds q[qpos[b]][32 ds + 8 g4 .. + 7].
  V8 qf[kRB][DS];
#pragma unroll
  for (int b = 0; b < kRB; ++b) {
    qpos[b] = q0 + 16 * (kRB * wave + b) + l16;
    const int qrow = min(qpos[b], len - 1);
#pragma unroll
    for (int ds = 0; ds < DS; ++ds)
      qf[b][ds] = *reinterpret_cast<const V8*>(qp + int64_t(qrow) * a.q.stride_t + 32 * ds + 8 * g4);
  }

  // ---- key/value tiles: global -> LDS directly (global_load_lds_dwordx4: a lane's 16 bytes land at the wave-
  // uniform LDS base + 16 * lane).  Row r, chunk c of a tile is stored at chunk c ^ (r mod DC), so each lane loads
  // the global chunk that belongs at its LDS slot.  K runs one tile ahead of V: the score MFMAs of tile kb + 1 are
  // issued beside the softmax of tile kb, which has no dependence on them. ----
  const int kend = min(len, q0 + kBM);  // keys this block can see
  const int nkb = (kend + kBN - 1) / kBN;
  constexpr int GROUPS = kBN * DC / kWave;  // 64-piece groups per K or V tile
  constexpr int kWaves = kAttnThreads / kWave;
  constexpr int GPW = GROUPS / kWaves;      // groups per wave per tile
  static_assert(GROUPS % kWaves == 0, "tile groups per wave");
  const int uwave = __builtin_amdgcn_readfirstlane(wave);
  int lrow[GPW], lcol[GPW];      // this lane's tile row and global 16-byte chunk, per group
  int64_t koffs[GPW], voffs[GPW];  // ... as element offsets from the tile's first key row
#pragma unroll
  for (int k = 0; k < GPW; ++k) {
    const int slot = kWave * (uwave + kWaves * k) + lane;
    lrow[k] = slot / DC;
    lcol[k] = (slot % DC) ^ (lrow[k] % DC);
    koffs[k] = int64_t(lrow[k]) * a.k.stride_t + 8 * lcol[k];
    voffs[k] = int64_t(lrow[k]) * a.v.stride_t + 8 * lcol[k];
  }
  // Rows past the sequence end (last tile only) read the last key row instead; the mask removes them.
  auto issue = [&](const T* base, int64_t stride, const int64_t (&offs)[GPW], T* tile, int kb) {
    const T* tb = base + int64_t(kb) * kBN * stride;
    const int lim = len - 1 - kb * kBN;
    if (lim >= kBN - 1) {
#pragma unroll
      for (int k = 0; k < GPW; ++k) lds_dma16(tb + offs[k], tile + kWave * 8 * (uwave + kWaves * k));
    } else {
#pragma unroll
      for (int k = 0; k < GPW; ++k)
        lds_dma16(tb + int64_t(min(lrow[k], lim)) * stride + 8 * lcol[k], tile + kWave * 8 * (uwave + kWaves * k));
    }
  };

  // This lane's LDS element offsets inside a tile: the K fragment of k step ds (row block 0), and the V^T fragment
  // of output column tile t (key rows 4 g4 + (l16 >> 2) + {0, 16, 32, 48}: the swizzle is the same for all four).
  int koff[DS], voff[DT];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) koff[ds] = l16 * D + (((4 * ds + g4) ^ (l16 % DC)) << 3);
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    const int col = 16 * t + 4 * (l16 & 3), r0 = 4 * g4 + (l16 >> 2);
    voff[t] = r0 * D + (((col >> 3) ^ (r0 % DC)) << 3) + (col & 7);
  }

  const float c = a.scale * kLog2e;  // scores in log2 units
  // Per lane and row block: m is the exponent base (log2 units) of the probabilities accumulated so far; it only
  // moves when a tile's row max exceeds it by more than kLazy, so every probability stays below 2^kLazy and the
  // accumulators are rescaled on a few tiles only.  lsum accumulates the row sums of the same bf16/f16
  // probabilities the P V products use (an all-ones A operand on the MFMA; every element of lsum[b] holds the sum).
  float m[kRB], mx[kRB];
  floatx4 o[kRB][DT], lsum[kRB];
#pragma unroll
  for (int b = 0; b < kRB; ++b) {
    m[b] = kNegInf;
    lsum[b] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < DT; ++t) o[b][t] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  V8 ones;
#pragma unroll
  for (int i = 0; i < 8; ++i) ones[i] = static_cast<T>(1.f);

  // S^T of the K tile at kt: lane holds S[qpos[b]][key0 + 16 t + 4 g4 + i]; each K fragment serves both row blocks.
  auto scores = [&](const T* kt, floatx4 (&s)[kRB][4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int b = 0; b < kRB; ++b) s[b][t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const V8 kf = *reinterpret_cast<const V8*>(kt + 16 * t * D + koff[ds]);
#pragma unroll
        for (int b = 0; b < kRB; ++b) s[b][t] = M::run(kf, qf[b][ds], s[b][t]);
      }
    }
  };
  // Only a tile that crosses this wave's diagonal or the sequence end needs the causal mask (a uniform branch).
  auto mask = [&](int kb, floatx4 (&s)[kRB][4]) {
    const bool full = (kb + 1) * kBN - 1 <= q0 + 32 * wave && (kb + 1) * kBN <= len;
    if (!full) {
#pragma unroll
      for (int b = 0; b < kRB; ++b)
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kb * kBN + 16 * t + 4 * g4 + i;
            if (!(key <= qpos[b] && key < len)) s[b][t][i] = kNegInf;
          }
    }
  };
  // Row max of one tile's raw scores, in log2 units.
  auto rowmax = [&](const floatx4 (&s)[kRB][4]) {
#pragma unroll
    for (int b = 0; b < kRB; ++b) {
      float x = kNegInf;  // the scale c > 0 is applied once, after the max
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) x = fmaxf(x, s[b][t][i]);
      x = xor_max(x, 16);
      x = xor_max(x, 32);
      mx[b] = x * c;
    }
  };
  // Moves the base of rows whose new max exceeds it by more than kLazy (a uniform branch per row block).
  auto rebase = [&]() {
#pragma unroll
    for (int b = 0; b < kRB; ++b) {
      const bool move = mx[b] > m[b] + kLazy;  // false while both are -inf (no visible key yet)
      if (__any(move)) {
        const float alpha = move ? __builtin_amdgcn_exp2f(m[b] - mx[b]) : 1.f;  // 0 from a base of -inf
        if (move) m[b] = mx[b];
#pragma unroll
        for (int i = 0; i < 4; ++i) lsum[b][i] *= alpha;
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[b][t][i] *= alpha;
      }
    }
  };
  // Probabilities 2^(c s - m) of one tile as bf16/f16 MFMA operands.
  auto probs = [&](floatx4 (&s)[kRB][4], V8 (&pf)[kRB][2]) {
#pragma unroll
    for (int b = 0; b < kRB; ++b) {
      const float base = m[b] == kNegInf ? 0.f : m[b];
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) s[b][t][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[b][t][i], c, -base));
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) pf[b][s2] = cat<V4, V8>(M::pack(s[b][2 * s2]), M::pack(s[b][2 * s2 + 1]));
    }
  };
  // O^T += V^T P^T for the V tile at LDS byte address vt: V^T rows 32 s2 + 4 g4 + r (and + 16), column 16 t + l16,
  // through the transposing read; each V^T fragment serves both row blocks.  Then the row sums.
  // The reads are issued as inline assembly, one column tile ahead of their MFMAs, with their own lgkmcnt waits:
  // the compiler cannot tell the transposing read from the key/value DMA still in flight into the other buffers,
  // and would otherwise wait for that DMA (vmcnt(0)) before the first read.  LDS operations complete in order, so
  // "lgkmcnt(4)" after the next tile's four reads covers this tile's reads whatever else the compiler interleaves.
  auto pv = [&](uint32_t vt, const V8 (&pf)[kRB][2]) {
    short4 x[2][4];
    auto rd = [&](int t, short4 (&r)[4]) { attn::tr_read4<D>(vt + 2 * voff[t], r); };
    rd(0, x[0]);
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      short4(&r)[4] = x[t & 1];
      if (t + 1 < DT) {
        rd(t + 1, x[(t + 1) & 1]);
        asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]));
      } else {
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]));
      }
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const V8 vf = cat<V4, V8>(__builtin_bit_cast(V4, r[2 * s2]), __builtin_bit_cast(V4, r[2 * s2 + 1]));
#pragma unroll
        for (int b = 0; b < kRB; ++b) o[b][t] = M::run(vf, pf[b][s2], o[b][t]);
      }
    }
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int b = 0; b < kRB; ++b) lsum[b] = M::run(ones, pf[b][s2], lsum[b]);
  };
  const uint32_t vlds = attn::lds_addr(vs);

  issue(kp, a.k.stride_t, koffs, ks, 0);
  issue(vp, a.v.stride_t, voffs, vs, 0);
  if (nkb > 1) issue(kp, a.k.stride_t, koffs, ks + TILE, 1);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  floatx4 s[kRB][4];
  scores(ks, s);
  mask(0, s);
  rowmax(s);
  rebase();
  __syncthreads();  // every wave has read K tile 0 before the first step refills its buffer
  // Step kb: the probabilities of tile kb beside the score MFMAs of tile kb + 1, the P V MFMAs of tile kb, then the
  // mask and row max of tile kb + 1 (one basic block up to the mask, so the VALU and MFMA work can interleave).
  int kb = 0;
  for (; kb + 1 < nkb; ++kb) {  // the accumulators start at zero right before this loop
    const int cur = kb & 1;
    // K tile kb (read in the previous step) and V tile kb - 1 are free
    if (kb + 2 < nkb) issue(kp, a.k.stride_t, koffs, ks + cur * TILE, kb + 2);
    issue(vp, a.v.stride_t, voffs, vs + (cur ^ 1) * TILE, kb + 1);
    V8 pf[kRB][2];
    probs(s, pf);
    scores(ks + (cur ^ 1) * TILE, s);
    // The P V MFMAs at raised priority: the other workgroup's wave on this SIMD fills the gaps with its VALU work
    // instead of interleaving with them (packed c5 1,141 -> 1,124 us, bit-identical; the score MFMAs at raised
    // priority as well, or alone, were slower).
    __builtin_amdgcn_s_setprio(1);
    pv(vlds + cur * TILE * 2, pf);
    __builtin_amdgcn_s_setprio(0);
    mask(kb + 1, s);
    rowmax(s);
    rebase();
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of K tile kb + 2 and V tile kb + 1 have landed
    __syncthreads();                 // ... everyone's, and every wave is done with K tile kb + 1 and V tile kb
  }
  {
    V8 pf[kRB][2];
    probs(s, pf);
    pv(vlds + (kb & 1) * TILE * 2, pf);
  }

  // The row log-sum-exp of the scaled scores in log2 units, m + log2(row sum): the backward's probabilities are
  // 2^(c s - lse), the same normalisation as the output's.
  if (a.lse && g4 == 0) {
    float* lp = a.lse + (int64_t(bidx) * H + h) * a.seq_len + bos;
#pragma unroll
    for (int b = 0; b < kRB; ++b)
      if (qpos[b] < len) lp[qpos[b]] = m[b] + __builtin_amdgcn_logf(lsum[b][0]);
  }
#pragma unroll
  for (int b = 0; b < kRB; ++b) {
    if (qpos[b] < len) {
      const float inv = 1.f / lsum[b][0];
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        floatx4 y = o[b][t];
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] *= inv;
        *reinterpret_cast<V4*>(op + int64_t(qpos[b]) * a.out.stride_t + 16 * t + 4 * g4) = M::pack(y);
      }
    }
  }
}

template <int D, typename T>
hipError_t launch_attention_typed(const gdr_attention_args& a, hipStream_t stream) {
  constexpr int lds = 4 * kBN * D * 2;  // K and V, double-buffered
  const hipError_t e = configure_lds<&attention_fwd_kernel<D, T>>(lds);
  if (e != hipSuccess) return e;
  const int nqb = (a.seq_len + kBM - 1) / kBM;
  const int64_t slots = a.cu_seqlens ? int64_t(nqb) + a.n_seqs : int64_t(a.batch) * nqb;
  if (slots * a.heads > 0)
    hipLaunchKernelGGL((attention_fwd_kernel<D, T>), dim3(unsigned(slots * a.heads)), dim3(kAttnThreads), lds, stream,
                       a, nqb);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_attention(const gdr_attention_args& a, hipStream_t stream) {
  if (a.q.dtype == GDR_BF16)
    return a.head_dim == 64 ? launch_attention_typed<64, __bf16>(a, stream) : launch_attention_typed<128, __bf16>(a, stream);
  return a.head_dim == 64 ? launch_attention_typed<64, _Float16>(a, stream)
                          : launch_attention_typed<128, _Float16>(a, stream);
}

}  // namespace gdr
