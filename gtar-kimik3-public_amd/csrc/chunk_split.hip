// Chunkwise (prefill) forward of the gated delta-rule family on gfx950 in two launches: a chunk-parallel
// preparation kernel and a sequential state-scan kernel, joined by a workspace in HBM.
//
// Reference: the forward of ChunkKimiDeltaAttention (src/ops/kimi_delta_attention.py:535-558) -- chunk_cumsum
// (utils.py:15-23), kernel matrices (:71-106), WY representation (:109-136), state scan (:139-170), output
// (:173-197) -- and its Gated DeltaNet / GLA / DeltaNet twins (gated_deltanet.py:62-162,
// gated_linear_attention.py:59-144, deltanet.py:60-149).
//
// Per chunk of C = 64 tokens with state S entering it (B = in-chunk inclusive cumsum of the log gate):
//   P = tril(K K^T (x) e^{B_t - B_s}, -1),   A = (I + diag(beta) P)^{-1}
//   W = A diag(beta) K e^B,   U = A diag(beta) V          (GLA: no W, U = V)
//   u = U - W S,   O = scale [(Q e^B) S + tril(Q K^T (x) e^{B_t - B_s}) u],   S' = diag(e^{B_end}) S + (K e^{B_end - B})^T u
//
// Everything that does not depend on S is chunk-local, so it runs in `chunk_prep_kernel` with one workgroup per
// (chunk, head): thousands of independent workgroups that fill all 256 CUs.  The prep kernel writes one record
// per (chunk, head) -- W, Q e^B, (K e^{B_end - B})^T, the ten gated score tiles, e^{B_end} and U^T -- laid out
// exactly as the scan kernel's LDS image, so the scan kernel stages a record with straight 16-byte copies.
// `chunk_scan_kernel` keeps the fp32 state of one (sequence, head) x 64-column slice in the registers of four
// compute waves for the whole sequence and per chunk runs only MFMA work: X = W S and Q e^B S (bf16, 32-deep),
// u = U - X, the intra-chunk output Sc u and the state update; four loader waves stream the next chunk's record
// into the other half of a double-buffered LDS region meanwhile.  The per-chunk critical path has no triangular
// solve and no transcendental: those are all in the prep kernel.
//
// Numerics of the prep kernel: decay factors are anchored per 16-row block so that every factor folded into a
// bf16 MFMA operand of the gated K K^T / Q K^T strips is <= 1, except the diagonal-tile key factor e^{-T_i},
// which is bounded by the block's own decay span; channels whose span exceeds kHotSpan are evaluated exactly
// elementwise instead (the reference evaluates diagonal blocks elementwise, utils.py:48-53).  The diagonal
// 16x16 blocks of (I + diag(beta) P) are inverted in fp32; W and U come out of a blocked forward substitution on
// v_mfma_f32_16x16x16_bf16 with fp32 accumulation.  W, U, Q e^B and K e^{B_end - B} are stored as bf16, as the
// reference stores W, U and u.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "chunk_common.h"
#include "gdr_internal.h"
#include "split_common.h"

namespace gdr {

using namespace chunk;

namespace {

// A compile-time int passed to a generic lambda.
template <int N>
struct IntC {
  static constexpr int value = N;
};

// What the state scan writes (chunk_scan_kernel's kMode).
constexpr int kScanOut = 0, kScanStates = 1, kScanBoth = 2;

// LDS of the prep kernel (bytes); 3 workgroups fit a CU for K = 128.
template <int K>
struct PrepLds {
  static constexpr int KP = K + 8;
  static constexpr int KAP = 0;                   // bf16 [64][KP] k e^{a_p - b}  (block-end anchor, strip keys)
  static constexpr int VST = KAP;                 //   after the strips: bf16 [64][KP] one K-column pass of V
  static constexpr int KD = KAP + 64 * KP * 2;    // bf16 [64][KP] k e^B         (right-hand side of the solve)
  static constexpr int SC = KD + 64 * KP * 2;     // bf16 [10][256] gated score tiles
  static constexpr int EPRE = SC;                 //   before the strips: fp32 [4][K] e^{a_{i-1}} per block
  static constexpr int ETAIL = SC + 4 * K * 4;    //   before the strips: fp32 [4][K] e^{B_end - a_i} per block
  static constexpr int NEGL = SC + 10 * 512;      // bf16 [6][256]  -diag(beta) P, tile (i, j < i)
  static constexpr int LII = NEGL + 6 * 512;      // fp32 [4][256]  diag(beta) P_ii (strictly lower)
  static constexpr int TOT = LII + 4 * 1024;      // fp32 [4][K]    per-block log2-gate totals
  static constexpr int AINV = TOT;                //   after the strips: bf16 [4][256] (I + diag(beta) P_ii)^{-1}
  static constexpr int RDS = TOT + 4 * K * 4;     // fp32 [4][K]    diagonal key factor e^{-T_i} (0: hot channel)
  static constexpr int FAR = RDS + 4 * K * 4;     // fp32 [3][K]    key factors of tiles (2,0), (3,0), (3,1)
  static constexpr int BETA = FAR + 3 * K * 4;    // fp32 [64]
  static constexpr int NRM = BETA + 256;          // fp32 [2][64]   fused prologue: 1 / ||q||, 1 / ||k|| per row
  static constexpr int BYTES = NRM + 512;
  static_assert(8 * K * 4 <= 16 * 512, "EPRE/ETAIL alias");
  static_assert(SC + 64 * K * 2 <= FAR, "fused prologue: the z staging block [64][K] fits in SC .. RDS");
  static_assert(4 * 512 <= 11 * K * 4, "AINV alias");
};

// softplus(x) = max(x, 0) + log1p(e^{-|x|}) in fp32, with two transcendental instructions.  log1p(y), y in (0, 1]:
// for y > 2^-6 as log(1 + y), whose rounding of 1 + y (2^-24 absolute) is below 2^-18 of the result; below that as
// the series y - y^2/2 + y^3/3 - y^4/4 + y^5/5, whose truncation is below y^5/6 < 2^-32 of the result.
__device__ __forceinline__ float softplus_f32(float x) {
  const float y = __builtin_amdgcn_exp2f(-fabsf(x) * kLog2e);
  const float series = y * (1.f - y * (0.5f - y * (1.f / 3.f - y * (0.25f - y * 0.2f))));
  const float l1p = y > 0x1p-6f ? __builtin_amdgcn_logf(1.f + y) * kLn2 : series;
  return fmaxf(x, 0.f) + l1p;
}

// The fused prologue's short convolution (ShortConvolution, src/layers/short_convolution.py:11-20) of width W:
// silu(sum_{j < W} w[c][j] x[t - W + 1 + j][c]) for 8 consecutive channels at the 4 sequence rows r0 .. r0 + 3,
// accumulated in fp32 and rounded once to bf16 (as gdr_short_conv_fwd).  The W + 3 input rows r0 - W + 1 .. r0 + 3
// are loaded once; rows before the sequence come from its conv state [C][W - 1] (`st8` points at the first of the 8
// channels' rows) or are zero, and rows past `last` (the sequence's last row) read row `last` (their outputs are
// masked by the caller).  `x0` is row 0 of the sequence at the first channel, `w8` the 8 channels' weight rows
// ([8][W], 16 W contiguous bytes).
template <int W>
__device__ __forceinline__ void conv_silu8x4(const __bf16* x0, int64_t x_st, int r0, int last, const __bf16* w8,
                                             const __bf16* st8, uint4 (&out)[4]) {
  uint32_t w[4 * W];  // packed bf16 pairs: weight (e, j) is bf16 number W e + j
#pragma unroll
  for (int u = 0; u < W; ++u) {
    const uint4 wu = *reinterpret_cast<const uint4*>(w8 + 8 * u);
    w[4 * u] = wu.x, w[4 * u + 1] = wu.y, w[4 * u + 2] = wu.z, w[4 * u + 3] = wu.w;
  }
  auto wf = [&](int m) {  // bf16 number m as fp32
    const uint32_t word = w[m >> 1];
    return __uint_as_float((m & 1) ? (word & 0xffff0000u) : (word << 16));
  };
  uint4 xr[W + 3];
#pragma unroll
  for (int m = 0; m < W + 3; ++m) {
    const int r = r0 - (W - 1) + m;
    if (r >= 0) {
      xr[m] = *reinterpret_cast<const uint4*>(x0 + int64_t(min(r, last)) * x_st);
    } else {
      bf16x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = st8 ? st8[(W - 1) * e + (W - 1) + r] : bf(0.f);
      xr[m] = __builtin_bit_cast(uint4, v);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < W; ++j) {
      float xv[8];
      unpack8(xr[i + j], xv);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += wf(W * e + j) * xv[e];
    }
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = bf(silu_rcp(acc[e]));
    out[i] = __builtin_bit_cast(uint4, o);
  }
}

// The same for one channel (the hot-channel re-fetch), returned as the bf16-rounded value.
template <int W>
__device__ __forceinline__ float conv_silu1(const __bf16* x0, int64_t x_st, int t, const __bf16* ww,
                                           const __bf16* st) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < W; ++j) {
    const int r = t - (W - 1) + j;
    const float xv = r >= 0 ? f32(x0[int64_t(r) * x_st]) : (st ? f32(st[(W - 1) + r]) : 0.f);
    acc += f32(ww[j]) * xv;
  }
  return f32(bf(silu_rcp(acc)));
}

// Calls f(IntC<W>{}) for a convolution width known at run time (2 to 8, uniform over the workgroup; validated by
// the API): one instantiation of the convolution per width.
template <typename F>
__device__ __forceinline__ void with_conv_width(int width, const F& f) {
  switch (width) {
    case 2: f(IntC<2>{}); break;
    case 3: f(IntC<3>{}); break;
    case 4: f(IntC<4>{}); break;
    case 5: f(IntC<5>{}); break;
    case 6: f(IntC<6>{}); break;
    case 7: f(IntC<7>{}); break;
    default: f(IntC<8>{}); break;
  }
}

// The low-rank gate of the fused prologue for the chunk's 64 rows:
//   g[t][c] = -e^{A_log[h]} softplus(z_t . W[h K + c] + bias[h K + c])
// Wave w computes channels [w K / 4, (w + 1) K / 4) of all 64 rows as Gᵀ = W_h Zᵀ on v_mfma_f32_16x16x32_bf16 (A = 16
// channels x 32 of R from W's rows, B = 32 of R x 16 tokens from z's rows), so each wave reads only its quarter of W.
// z goes through LDS once per workgroup, K of R at a time (`zs`, [64][K] bf16, 16-byte chunk c of row r stored at
// chunk c ^ (r mod K / 8), copied with global_load_lds_dwordx4: the permutation is applied to the source addresses,
// since the copy lands lane i at base + 16 i).  Lane (l16, g4) ends with channels 16 t + 4 g4 + i of token 16 j + l16;
// the values go to the fp32 LDS rows `gst` (row pitch K + 4), from which every lane later reads its own row.
// s_waitcnt vmcnt(N) and the workgroup barrier, tied to the low-rank gate's W fragments and bias (loaded by inline
// assembly, so the compiler does not track them): no instruction reading them can be scheduled before the wait.
template <int N, int CT, int S>
__device__ __forceinline__ void wait_tied(bf16x8 (&wa)[CT][S], floatx4 (&bias)[CT]) {
  static_assert(CT * S == 8 || CT * S == 2, "every W fragment is tied");
  if constexpr (CT * S == 8)
    asm volatile("s_waitcnt vmcnt(%10)\n\ts_barrier"
                 : "+v"(wa[0][0]), "+v"(wa[0][1]), "+v"(wa[0][2]), "+v"(wa[0][3]), "+v"(wa[CT - 1][0]),
                   "+v"(wa[CT - 1][1]), "+v"(wa[CT - 1][2]), "+v"(wa[CT - 1][3]), "+v"(bias[0]), "+v"(bias[CT - 1])
                 : "n"(N)
                 : "memory");
  else
    asm volatile("s_waitcnt vmcnt(%3)\n\ts_barrier"
                 : "+v"(wa[0][0]), "+v"(wa[0][S - 1]), "+v"(bias[0])
                 : "n"(N)
                 : "memory");
}

// `after_first_block()` issues the caller's own row loads (kAfterLoads vector loads per lane) right behind the first
// block's W and z requests.  One counted wait, vmcnt(kAfterLoads), then lets the block's products start while those
// row loads are still in flight, so their latency overlaps the gate instead of following it.  For that count to hold:
//   * the W fragments and the bias are loaded by inline assembly, and the z fragments are read from LDS by inline
//     assembly: the compiler does not see them as loads, so it does not put a wait of its own (a vmcnt(0) behind the
//     z copies, whose LDS writes it cannot tell apart from these reads) in front of the products;
//   * the counted wait is tied ("+v") to every W fragment and bias register, so no instruction reading them can be
//     scheduled before it, and it carries the workgroup barrier after which every wave's z copies have landed;
//   * scheduling barriers keep the row loads behind the copies (vector memory requests complete in issue order).
template <int K, int kAfterLoads, typename AfterFirstBlock>
__device__ __forceinline__ void lowrank_gate_rows(const gdr_prologue& pro, int h, const __bf16* zchunk, int64_t z_st,
                                                  int last_row, float* gst, __bf16* zs, int wave, int l16, int g4,
                                                  const AfterFirstBlock& after_first_block) {
  constexpr int CT = K / 64;          // 16-channel tiles per wave
  constexpr int RB = K, C16 = RB / 8;  // R per LDS block, 16-byte chunks per staged row
  const int R = pro.rank, ch0 = wave * (K / 4), lane = threadIdx.x & 63;
  const __bf16* w = static_cast<const __bf16*>(pro.gate_weight) + (size_t(h) * K + ch0 + l16) * R + 8 * g4;
  floatx4 acc[CT][4];
#pragma unroll
  for (int t = 0; t < CT; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[t][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  // A_log and the bias are requested first, and each block's W fragments before its z rows: one wait then covers
  // every load of a block, instead of a memory round trip per dependent fragment.
  const float a_log_h = pro.a_log[h];
  floatx4 bias[CT];
  const float* bias_p = pro.gate_bias ? pro.gate_bias + size_t(h) * K + ch0 + 4 * g4 : nullptr;
#pragma unroll
  for (int t = 0; t < CT; ++t) {
    bias[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (bias_p) asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(bias[t]) : "v"(bias_p + 16 * t));
  }
  for (int r0 = 0; r0 < R; r0 += RB) {  // the accumulators start at zero right before this loop
    bf16x8 wa[CT][RB / 32];
#pragma unroll
    for (int t = 0; t < CT; ++t)
#pragma unroll
      for (int s = 0; s < RB / 32; ++s)
        asm volatile("global_load_dwordx4 %0, %1, off"
                     : "=v"(wa[t][s])
                     : "v"(w + size_t(16 * t) * R + min(r0 + 32 * s, R - 32)));
    // stage z[0:64][r0 : r0 + RB] (columns past R read column R - 8 and meet zero z operands below)
#pragma unroll
    for (int k = 0; k < 64 * C16 / 256; ++k) {
      const int slot = 64 * (4 * k + wave) + lane;  // LDS chunk index: row slot / C16, chunk slot % C16
      const int row = slot / C16, c = (slot % C16) ^ (row % C16);
      const int col = min(r0 + 8 * c, R - 8);
      lds_dma16(zchunk + int64_t(min(row, last_row)) * z_st + col, zs + 8 * 64 * (4 * k + wave));
    }
    // Wait for this block's W, bias and z (the caller's row loads, issued after them, may stay in flight), then
    // the barrier: every wave's z copies have landed.
    if (r0 == 0) {
      __builtin_amdgcn_sched_barrier(0);
      after_first_block();
      __builtin_amdgcn_sched_barrier(0);
      wait_tied<kAfterLoads>(wa, bias);
    } else {
      wait_tied<0>(wa, bias);
    }
#pragma unroll
    for (int s = 0; s < RB / 32; ++s) {
      const bool live = r0 + 32 * s < R;
      bf16x8 zb[4];  // rows 16 j + l16 of zs, columns r0 + 32 s + 8 g4 .. + 7 (the four rows share the swizzle)
      const int c = (4 * s + g4) ^ (l16 % C16);
      const uint32_t za = static_cast<uint32_t>(
          (uintptr_t)(__attribute__((address_space(3))) const __bf16*)(zs + l16 * RB + 8 * c));
      asm volatile(
          "ds_read_b128 %0, %4\n\t"
          "ds_read_b128 %1, %4 offset:%5\n\t"
          "ds_read_b128 %2, %4 offset:%6\n\t"
          "ds_read_b128 %3, %4 offset:%7\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(zb[0]), "=&v"(zb[1]), "=&v"(zb[2]), "=&v"(zb[3])
          : "v"(za), "n"(2 * 16 * RB), "n"(2 * 32 * RB), "n"(2 * 48 * RB));
#pragma unroll
      for (int j = 0; j < 4; ++j) zb[j] = live ? zb[j] : bf16x8{};
#pragma unroll
      for (int t = 0; t < CT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[t][j] = mfma32(wa[t][s], zb[j], acc[t][j]);
    }
    lds_barrier();  // every wave is done with this block of zs
  }
  const float neg_a = -__builtin_amdgcn_exp2f(a_log_h * kLog2e);
#pragma unroll
  for (int t = 0; t < CT; ++t) {
    const int ch = ch0 + 16 * t + 4 * g4;
    const float4 bias_t = make_float4(bias[t][0], bias[t][1], bias[t][2], bias[t][3]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 g = make_float4(
          neg_a * softplus_f32(acc[t][j][0] + bias_t.x), neg_a * softplus_f32(acc[t][j][1] + bias_t.y),
          neg_a * softplus_f32(acc[t][j][2] + bias_t.z), neg_a * softplus_f32(acc[t][j][3] + bias_t.w));
      *reinterpret_cast<float4*>(gst + (16 * j + l16) * (K + 4) + ch) = g;
    }
  }
}

// ======================================= prep: one workgroup per (chunk, head) =======================================
// 16 bytes of an input row that only this workgroup reads: with the non-temporal hint when kNT.
template <int kNT, typename R>
__device__ __forceinline__ R input16(const void* p) {
  if constexpr (kNT) return load_nt16<R>(p);
  else return *static_cast<const R*>(p);
}

// kPro: the fused layer prologue.  0: none (the plain op); 1: `pro.flags` selects the in-kernel q / k
// normalisation and the beta sigmoid; 2: as 1, and the per-channel gate comes from the low-rank projection; plus 4:
// the short convolutions of q, k, v (width 4) run in the kernel too; plus 16 as well: their width is the call's
// `pro.conv_size` (2 to 8), one code path per width behind a uniform switch.  Three workgroups fit a CU's LDS; the
// f16 build, whose diagonal strip tile carries extra bf16 operands, and the any-width convolution, whose widest
// path holds 11 input rows and 8 weight rows per thread, are held to two so that they do not spill.  kNT (plain
// op only): the q, k, gate and V rows are loaded with the non-temporal hint (`use_nt_hint` below decides).
template <int VARIANT, int K, int kPro = 0, int kNT = 0, typename T = __bf16>
__global__ __launch_bounds__(256, (__is_same(T, _Float16) || (kPro & 16)) ? 2 : 3) void chunk_prep_kernel(const gdr_args a, int nc,
                                                                                         int64_t rec_bytes,
                                                                                         const gdr_prologue pro) {
  constexpr bool kLowRank = (kPro & 3) == 2;
  constexpr bool kConv = (kPro & 4) != 0;
  constexpr bool kAnyWidth = (kPro & 16) != 0;  // the convolution's width comes from the call (2 to 8), else 4
  static_assert(!kLowRank || VARIANT == GDR_KDA || VARIANT == GDR_GLA, "low-rank gate: per-channel variants");
  static_assert(kPro == 0 || __is_same(T, __bf16), "the fused prologue reads bf16 inputs");
  using V8 = vec8<T>;
  using V4 = vec4<T>;
  constexpr bool kDelta = VARIANT != GDR_GLA;
  constexpr int kGate = (VARIANT == GDR_KDA || VARIANT == GDR_GLA) ? 2 : (VARIANT == GDR_GDN ? 1 : 0);
  constexpr int KS = K / 32;
  using L = PrepLds<K>;
  using R = Rec<K>;
  constexpr int KP = L::KP;
  constexpr float kHot = kHotSpan * kLog2e;  // hot threshold on -T in log2 units
  extern __shared__ __align__(16) unsigned char smem[];

  // ---- workgroup -> (sequence n, head h, chunk c) ----
  const int H = a.heads;
  const int h = blockIdx.x % H;
  int slot = blockIdx.x / H, n, c, bos = 0, len = a.seq_len;
  if (a.cu_seqlens) {
    n = packed_slot_seq(a.cu_seqlens, a.n_seqs, a.seq_len, kChunk, slot);
    bos = packed_begin(a.cu_seqlens, n, a.seq_len);
    len = packed_end(a.cu_seqlens, n, a.seq_len) - bos;
    c = slot - varlen_base(a.cu_seqlens, n, a.seq_len);
    if (c < 0 || c * kChunk >= len) return;  // gap slot: uniform over the workgroup, before any barrier
  } else {
    // Launch order is chunk-major from the last chunk down: the records written last are the first chunks, which
    // the scan reads first, so they are the ones still held by the memory-side cache when it starts.
    n = slot % a.batch;
    c = nc - 1 - slot / a.batch;
    slot = n * nc + c;
  }
  const int bidx = a.cu_seqlens ? 0 : n;
  ChunkCtxT<T> x;
  x.q_st = a.q.stride_t; x.k_st = a.k.stride_t; x.v_st = a.v.stride_t; x.o_st = 0;
  x.g_st = a.gate.stride_t; x.b_st = a.beta.stride_t;
  x.qp = static_cast<const T*>(a.q.ptr) + bidx * a.q.stride_b + h * a.q.stride_h + bos * x.q_st;
  x.kp = static_cast<const T*>(a.k.ptr) + bidx * a.k.stride_b + h * a.k.stride_h + bos * x.k_st;
  x.vp = static_cast<const T*>(a.v.ptr) + bidx * a.v.stride_b + h * a.v.stride_h + bos * x.v_st;
  x.gp = kGate ? static_cast<const float*>(a.gate.ptr) + bidx * a.gate.stride_b + h * a.gate.stride_h + bos * x.g_st
               : nullptr;
  x.betap = kDelta ? static_cast<const float*>(a.beta.ptr) + bidx * a.beta.stride_b + h * a.beta.stride_h +
                         bos * x.b_st
                   : nullptr;
  x.op = nullptr;
  x.len = len;
  x.nchunks = 0; x.v0 = 0; x.V = a.value_dim; x.sbase = 0; x.h0 = nullptr; x.ht = nullptr; x.scale = 0.f;
  unsigned char* rec = static_cast<unsigned char*>(a.workspace) + (int64_t(slot) * H + h) * rec_bytes;
  // fused prologue: in-kernel short convolutions of q, k, v (channels h K + ch of [H K] for q, k; h V + col for v)
  constexpr bool conv = kConv;
  const int64_t ck = int64_t(H) * K, cvv = int64_t(H) * a.value_dim;
  const int cw = kAnyWidth ? pro.conv_size : 4;  // convolution width W
  const __bf16* cwq = static_cast<const __bf16*>(pro.conv_weight[0]) + (int64_t(h) * K) * cw;
  const __bf16* cwk = static_cast<const __bf16*>(pro.conv_weight[1]) + (int64_t(h) * K) * cw;
  const __bf16* cwv = static_cast<const __bf16*>(pro.conv_weight[2]) + (int64_t(h) * a.value_dim) * cw;
  auto state_rows = [&](int i, int64_t nch, int64_t ch0) -> const __bf16* {  // [C][W - 1] rows of this sequence
    const __bf16* st = static_cast<const __bf16*>(pro.conv_state_in[i]);
    return st ? st + (int64_t(n) * nch + ch0) * (cw - 1) : nullptr;
  };
  // 8 channels x 4 rows of the convolution at the call's width.  Inlined by force: as a called function its output
  // array went through scratch memory.
  auto conv8x4 = [&](const __bf16* x0, int64_t x_st, int r0, const __bf16* w8, const __bf16* st8,
                     uint4 (&o)[4]) __attribute__((always_inline)) {
    if constexpr (kAnyWidth)
      with_conv_width(cw, [&](auto wc) __attribute__((always_inline)) {
        conv_silu8x4<decltype(wc)::value>(x0, x_st, r0, len - 1, w8, st8, o);
      });
    else
      conv_silu8x4<4>(x0, x_st, r0, len - 1, w8, st8, o);
  };
  auto conv1 = [&](const __bf16* x0, int64_t x_st, int t, const __bf16* ww, const __bf16* st)
                   __attribute__((always_inline)) {
    float r = 0.f;
    if constexpr (kAnyWidth)
      with_conv_width(cw, [&](auto wc) __attribute__((always_inline)) {
        r = conv_silu1<decltype(wc)::value>(x0, x_st, t, ww, st);
      });
    else
      r = conv_silu1<4>(x0, x_st, t, ww, st);
    return r;
  };

  T* kap = reinterpret_cast<T*>(smem + L::KAP);
  T* vst = reinterpret_cast<T*>(smem + L::VST);
  T* ainv = reinterpret_cast<T*>(smem + L::AINV);
  T* kd = reinterpret_cast<T*>(smem + L::KD);
  T* sct = reinterpret_cast<T*>(smem + L::SC);
  float* epre_v = reinterpret_cast<float*>(smem + L::EPRE);
  float* etail_v = reinterpret_cast<float*>(smem + L::ETAIL);
  T* negl = reinterpret_cast<T*>(smem + L::NEGL);
  float* lii = reinterpret_cast<float*>(smem + L::LII);
  float* tot = reinterpret_cast<float*>(smem + L::TOT);
  float* rds = reinterpret_cast<float*>(smem + L::RDS);
  float* far = reinterpret_cast<float*>(smem + L::FAR);
  float* sbeta = reinterpret_cast<float*>(smem + L::BETA);
  float* snorm = reinterpret_cast<float*>(smem + L::NRM);

  // A-operand lane layout: lane (l16, g4) of wave p holds row 16 p + l16, channels 32 kk + 8 g4 + j.
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l16 = lane & 15, g4 = lane >> 4;
  const int p = wave;
  const int crow = c * kChunk + 16 * p + l16;  // token index within the sequence
  const bool valid = crow < len;
  const int tc = min(crow, len - 1);

  // V is consumed in passes of K columns staged row-major in LDS (the strip-key region, free by then).
  constexpr int kVPieces = 64 * K / 8;                 // 16-byte pieces of a full pass
  constexpr int kVLoads = (kVPieces + 255) / 256;      // per thread
  const int n_pass = (a.value_dim + K - 1) / K;
  auto pass_width = [&](int pass) { return min(K, a.value_dim - pass * K); };
  // With the in-kernel convolution, thread u (< 16 w8) holds rows 4 (u / w8) .. + 3 of column group u % w8 (the four
  // rows share their input window); otherwise piece i of a thread is 16-byte piece threadIdx.x + 256 i of the pass.
  constexpr int kVRegs = kConv ? 4 : kVLoads;
  static_assert(!kConv || 16 * K / 8 <= 256, "conv mapping: one row quad per thread");
  uint4 vpre[kVRegs];
  auto load_v_pass = [&](int pass) {  // unconditional loads from clamped rows / pieces; masked when staged
    const int w8 = pass_width(pass) / 8;
    if constexpr (kConv) {
      const int u = min(int(threadIdx.x), 16 * w8 - 1);
      const int col = pass * K + (u % w8) * 8;
      conv8x4(x.vp + col, x.v_st, c * kChunk + 4 * (u / w8), cwv + col * cw,
                    state_rows(2, cvv, int64_t(h) * a.value_dim + col), vpre);
    } else {
#pragma unroll
      for (int i = 0; i < kVLoads; ++i) {
        const int pc = min(int(threadIdx.x) + 256 * i, 64 * w8 - 1);
        const int row = pc / w8, cc = (pc % w8) * 8;
        const int t = min(c * kChunk + row, len - 1);
        vpre[i] = input16<kNT, uint4>(x.vp + t * x.v_st + pass * K + cc);
      }
    }
  };
  auto stage_v_pass = [&](int pass) {
    const int w8 = pass_width(pass) / 8;
#pragma unroll
    for (int i = 0; i < kVRegs; ++i) {
      const int pc = threadIdx.x + 256 * i;
      const int u = threadIdx.x;
      const bool have = kConv ? u < 16 * w8 : pc < 64 * w8;
      if (have) {
        const int row = kConv ? 4 * (u / w8) + i : pc / w8, cc = kConv ? (u % w8) * 8 : (pc % w8) * 8;
        const uint32_t keep = c * kChunk + row < len ? 0xffffffffu : 0u;
        *reinterpret_cast<uint4*>(vst + row * KP + cc) =
            make_uint4(vpre[i].x & keep, vpre[i].y & keep, vpre[i].z & keep, vpre[i].w & keep);
      }
    }
  };

  // ---- 1. loads: this lane's q, k, gate, beta row; the first pass of V ----
  // With a scalar gate (or none) the waves issue these loads at raised priority, so a new workgroup's requests go
  // out ahead of the arithmetic of the other workgroups on its SIMDs (c4 GDN 246 -> 241.5 us per call, DeltaNet
  // 236 -> 233.5 us, bit-identical); with a per-channel gate it made the call 1-2 us slower.
  constexpr bool kLoadPriority = kGate != 2;
  if constexpr (kLoadPriority) __builtin_amdgcn_s_setprio(3);
  uint4 qraw[KS], kraw[KS];
  float bl[KS][8];
  if constexpr (kLowRank) {
    // The gate rows are computed into the KAP / KD region, which nothing uses before step 3b (after two barriers).
    const __bf16* zchunk = static_cast<const __bf16*>(pro.gate_lowrank.ptr) + bidx * pro.gate_lowrank.stride_b +
                           int64_t(bos + c * kChunk) * pro.gate_lowrank.stride_t;
    auto issue_rows = [&]() {  // without the in-kernel convolution: this lane's q, k rows (kAfterLoads = 2 KS loads)
      if constexpr (!kConv) {
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
          const int ch = 32 * kk + 8 * g4;
          qraw[kk] = *reinterpret_cast<const uint4*>(x.qp + tc * x.q_st + ch);
          kraw[kk] = *reinterpret_cast<const uint4*>(x.kp + tc * x.k_st + ch);
        }
      }
    };
    lowrank_gate_rows<K, kConv ? 0 : 2 * KS>(pro, h, zchunk, pro.gate_lowrank.stride_t, len - 1 - c * kChunk,
                         reinterpret_cast<float*>(smem), reinterpret_cast<__bf16*>(smem + L::SC), wave, l16, g4,
                         issue_rows);
    lds_barrier();
  }
  if constexpr (kConv) {
    // The convolved q, k rows are staged in the KAP / KD tiles (bf16 [64][KP]; free until step 3b): unit u covers
    // rows 4 (u / (K / 8)) .. + 3 of channel group u % (K / 8) of tensor u / (16 K / 8).  Low-rank gate rows, which
    // occupy the same region, are read first.
    if constexpr (kLowRank) {
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const float* gr = reinterpret_cast<const float*>(smem) + (16 * p + l16) * (K + 4) + 32 * kk + 8 * g4;
        const float4 g0 = *reinterpret_cast<const float4*>(gr);
        const float4 g1 = *reinterpret_cast<const float4*>(gr + 4);
        bl[kk][0] = g0.x; bl[kk][1] = g0.y; bl[kk][2] = g0.z; bl[kk][3] = g0.w;
        bl[kk][4] = g1.x; bl[kk][5] = g1.y; bl[kk][6] = g1.z; bl[kk][7] = g1.w;
      }
      __syncthreads();
    }
    constexpr int G8 = K / 8, kUnits = 2 * 16 * G8;
#pragma unroll
    for (int u0 = 0; u0 < kUnits; u0 += 256) {
      const int u = u0 + threadIdx.x;
      if (u < kUnits) {
        const int tsr = u / (16 * G8), rq = (u / G8) % 16, ch = (u % G8) * 8;
        uint4 o[4];
        conv8x4((tsr ? x.kp : x.qp) + ch, tsr ? x.k_st : x.q_st, c * kChunk + 4 * rq, (tsr ? cwk : cwq) + ch * cw,
                state_rows(tsr, ck, int64_t(h) * K + ch), o);
        T* tile = tsr ? kd : kap;
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(tile + (4 * rq + i) * KP + ch) = o[i];
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    const int ch = 32 * kk + 8 * g4;
    if constexpr (kConv) {
      qraw[kk] = *reinterpret_cast<const uint4*>(kap + (16 * p + l16) * KP + ch);
      kraw[kk] = *reinterpret_cast<const uint4*>(kd + (16 * p + l16) * KP + ch);
    } else if constexpr (!kLowRank) {  // (with the low-rank gate they were requested during its products)
      qraw[kk] = input16<kNT, uint4>(x.qp + tc * x.q_st + ch);
      kraw[kk] = input16<kNT, uint4>(x.kp + tc * x.k_st + ch);
    }
    if constexpr (kLowRank && kConv) {
      // bl was read before the conv stage
    } else if constexpr (kLowRank) {
      const float* gr = reinterpret_cast<const float*>(smem) + (16 * p + l16) * (K + 4) + ch;
      const float4 g0 = *reinterpret_cast<const float4*>(gr);
      const float4 g1 = *reinterpret_cast<const float4*>(gr + 4);
      bl[kk][0] = g0.x; bl[kk][1] = g0.y; bl[kk][2] = g0.z; bl[kk][3] = g0.w;
      bl[kk][4] = g1.x; bl[kk][5] = g1.y; bl[kk][6] = g1.z; bl[kk][7] = g1.w;
    } else if constexpr (kGate == 2) {
      const float4 g0 = input16<kNT, float4>(x.gp + tc * x.g_st + ch);
      const float4 g1 = input16<kNT, float4>(x.gp + tc * x.g_st + ch + 4);
      bl[kk][0] = g0.x; bl[kk][1] = g0.y; bl[kk][2] = g0.z; bl[kk][3] = g0.w;
      bl[kk][4] = g1.x; bl[kk][5] = g1.y; bl[kk][6] = g1.z; bl[kk][7] = g1.w;
    }
  }
  if constexpr (kGate == 1) {
    const float g = x.gp[tc * x.g_st];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
#pragma unroll
      for (int j = 0; j < 8; ++j) bl[kk][j] = g;
  }
  if constexpr (kGate == 0) {
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
#pragma unroll
      for (int j = 0; j < 8; ++j) bl[kk][j] = 0.f;
  }
  float beta_t = kDelta ? x.betap[tc * x.b_st] : 0.f;
  if (kPro && kDelta && (pro.flags & GDR_PRO_BETA_LOGITS))
    beta_t = 1.f / (1.f + __builtin_amdgcn_exp2f(-beta_t * kLog2e));
  if (kPro && (pro.flags & GDR_PRO_NORM_QK)) {  // F.normalize over the K channels of this row (spread over the 4 lanes g4)
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      float qf[8], kf[8];
      unpack8<T>(qraw[kk], qf);
      unpack8<T>(kraw[kk], kf);
#pragma unroll
      for (int j = 0; j < 8; ++j) sq += qf[j] * qf[j], sk += kf[j] * kf[j];
    }
    sq = xor_sum(sq, 16);
    sk = xor_sum(sk, 16);
    sq = xor_sum(sq, 32);
    sk = xor_sum(sk, 32);
    const float iq = 1.f / fmaxf(sqrtf(sq), 1e-12f), ik = 1.f / fmaxf(sqrtf(sk), 1e-12f);
    if (g4 == 0) snorm[16 * p + l16] = iq, snorm[64 + 16 * p + l16] = ik;  // for the hot-block fix-up
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      float qf[8], kf[8];
      unpack8<T>(qraw[kk], qf);
      unpack8<T>(kraw[kk], kf);
      V8 nq, nk;
#pragma unroll
      for (int j = 0; j < 8; ++j) nq[j] = cv<T>(qf[j] * iq), nk[j] = cv<T>(kf[j] * ik);
      qraw[kk] = *reinterpret_cast<const uint4*>(&nq);
      kraw[kk] = *reinterpret_cast<const uint4*>(&nk);
    }
  }
  load_v_pass(0);
  if constexpr (kLoadPriority) __builtin_amdgcn_s_setprio(0);

  // ---- 2. in-block inclusive cumsum of the log2 gate over the 16 rows (one DPP row per channel group) ----
  if constexpr (kGate) {
    const float keep = valid ? kLog2e : 0.f;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
#pragma unroll
      for (int j = 0; j < 8; ++j) bl[kk][j] = row_scan16(bl[kk][j] * keep);
    if (l16 == 15) {
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        float* dst = tot + p * K + 32 * kk + 8 * g4;
        *reinterpret_cast<float4*>(dst) = make_float4(bl[kk][0], bl[kk][1], bl[kk][2], bl[kk][3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(bl[kk][4], bl[kk][5], bl[kk][6], bl[kk][7]);
      }
    }
  }
  if (g4 == 0) sbeta[16 * p + l16] = valid ? beta_t : 0.f;
  lds_barrier();

  // ---- 3a. channel vectors, spread over the workgroup: EPRE[i] = e^{a_{i-1}}, ETAIL[i] = e^{B_end - a_i};
  // strip key factors RDS[i] = e^{-T_i} (0 for a hot channel) and FAR = e^{a_{i-1} - a_j} for tiles (2,0),
  // (3,0), (3,1) ----
  // Thread x covers channel x mod K of the vectors v = x / K, x / K + 256 / K, ... (15 vectors of K channels), so it
  // reads that channel's four block totals once.
  static_assert(256 % K == 0, "channel vectors: a thread keeps one channel");
  if constexpr (kGate) {
    const int ch = threadIdx.x % K;
    const float t0 = tot[ch], t1 = tot[K + ch], t2 = tot[2 * K + ch], t3 = tot[3 * K + ch];
#pragma unroll
    for (int v = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / K); v < 15; v += 256 / K) {  // wave-uniform v
      if (v < 4) {
        const float t = v == 0 ? t0 : v == 1 ? t1 : v == 2 ? t2 : t3;
        rds[v * K + ch] = -t > kHot ? 0.f : __builtin_amdgcn_exp2f(-t);
      } else if (v < 7) {
        far[(v - 4) * K + ch] = __builtin_amdgcn_exp2f(v == 4 ? t1 : (v == 5 ? t1 + t2 : t2));
      } else if (v < 11) {
        const int i = v - 7;
        epre_v[i * K + ch] = __builtin_amdgcn_exp2f(i == 0 ? 0.f : i == 1 ? t0 : i == 2 ? t0 + t1 : t0 + t1 + t2);
      } else {
        const int i = v - 11;
        etail_v[i * K + ch] = __builtin_amdgcn_exp2f(i == 0 ? t1 + t2 + t3 : i == 1 ? t2 + t3 : i == 2 ? t3 : 0.f);
      }
    }
    if (threadIdx.x < K) reinterpret_cast<float*>(rec + R::GAM)[ch] = __builtin_amdgcn_exp2f(t0 + t1 + t2 + t3);
  } else {
    if (threadIdx.x < K) reinterpret_cast<float*>(rec + R::GAM)[threadIdx.x] = 1.f;
  }
  lds_barrier();

  // ---- 3b. operands: Lq, Lk = (q, k) e^{B - a_{p-1}} (block-start anchor), Kap = k e^{a_p - B} (block-end
  // anchor); Q e^B (times the output scale) and K e^{B_end - B} to the record ----
  V8 lq[KS], lk[KS];
  // f16 operands: the diagonal strip tile runs on bf16 operands formed here in fp32 (see step 4)
  constexpr bool kWideDiag = kGate && __is_same(T, _Float16);
  bf16x8 dq[kWideDiag ? KS : 1], dk[kWideDiag ? KS : 1], dkey[kWideDiag ? KS : 1];
  const uint32_t keep_bits = valid ? 0xffffffffu : 0u;
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    const int ch = 32 * kk + 8 * g4;
    float qf[8], kf[8];
    unpack8<T>(make_uint4(qraw[kk].x & keep_bits, qraw[kk].y & keep_bits, qraw[kk].z & keep_bits,
                       qraw[kk].w & keep_bits), qf);
    unpack8<T>(make_uint4(kraw[kk].x & keep_bits, kraw[kk].y & keep_bits, kraw[kk].z & keep_bits,
                       kraw[kk].w & keep_bits), kf);
    float tw[8], ep[8], et[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) tw[j] = 0.f, ep[j] = et[j] = 1.f;
    if constexpr (kGate) {
      const float4 a0 = *reinterpret_cast<const float4*>(tot + p * K + ch);
      const float4 a1 = *reinterpret_cast<const float4*>(tot + p * K + ch + 4);
      const float4 b0 = *reinterpret_cast<const float4*>(epre_v + p * K + ch);
      const float4 b1 = *reinterpret_cast<const float4*>(epre_v + p * K + ch + 4);
      const float4 d0 = *reinterpret_cast<const float4*>(etail_v + p * K + ch);
      const float4 d1 = *reinterpret_cast<const float4*>(etail_v + p * K + ch + 4);
      const float ta[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
      const float tb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
      const float td[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) tw[j] = ta[j], ep[j] = tb[j], et[j] = td[j];
    }
    V8 vq, vk, vkap, vkd, vkt, vqd;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float ell = 1.f, rho = 1.f;
      if constexpr (kGate) {
        ell = __builtin_amdgcn_exp2f(bl[kk][j]);
        rho = __builtin_amdgcn_exp2f(tw[j] - bl[kk][j]);
      }
      const float q1 = qf[j] * ell, k1 = kf[j] * ell, kp1 = kf[j] * rho;
      vq[j] = cv<T>(q1);
      vk[j] = cv<T>(k1);
      vkap[j] = cv<T>(kp1);
      vkd[j] = cv<T>(k1 * ep[j]);
      vkt[j] = cv<T>(kp1 * et[j]);
      vqd[j] = cv<T>(q1 * (ep[j] * a.scale));
      if constexpr (kWideDiag) {  // q e^{B - a_{p-1}}, k e^{B - a_{p-1}} and k e^{a_{p-1} - B} (0 for a hot channel)
        dq[kk][j] = bf(q1);
        dk[kk][j] = bf(k1);
        dkey[kk][j] = bf(-tw[j] > kHot ? 0.f : kf[j] * __builtin_amdgcn_exp2f(-bl[kk][j]));
      }
    }
    lq[kk] = vq;
    lk[kk] = vk;
    const int ro = (16 * p + l16) * KP + ch;
    *reinterpret_cast<V8*>(kap + ro) = vkap;
    if constexpr (kDelta) *reinterpret_cast<V8*>(kd + ro) = vkd;
    // scale Q e^B in the permuted channel order: this lane's channels 8 g4 .. 8 g4 + 7 of the group land as two
    // 4-channel pieces at positions pb and pb + 8
    const int pb = 32 * kk + 16 * (g4 & 1) + 4 * (g4 >> 1);
    T* qrec = reinterpret_cast<T*>(rec + R::QD);
    *reinterpret_cast<V4*>(qrec + R::rk(16 * p + l16, pb)) = V4{vqd[0], vqd[1], vqd[2], vqd[3]};
    *reinterpret_cast<V4*>(qrec + R::rk(16 * p + l16, pb + 8)) = V4{vqd[4], vqd[5], vqd[6], vqd[7]};
    *reinterpret_cast<V8*>(reinterpret_cast<T*>(rec + R::KT) + R::rk(16 * p + l16, ch)) = vkt;
  }
  lds_barrier();

  // ---- 4. gated strips of block row p: tiles (p, j <= p) of Sc and P ----
  // Off-diagonal key factors are <= 1.  The diagonal tile's e^{-T_p} is bounded only by the hot threshold (e^60):
  // with f16 operands (range 65504, subnormal below 6e-5) the diagonal tile instead runs on the bf16 operands formed
  // in fp32 in step 3b from this lane's own row (the diagonal tile's key rows are the lanes' own rows), the
  // precision the bf16 path gives it; the f16 result of that tile is replaced by a select (every MFMA runs).
  floatx4 diag_s = {0.f, 0.f, 0.f, 0.f}, diag_p = {0.f, 0.f, 0.f, 0.f};
  if constexpr (kWideDiag) {
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      diag_s = mfma32(dq[kk], dkey[kk], diag_s);
      if constexpr (kDelta) diag_p = mfma32(dk[kk], dkey[kk], diag_p);
    }
  }
  for (int j = 0; j <= p; ++j) {
    floatx4 acc_s = {0.f, 0.f, 0.f, 0.f}, acc_p = {0.f, 0.f, 0.f, 0.f};
    const bool diag = j == p, adjacent = j + 1 == p;
    const float* kscale = diag ? rds + p * K : far + ((p == 2) ? 0 : (j == 0 ? 1 : 2)) * K;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int ch = 32 * kk + 8 * g4;
      V8 bk = *reinterpret_cast<const V8*>(kap + (16 * j + l16) * KP + ch);
      if (kGate && !adjacent) {
        const float4 f0 = *reinterpret_cast<const float4*>(kscale + ch);
        const float4 f1 = *reinterpret_cast<const float4*>(kscale + ch + 4);
        const float f[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) bk[e] = cv<T>(f32(bk[e]) * f[e]);
      }
      acc_s = mfma32(lq[kk], bk, acc_s);
      if constexpr (kDelta) acc_p = mfma32(lk[kk], bk, acc_p);
    }
    if constexpr (kWideDiag) {
#pragma unroll
      for (int r = 0; r < 4; ++r) acc_s[r] = diag ? diag_s[r] : acc_s[r], acc_p[r] = diag ? diag_p[r] : acc_p[r];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 4 * g4 + r, sl = l16;
      sct[tri_tile(p, j) * 256 + t * 16 + sl] = cv<T>(diag && t < sl ? 0.f : acc_s[r]);
      if constexpr (kDelta) {
        const float pv = acc_p[r] * sbeta[16 * p + t];
        if (diag) lii[p * 256 + t * 16 + sl] = t > sl ? pv : 0.f;
        else negl[strict_tile(p, j) * 256 + t * 16 + sl] = cv<T>(-pv);
      }
    }
  }
  // exact elementwise diagonal block for hot channels (rare)
  if constexpr (kGate) {
    constexpr int LPR = K / 8;
    const int cgh = lane % LPR;
    uint32_t hot_mask = 0;
#pragma unroll
    for (int m = 0; m < 8; ++m) hot_mask |= (-tot[p * K + 8 * cgh + m] > kHot) ? (1u << m) : 0u;
    if (__any(hot_mask != 0)) {
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      auto fixup = [&](const auto& rows) {
        hot_diag_fixup<K, kDelta>(c * kChunk, p, len, hot_mask, sct + tri_tile(p, p) * 256, lii + p * 256,
                                  sbeta + 16 * p, rows);
      };
      if constexpr (kPro != 0) {
      if (kLowRank || kConv || (pro.flags & GDR_PRO_NORM_QK)) {
        // The fused prologue's inputs are not in memory as the kernel used them: q, k are renormalised with the
        // row norms kept in LDS, and the gate is recomputed from z and W (the R-long dot split over the 4 lanes
        // that share a row).
        const bool norm = pro.flags & GDR_PRO_NORM_QK;
        auto rows = [&](int tcr, int ch, float& q, float& k, float& g) {
          InputRowsT<T>{x, kGate}(tcr, ch, q, k, g);  // g is replaced below when it is computed
          if (conv) {
            q = conv1(x.qp + ch, x.q_st, tcr, cwq + ch * cw, state_rows(0, ck, int64_t(h) * K + ch));
            k = conv1(x.kp + ch, x.k_st, tcr, cwk + ch * cw, state_rows(1, ck, int64_t(h) * K + ch));
          }
          const int r = tcr - c * kChunk;          // row within the chunk (clamped rows stay inside it)
          if (norm) q = f32(cv<T>(q * snorm[r])), k = f32(cv<T>(k * snorm[64 + r]));
          if constexpr (kLowRank) {
            const int R = pro.rank, part = lane >> 4, span = R / 4;
            const __bf16* zr = static_cast<const __bf16*>(pro.gate_lowrank.ptr) + bidx * pro.gate_lowrank.stride_b +
                               int64_t(bos + tcr) * pro.gate_lowrank.stride_t + part * span;
            const __bf16* wr = static_cast<const __bf16*>(pro.gate_weight) + (size_t(h) * K + ch) * R + part * span;
            float acc = 0.f;
            for (int e = 0; e < span; e += 8) {
              float zf[8], wf[8];
              unpack8<__bf16>(*reinterpret_cast<const uint4*>(zr + e), zf);
              unpack8<__bf16>(*reinterpret_cast<const uint4*>(wr + e), wf);
#pragma unroll
              for (int j = 0; j < 8; ++j) acc += zf[j] * wf[j];
            }
            acc += __shfl_xor(acc, 16, kWave);
            acc += __shfl_xor(acc, 32, kWave);
            const float bias = pro.gate_bias ? pro.gate_bias[size_t(h) * K + ch] : 0.f;
            g = -__builtin_amdgcn_exp2f(pro.a_log[h] * kLog2e) * softplus_f32(acc + bias);
          }
        };
        fixup(rows);
      } else {
        fixup(InputRowsT<T>{x, kGate});
      }
      } else {
        fixup(InputRowsT<T>{x, kGate});
      }
    }
  }
  lds_barrier();

  // ---- 5. diagonal inverses (wave p, 16 lanes, fp32 forward substitution); V pass 0 staged; score tiles
  // (times the output scale) to the record ----
  if constexpr (kDelta) {
    if (lane < 16) {
      const float* lt = lii + p * 256;
      float xcol[16];
      xcol[0] = lane == 0 ? 1.f : 0.f;
#pragma unroll
      for (int r = 1; r < 16; ++r) {
        float lrow[16];
#pragma unroll
        for (int m4 = 0; m4 < (r + 3) / 4; ++m4) {
          const float4 v = *reinterpret_cast<const float4*>(lt + r * 16 + 4 * m4);
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
      for (int r = 0; r < 16; ++r) ainv[p * 256 + r * 16 + lane] = cv<T>(xcol[r]);
    }
  }
  stage_v_pass(0);
  for (int i = threadIdx.x; i < 10 * 256 / 8; i += 256) {
    V8 v8 = reinterpret_cast<const V8*>(sct)[i];
#pragma unroll
    for (int e = 0; e < 8; ++e) v8[e] = cv<T>(f32(v8[e]) * a.scale);
    reinterpret_cast<V8*>(rec + R::SC)[i] = v8;
  }
  lds_barrier();

  // ---- 6. [W | U] = A diag(beta) [K e^B | V] by blocked forward substitution over 16-column tiles.
  // Block i: Y_i = diag(beta_i) R_i - sum_{j<i} L_ij X_j,  X_i = A_ii Y_i.  X_i (accumulator layout: rows 4 g4 + r,
  // column l16) feeds the later blocks; for W the transposed product X_i^T = Y_i^T A_ii^T (the same two operands
  // with their roles swapped) puts four consecutive channels of one row in each lane for 8-byte row stores.  The
  // right-hand side comes from row-major LDS tiles through one transposing read per block. ----
  T* wrec = reinterpret_cast<T*>(rec + R::W);
  T* utrec = reinterpret_cast<T*>(rec + R::FIX);
  const floatx4 zero4 = {0.f, 0.f, 0.f, 0.f};
  // One wave solves a group of column tiles together, block by block, so that their dependent MFMA chains
  // interleave and the L and A_ii fragments are read once per block: NW tiles of W (column tiles first + 4 t of
  // K e^B) and NU tiles of U (column tiles first + 4 u of the staged V pass, output columns out0 + 16 (first + 4 u)).
  auto solve_group = [&](auto nw_c, auto nu_c, int first, int out0) {
    constexpr int NW = decltype(nw_c)::value, NU = decltype(nu_c)::value, NT = NW + NU;
    V4 rv[NT][4], xs[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int rhs_off = t < NW ? L::KD : L::VST, col0 = 16 * (first + 4 * (t < NW ? t : t - NW));
#pragma unroll
      for (int i = 0; i < 4; ++i)  // rows 16 i + 4 g4 + r, column col0 + l16
        rv[t][i] = lds_read_tr<T>(smem, rhs_off + ((16 * i + 4 * g4 + (l16 >> 2)) * KP + col0 + 4 * (l16 & 3)) * 2);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      floatx4 z[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) z[t][r] = f32(rv[t][i][r]);
      if constexpr (kDelta) {
        const float4 b4 = *reinterpret_cast<const float4*>(sbeta + 16 * i + 4 * g4);
#pragma unroll
        for (int t = 0; t < NT; ++t) z[t][0] *= b4.x, z[t][1] *= b4.y, z[t][2] *= b4.z, z[t][3] *= b4.w;
#pragma unroll
        for (int j = 0; j < i; ++j) {
          const V4 nl = *reinterpret_cast<const V4*>(negl + strict_tile(i, j) * 256 + l16 * 16 + 4 * g4);
#pragma unroll
          for (int t = 0; t < NT; ++t) z[t] = mfma16(nl, xs[t][j], z[t]);
        }
        const V4 ai = *reinterpret_cast<const V4*>(ainv + i * 256 + l16 * 16 + 4 * g4);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const V4 zb = pack4<T>(z[t]);
          xs[t][i] = pack4<T>(mfma16(ai, zb, zero4));
          if (t < NW) {
            // X_i^T: row 16 i + l16, channels col0 + 4 g4 + r, stored in the permuted channel order
            const int col0 = 16 * (first + 4 * t);
            const V4 xt = pack4<T>(mfma16(zb, ai, zero4));
            const int wpos = 32 * (col0 >> 5) + 8 * g4 + 4 * ((col0 >> 4) & 1);
            *reinterpret_cast<V4*>(wrec + R::rk(16 * i + l16, wpos)) = xt;
          }
        }
      } else {
#pragma unroll
        for (int t = 0; t < NT; ++t) xs[t][i] = pack4<T>(z[t]);
      }
#pragma unroll
      for (int t = NW; t < NT; ++t) {
        const int oc = out0 + 16 * (first + 4 * (t - NW));
        *reinterpret_cast<V4*>(utrec + R::rt(oc + l16, 16 * i + 4 * g4)) = xs[t][i];
      }
    }
  };
  // Full passes (K value columns) give every wave K / 64 tiles of U; W has K / 64 tiles per wave.
  constexpr int TW = kDelta ? K / 64 : 0, TU = K / 64;
  for (int pass = 0; pass < n_pass; ++pass) {
    if (pass > 0) {  // value dims beyond K: later passes staged synchronously
      load_v_pass(pass);
      lds_barrier();
      stage_v_pass(pass);
      lds_barrier();
    }
    const int tiles = pass_width(pass) / 16;
    if (tiles == K / 16) {
      if (pass == 0) solve_group(IntC<TW>{}, IntC<TU>{}, wave, 0);
      else solve_group(IntC<0>{}, IntC<TU>{}, wave, pass * K);
    } else {
      if constexpr (TW > 0) {
        if (pass == 0) solve_group(IntC<TW>{}, IntC<0>{}, wave, 0);
      }
      for (int nt = wave; nt < tiles; nt += 4) solve_group(IntC<0>{}, IntC<1>{}, nt, pass * K);
    }
  }

  // fused prologue: the last chunk of a sequence stores the last W - 1 inputs of each of its head's q, k, v
  // channels, reaching back into the state it was given when the sequence is shorter than W - 1
  if constexpr (kConv) {
  if ((c + 1) * kChunk >= len) {
    const int S = cw - 1, V = a.value_dim, nqk = 2 * K * S, ntot = nqk + V * S;
    for (int idx = threadIdx.x; idx < ntot; idx += 256) {
      const int i = idx < nqk ? idx / (K * S) : 2;
      const int rem = idx < nqk ? idx % (K * S) : idx - nqk, ch = rem / S, sl = rem % S;
      __bf16* so = static_cast<__bf16*>(pro.conv_state_out[i]);
      if (!so) continue;
      const int64_t nch = i < 2 ? ck : cvv;
      const int64_t row = int64_t(n) * nch + (i < 2 ? int64_t(h) * K : int64_t(h) * V) + ch;
      const int r = len - S + sl;
      __bf16 val;
      if (r >= 0) {
        const __bf16* xp = i == 0 ? x.qp : i == 1 ? x.kp : x.vp;
        const int64_t xs = i == 0 ? x.q_st : i == 1 ? x.k_st : x.v_st;
        val = xp[int64_t(r) * xs + ch];
      } else {
        const __bf16* si = static_cast<const __bf16*>(pro.conv_state_in[i]);
        val = si ? si[row * S + sl + len] : bf(0.f);
      }
      so[row * S + sl] = val;
    }
  }
  }
}

// ============================ scan: one workgroup per (sequence, head) x SL value columns ============================
// SL (16, 32 or 64 columns) is chosen per launch so that the workgroups cover the CUs: every compute wave owns 16
// state columns and reads the whole record's W, Q e^B and K e^{B_end - B} from LDS each step, so narrower slices mean
// fewer compute waves per CU sharing its LDS bandwidth and more CUs at work.
template <int SL, int NT>
struct ScanShape {
  static constexpr int kCompute = SL / (16 * NT);                // compute waves, NT 16-column state tiles each
  // loader waves: in the output mode with at most two compute waves, enough for eight waves (two per SIMD), else
  // four.  The record copy, not the arithmetic, sets the step's pace there.
  static constexpr int loaders(int mode) { return mode == 0 && kCompute <= 2 ? 8 - kCompute : 4; }
  static constexpr int kOP = SL + 8;                             // row pitch (elements) of the output tile in LDS
  static constexpr int kStorers = 2;                             // kSave modes: waves storing the state / u tiles
  static constexpr int threads(int mode) { return 64 * (kCompute + loaders(mode)) + (mode != 0 ? 64 * kStorers : 0); }
};

// ============================ packed sequences: the scan's order, longest first ============================
// The scan's workgroups run from a few steps (short sequences) to nc steps each, several per CU slot over the launch,
// and the launch ends when its last workgroup does.  Taking the sequences longest first (the list-scheduling rule
// that finishes earliest) instead of in index order shortens that tail: for the packed configuration's 32 sequences
// at 16 heads, a simulation of the dispatch gives a makespan of 171 steps against 199 (166 with no tail at all).
// One workgroup ranks the sequences by length (descending, ties by index): seq_order[r] is the sequence of rank r.
constexpr int kSeqOrderMax = 512;  // packed calls with more sequences keep the index order
// Whether a packed call's workspace holds the order (its size does not depend on the device).
inline bool seq_order_room(const gdr_args& a) { return a.cu_seqlens && a.n_seqs >= 2 && a.n_seqs <= kSeqOrderMax; }
__global__ __launch_bounds__(kSeqOrderMax) void seq_order_kernel(const int32_t* __restrict__ cu, int n_seqs, int T,
                                                                 int32_t* __restrict__ order) {
  __shared__ int lens[kSeqOrderMax];
  const int s = threadIdx.x;
  if (s < n_seqs) lens[s] = packed_end(cu, s, T) - packed_begin(cu, s, T);
  __syncthreads();
  if (s < n_seqs) {
    const int ls = lens[s];
    int rank = 0;
    for (int m = 0; m < n_seqs; ++m) rank += (lens[m] > ls || (lens[m] == ls && m < s)) ? 1 : 0;
    order[rank] = s;
  }
}

// kMode: kScanOut writes the output (and the final state); kScanStates (the backward's recompute) instead writes the
// state entering every chunk to `states` [NC][K][V] (bf16, rounded as the MFMA operand) and the bf16 u to `ubuf`
// [NC * 64][V], per (sequence, head), skipping the readout; kScanBoth (the forward for training) writes all of it.
template <int VARIANT, int K, typename OutT, int SL, int NT, int kMode = kScanOut, typename T = __bf16>
__global__ __launch_bounds__((ScanShape<SL, NT>::threads(kMode)), 1) void chunk_scan_kernel(const gdr_args a, int n_slices,
                                                                                int xcd_map, int nc,
                                                                                int64_t rec_bytes, int nt_hint,
                                                                                __bf16* __restrict__ states,
                                                                                __bf16* __restrict__ ubuf,
                                                                                const int32_t* __restrict__ seq_order) {
  constexpr bool kSave = kMode != kScanOut, kOut = kMode != kScanStates;
  constexpr bool kDelta = VARIANT != GDR_GLA;
  constexpr int KT = K / 16, KS = K / 32;
  using V8 = vec8<T>;
  using V4 = vec4<T>;
  constexpr int kScanCompute = ScanShape<SL, NT>::kCompute, kOP = ScanShape<SL, NT>::kOP;
  constexpr int kScanLoaders = ScanShape<SL, NT>::loaders(kMode);
  using R = Rec<K>;

  constexpr int SB = R::FIX + R::ut_slice(SL);     // LDS bytes per buffer
  constexpr int kSP = SL + 8;                      // bf16 pitch of the kSave tiles
  constexpr int kSaveOff = 2 * SB + (kOut ? 2 * 64 * kOP * int(sizeof(OutT)) : 0);
  static_assert(!kSave || (__is_same(T, __bf16) && NT == 1), "kSave: bf16 operands, one tile per wave");
  constexpr int NF = R::FIX / 16, NU = R::ut_slice(SL) / 16;
  // GLA reads no W (u = U): its copies start at the record's Q e^B
  constexpr int G0 = kDelta ? 0 : R::QD / 1024;                 // first 64-piece group copied
  constexpr int NG = ((NF + NU + 63) / 64 - G0 + kScanLoaders - 1) / kScanLoaders;  // 64-piece groups per loader wave
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
  const int H = a.heads;
  const int n = seq_order ? seq_order[bh / H] : bh / H, h = bh % H;  // packed calls: longest sequences first
  int bos = 0, len = a.seq_len, base = n * nc, bidx = n;
  if (a.cu_seqlens) {
    bos = packed_begin(a.cu_seqlens, n, a.seq_len);
    len = packed_end(a.cu_seqlens, n, a.seq_len) - bos;
    base = varlen_base(a.cu_seqlens, n, a.seq_len);
    bidx = 0;
  }
  const int nchunks = (len + kChunk - 1) / kChunk;
  const int v0 = slice * SL;
  const unsigned char* ws = static_cast<const unsigned char*>(a.workspace);
  // wave index made explicitly wave-uniform so that role and group branches are scalar branches
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;

  if (wave >= kScanCompute && wave < kScanCompute + kScanLoaders) {
    // ---------------- loader waves ----------------
    // The record of chunk s + 1 is copied straight into LDS buffer (s + 1) & 1 while the compute waves work on
    // chunk s (global_load_lds_dwordx4: each lane's 16 bytes land at the wave-uniform LDS base + 16 * lane).
    const int lw = wave - kScanCompute;
    const unsigned char* rec0 = ws + (int64_t(base) * H + h) * rec_bytes;
    const int64_t rec_stride = int64_t(H) * rec_bytes;
    const int ut_off = R::FIX + v0 * 64 * 2;
    // The slice workgroups of one head read the same record lines.  Each starts its copy at its own offset into the
    // record (slice / n_slices of the way through), so that a line is first requested by one slice and found in the
    // XCD's L2 by the others later, instead of every slice asking for the same missing lines at the same moment.
    constexpr int kGroups = (NF + NU + 63) / 64 - G0;  // 64-piece groups copied
    const int rot = (slice * kGroups) / n_slices;
    auto copy_record = [&](int chunk, int buf) {
      const unsigned char* src = rec0 + chunk * rec_stride;
      unsigned char* dst = smem + buf * SB;
#pragma unroll
      for (int k = 0; k < NG; ++k) {
        const int j = lw + kScanLoaders * k;  // group of 64 16-byte pieces (past the record: no copy)
        const int g = j < kGroups ? G0 + (j + rot) % kGroups : 1 << 20;
        const int idx = 64 * g + lane;
        if (idx < NF + NU) {
          const int off = idx < NF ? idx * 16 : ut_off + (idx - NF) * 16;
          __builtin_amdgcn_global_load_lds(src + off, (__attribute__((address_space(3))) void*)(dst + 1024 * g),
                                           16, 0, 0);
        }
      }
    };
    // The compute waves leave each chunk's output in a double-buffered LDS tile [64][kOP]; the loaders store the
    // previous chunk's tile during the next step as whole SL-column rows with 16-byte stores.  They read the tile
    // into registers before issuing the next record copy: the compiler orders an LDS read that follows a
    // global_load_lds behind the whole copy (s_waitcnt vmcnt(0)), which would hold the stores back until the copy
    // had landed.
    const OutT* otile = reinterpret_cast<const OutT*>(smem + 2 * SB);
    OutT* op = static_cast<OutT*>(const_cast<void*>(a.out.ptr)) + bidx * a.out.stride_b + h * a.out.stride_h +
               bos * a.out.stride_t;
    constexpr int kPer = 16 / int(sizeof(OutT)), kRowPieces = SL / kPer;
    constexpr int kTilePieces = (kRowPieces + kScanLoaders - 1) / kScanLoaders;  // 16-byte pieces per lane
    uint4 tv[kTilePieces];
    auto read_tile = [&](int chunk) {
      const OutT* tl = otile + (chunk & 1) * 64 * kOP;
#pragma unroll
      for (int i = 0; i < kTilePieces; ++i) {
        const int pc = 64 * (lw + kScanLoaders * i) + lane;
        if (pc < 64 * kRowPieces) tv[i] = *reinterpret_cast<const uint4*>(tl + (pc / kRowPieces) * kOP + (pc % kRowPieces) * kPer);
      }
    };
    auto write_tile_as = [&](int chunk, auto nt) {  // nt: std::true_type for the hinted stores
#pragma unroll
      for (int i = 0; i < kTilePieces; ++i) {
        const int pc = 64 * (lw + kScanLoaders * i) + lane;
        const int tk = chunk * kChunk + pc / kRowPieces;
        const int64_t e = int64_t(tk) * a.out.stride_t + v0 + (pc % kRowPieces) * kPer;
        if (pc < 64 * kRowPieces && tk < len) {
          if constexpr (decltype(nt)::value) store_nt16(op, uint32_t(e * int64_t(sizeof(OutT))), tv[i]);
          else *reinterpret_cast<uint4*>(op + e) = tv[i];
        }
      }
    };
    auto write_tile = [&](int chunk) {
      if (nt_hint) write_tile_as(chunk, std::true_type{});
      else write_tile_as(chunk, std::false_type{});
    };
    if (nchunks > 0) copy_record(0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
    for (int s = 0; s < nchunks; ++s) {
      if constexpr (kOut) {
        if (s > 0) read_tile(s - 1);
      }
      if (s + 1 < nchunks) copy_record(s + 1, (s + 1) & 1);  // buffer (s + 1) & 1 held chunk s - 1: done
      if constexpr (kOut) {
        if (s > 0) write_tile(s - 1);
      }
      __builtin_amdgcn_s_waitcnt(0);
      lds_barrier();
    }
    if constexpr (kOut) {
      if (nchunks > 0) {
        read_tile(nchunks - 1);
        write_tile(nchunks - 1);
      }
    }
    return;
  }

  if (wave >= kScanCompute) {
    // ---------------- storer waves (kSave) ----------------
    // The compute waves leave the state entering each chunk ([K][kSP]) and u ([64][kSP]) as bf16 in
    // double-buffered LDS tiles; these waves store the previous chunk's tiles during the next step as 16-byte row
    // pieces.  They never wait for their stores (the loaders' wait for the record copy, which precedes each
    // barrier, would otherwise include them).
    if constexpr (kSave) {
      const int sw = wave - kScanCompute - kScanLoaders;
      const __bf16* stile = reinterpret_cast<const __bf16*>(smem + kSaveOff);
      auto store_save_as = [&](int chunk, auto nt) {  // nt: std::true_type for the hinted stores
        constexpr int kRowPieces = SL / 8, kStorers = ScanShape<SL, NT>::kStorers;
        const __bf16* sl = stile + (chunk & 1) * (K + kChunk) * kSP;
        __bf16* sc = states + (size_t(n * H + h) * nc + chunk) * K * a.value_dim;  // this chunk's state [K][V]
        __bf16* uc = ubuf + (size_t(n * H + h) * nc + chunk) * kChunk * a.value_dim;  // and its u [64][V]
        auto rows = [&](__bf16* base, int r0, int nrows) {  // tile rows r0 .. r0 + nrows - 1 to base's rows
#pragma unroll
          for (int pc = sw * 64 + lane; pc < nrows * kRowPieces; pc += 64 * kStorers) {
            const int row = pc / kRowPieces, col = (pc % kRowPieces) * 8;
            const uint4 v = *reinterpret_cast<const uint4*>(sl + (r0 + row) * kSP + col);
            const int e = row * a.value_dim + v0 + col;
            if constexpr (decltype(nt)::value) store_nt16(base, uint32_t(2 * e), v);
            else *reinterpret_cast<uint4*>(base + e) = v;
          }
        };
        rows(sc, 0, K);
        rows(uc, K, kChunk);
      };
      auto store_save = [&](int chunk) {
        if (nt_hint) store_save_as(chunk, std::true_type{});
        else store_save_as(chunk, std::false_type{});
      };
      lds_barrier();
      for (int s = 0; s < nchunks; ++s) {
        if (s > 0) store_save(s - 1);
        lds_barrier();
      }
      if (nchunks > 0) store_save(nchunks - 1);
    }
    return;
  }

  // ---------------- compute waves: NT 16-column tiles each ----------------
  const int l16 = lane & 15, g4 = lane >> 4;
  const int c0 = v0 + 16 * NT * wave;  // first column of this wave
  const size_t sbase = size_t(n * H + h) * K * a.value_dim;
  floatx4 st[NT][KT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int m = 0; m < KT; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        st[t][m][r] = a.h0 ? a.h0[sbase + size_t(16 * m + 4 * g4 + r) * a.value_dim + c0 + 16 * t + l16] : 0.f;
  lds_barrier();

  __bf16* stile = reinterpret_cast<__bf16*>(smem + kSaveOff);
  auto store_state = [&](int c) {  // the state entering chunk c (bf16, the MFMA operand's rounding) into its tile
    __bf16* tl = stile + (c & 1) * (K + kChunk) * kSP + (c0 - v0) + l16;
#pragma unroll
    for (int m = 0; m < KT; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) tl[(16 * m + 4 * g4 + r) * kSP] = bf(st[0][m][r]);
  };

  OutT* otile = reinterpret_cast<OutT*>(smem + 2 * SB);
  for (int s = 0; s < nchunks; ++s) {
    const unsigned char* bb = smem + (s & 1) * SB;
    if constexpr (kSave) store_state(s);
    const T* wl = reinterpret_cast<const T*>(bb + R::W);
    const T* ql = reinterpret_cast<const T*>(bb + R::QD);
    const T* scl = reinterpret_cast<const T*>(bb + R::SC);
    const float* gam = reinterpret_cast<const float*>(bb + R::GAM);
    const T* utl = reinterpret_cast<const T*>(bb + R::FIX);  // UT rows of this slice

    // Every LDS read of the step is issued ahead of its use, in the order of use (LDS reads return in order):
    // W / Q e^B fragments one row block ahead, the U rows with the first block, the score tiles and the first two
    // K e^{B_end - B} tiles (with their gamma) during the last block, each further Kt tile two tiles ahead.

    // state as the bf16 B operand: two accumulator tiles = one 32-deep k slot set {32kk + 4g4 + r, +16}
    V8 sB[NT][KS];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) sB[t][kk] = concat(pack4<T>(st[t][2 * kk]), pack4<T>(st[t][2 * kk + 1]));

    // X = W S (accumulator layout: token rows, state columns) and the transposed readout (Q e^B S)^T = S^T (Q e^B)^T
    // (the same operands with their roles swapped: state-column rows, token columns), so that each lane ends up
    // with four consecutive output columns of one token.  Every A fragment read from LDS feeds NT tiles.
    floatx4 acc_ot[NT][4];
    V4 ub[NT][4];
    V8 fq[2][KS], fw[2][KS];  // A fragments of row block i (k slots {32kk + 4g4 + r, +16})
    auto read_block = [&](int i, int buf) {
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const int r0 = R::rk(16 * i + l16, 32 * kk + 8 * g4);  // permuted order: one 16-byte read
        if constexpr (kOut) fq[buf][kk] = *reinterpret_cast<const V8*>(ql + r0);
        if constexpr (kDelta) fw[buf][kk] = *reinterpret_cast<const V8*>(wl + r0);
      }
    };
    V8 fk[4][2];    // Kt^T fragments of state tile m (transposing reads of the row-major tile), ring of 4
    float4 gm[4];   // gamma of the same rows
    auto read_kt = [&](int m) {
      const int buf = m % 4;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int tok = 32 * kk + 4 * g4 + (l16 >> 2);
        const int chn = 16 * m + 4 * (l16 & 3);
        const int off = (s & 1) * SB + R::KT;
        fk[buf][kk] = concat(lds_read_tr<T>(smem, off + R::rk(tok, chn) * 2),
                             lds_read_tr<T>(smem, off + R::rk(tok + 16, chn) * 2));
      }
      gm[buf] = *reinterpret_cast<const float4*>(gam + 16 * m + 4 * g4);
    };
    V4 fsc[10];
    read_block(0, 0);
    V4 uu[NT][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int t = 0; t < NT; ++t)
        uu[t][i] = *reinterpret_cast<const V4*>(utl + R::rt(c0 - v0 + 16 * t + l16, 16 * i + 4 * g4));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i + 1 < 4) {
        read_block(i + 1, (i + 1) & 1);
      } else {
        if constexpr (kOut) {
#pragma unroll
          for (int q = 0; q < 10; ++q) fsc[q] = *reinterpret_cast<const V4*>(scl + q * 256 + l16 * 16 + 4 * g4);
        }
        read_kt(0);
        read_kt(1);
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of this block's MFMAs
      floatx4 ax[NT], ao[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) ax[t] = ao[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          if constexpr (kOut) ao[t] = mfma32(sB[t][kk], fq[i & 1][kk], ao[t]);
          if constexpr (kDelta) ax[t] = mfma32(fw[i & 1][kk], sB[t][kk], ax[t]);
        }
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        floatx4 u;
#pragma unroll
        for (int r = 0; r < 4; ++r) u[r] = kDelta ? f32(uu[t][i][r]) - ax[t][r] : f32(uu[t][i][r]);
        ub[t][i] = pack4<T>(u);
        acc_ot[t][i] = ao[t];
        if constexpr (kSave) {
          __bf16* tl = stile + (s & 1) * (K + kChunk) * kSP + (K + 16 * i + 4 * g4) * kSP + (c0 - v0) + l16;
#pragma unroll
          for (int r = 0; r < 4; ++r) tl[r * kSP] = ub[t][i][r];
        }
      }
    }
    // O_i^T += u_j^T Sc_ij^T over j <= i, two 16-token blocks per 32-deep MFMA: the concatenated accumulator layouts
    // of u_j, u_{j+1} are the A layout of [u_j u_{j+1}]^T in the two-tile k order, and the score tiles read like
    // Sc_ij give B in the same order (a block past i contributes zeros).  Every MFMA accumulating onto the readout
    // has the readout's shape, so no accumulator passes between MFMAs of different shapes.
    if constexpr (kOut) {
      const V4 z4 = {};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j <= i; j += 2)
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            const bool pair = j + 1 <= i;
            acc_ot[t][i] = mfma32(concat(ub[t][j], pair ? ub[t][j + 1] : z4),
                                  concat(fsc[tri_tile(i, j)], pair ? fsc[tri_tile(i, j + 1)] : z4), acc_ot[t][i]);
          }
    }
    // S = diag(gamma) S + Kt^T u.  Each state tile takes two dependent MFMAs (tokens 0-31, then 32-63); they are
    // software-pipelined across tiles (tile m's first beside tile m-1's second), so consecutive MFMAs never depend on
    // each other and each tile's accumulation order is unchanged.
    auto update_half = [&](int m, int kk) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
        st[t][m] = mfma32(fk[m % 4][kk], concat(ub[t][2 * kk], ub[t][2 * kk + 1]), st[t][m]);
    };
#pragma unroll
    for (int m = 0; m < KT; ++m) {
      if (m + 2 < KT) read_kt(m + 2);
      __builtin_amdgcn_sched_barrier(0);
      const float4 g = gm[m % 4];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        st[t][m][0] *= g.x; st[t][m][1] *= g.y; st[t][m][2] *= g.z; st[t][m][3] *= g.w;
      }
      update_half(m, 0);
      if (m > 0) update_half(m - 1, 1);
    }
    update_half(KT - 1, 1);
    // output: lane holds O[token 16 i + l16][columns c0 + 16 t + 4 g4 .. + 3], into the chunk's LDS tile
    if constexpr (kOut) {
      OutT* tw = otile + (s & 1) * 64 * kOP;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t) store4(tw + (16 * i + l16) * kOP + (c0 - v0) + 16 * t + 4 * g4, acc_ot[t][i]);
    }
    lds_barrier();
  }
  if (a.ht) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int m = 0; m < KT; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          a.ht[sbase + size_t(16 * m + 4 * g4 + r) * a.value_dim + c0 + 16 * t + l16] = st[t][m][r];
  }
}

int64_t slots_per_head(const gdr_args& a) {
  if (a.cu_seqlens) return (a.seq_len + kChunk - 1) / kChunk + a.n_seqs;
  return int64_t(a.batch) * ((a.seq_len + kChunk - 1) / kChunk);
}

// Whether the call's single-use input rows (prep) and its outputs, states and u (scan) carry the non-temporal hint.
// It pays when the records are about one to four times the 256 MB memory-side cache: the hint keeps inputs and
// outputs from displacing the records the scan is about to read.  KDA at T = 4096, H = 16 (with the scan's output
// tile read ahead of the record copy), by batch: B = 4 (297 MB of records) 234 -> 225 us per call, B = 6
// 392 -> 380, B = 8 411 -> 402, B = 12 673 -> 664; the c4 variants (B = 2, T = 8192) 9-29 us faster per call; the
// training forward at B = 4 270 -> 248 us.  Smaller calls, whose inputs stay cached from one call to the next, and
// larger ones ran slower with the hint on every access (B = 1 96 -> 103 us, B = 2 133 -> 135, B = 16 808 -> 812,
// the 1.5 GB packed call 3 % slower), so they go without.  The scan's hinted stores take 32-bit byte offsets from
// each sequence's first output row, so every output row must lie within 4 GiB of it.
template <int K>
bool use_nt_hint(const gdr_args& a) {
  constexpr int64_t kMin = int64_t(256) << 20, kMax = int64_t(1) << 30;
  const int64_t records = slots_per_head(a) * a.heads * Rec<K>::bytes(a.value_dim);
  if (records < kMin || records > kMax) return false;
  return (int64_t(a.seq_len) * a.out.stride_t + a.value_dim) * 4 < (int64_t(1) << 32);
}

template <int VARIANT, int K, int kPro, typename T = __bf16, int kNT = 0>
hipError_t launch_prep(const gdr_args& a, const gdr_prologue& pro, hipStream_t stream) {
  const int nc = (a.seq_len + kChunk - 1) / kChunk;
  const int64_t n_prep = slots_per_head(a) * a.heads;
  constexpr int prep_lds = PrepLds<K>::BYTES;
  hipError_t e = configure_lds<&chunk_prep_kernel<VARIANT, K, kPro, kNT, T>>(prep_lds);
  if (e != hipSuccess) return e;
  if (n_prep > 0)
    hipLaunchKernelGGL((chunk_prep_kernel<VARIANT, K, kPro, kNT, T>), dim3(unsigned(n_prep)), dim3(256), prep_lds,
                       stream, a, nc, Rec<K>::bytes(a.value_dim), pro);
  return hipGetLastError();
}

// The plain op's prep on bf16 inputs, with the hinted input loads when the call asks for them.
template <int VARIANT, int K>
hipError_t launch_prep_plain(const gdr_args& a, hipStream_t stream) {
  return use_nt_hint<K>(a) ? launch_prep<VARIANT, K, 0, __bf16, 1>(a, gdr_prologue{}, stream)
                           : launch_prep<VARIANT, K, 0>(a, gdr_prologue{}, stream);
}

}  // namespace

// Compute units of the current device (queried once per device; 256 on MI355X).
int device_cus() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cus[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Value columns per scan workgroup: the widest slice (fewest record copies into LDS) whose workgroups still cover
// every CU, else the narrowest.
int scan_slice(int64_t bh, int value_dim) {
  const int64_t cus = device_cus();
  for (int sl : {64, 32})
    if (value_dim % sl == 0 && bh * (value_dim / sl) >= cus) return sl;
  return 16;
}

namespace {

template <int VARIANT, int K, typename OutT, int SL, int NT, int kMode, typename T>
hipError_t launch_scan_sl(const gdr_args& a, int nc, __bf16* states, __bf16* ubuf, const int32_t* seq_order,
                          hipStream_t stream) {
  using Sh = ScanShape<SL, NT>;
  constexpr int scan_lds = 2 * (Rec<K>::FIX + Rec<K>::ut_slice(SL)) +
                           (kMode == kScanStates ? 0 : 2 * 64 * Sh::kOP * int(sizeof(OutT))) +
                           (kMode == kScanOut ? 0 : 2 * (K + kChunk) * (SL + 8) * 2);
  static_assert(scan_lds <= 160 * 1024, "scan LDS");
  constexpr auto kernel = &chunk_scan_kernel<VARIANT, K, OutT, SL, NT, kMode, T>;
  hipError_t e = configure_lds<kernel>(scan_lds);
  if (e != hipSuccess) return e;
  const int n_seq = a.cu_seqlens ? a.n_seqs : a.batch;
  const int bh = n_seq * a.heads;
  const int n_slices = a.value_dim / SL;
  const int xcd_map = (bh % 8 == 0) ? 1 : 0;
  hipLaunchKernelGGL(kernel, dim3(bh * n_slices), dim3(Sh::threads(kMode)), scan_lds, stream, a, n_slices, xcd_map, nc,
                     Rec<K>::bytes(a.value_dim), int(use_nt_hint<K>(a)), states, ubuf, seq_order);
  return hipGetLastError();
}

template <int VARIANT, int K, typename OutT, int kMode, typename T = __bf16>
hipError_t launch_scan(const gdr_args& a, __bf16* states, __bf16* ubuf, hipStream_t stream,
                       const int32_t* seq_order = nullptr) {
  const int nc = (a.seq_len + kChunk - 1) / kChunk;
  const int n_seq = a.cu_seqlens ? a.n_seqs : a.batch;
  // The saving modes' extra LDS tiles cap the slice width: 32 columns (16 beside an fp32 output tile).
  constexpr int kMaxSL = kMode == kScanOut ? 64 : (kMode == kScanBoth && sizeof(OutT) == 4 ? 16 : 32);
  const int sl = std::min(scan_slice(int64_t(n_seq) * a.heads, a.value_dim), kMaxSL);
  if constexpr (kMaxSL >= 64) {
    if (sl == 64) return launch_scan_sl<VARIANT, K, OutT, 64, 1, kMode, T>(a, nc, states, ubuf, seq_order, stream);
  }
  if constexpr (kMaxSL >= 32) {
    if (sl == 32) return launch_scan_sl<VARIANT, K, OutT, 32, 1, kMode, T>(a, nc, states, ubuf, seq_order, stream);
  }
  return launch_scan_sl<VARIANT, K, OutT, 16, 1, kMode, T>(a, nc, states, ubuf, seq_order, stream);
}

// The longest-first order of a packed call's sequences, written into the workspace after the records.  NULL (index
// order) when the call is not packed, has more than kSeqOrderMax sequences, or launches no more scan workgroups than
// there are CUs (they then all start at once and the order cannot matter; the ranking launch costs about 5 us).
hipError_t launch_seq_order(const gdr_args& a, int64_t records, const int32_t** order, hipStream_t stream) {
  *order = nullptr;
  if (!seq_order_room(a)) return hipSuccess;
  if (int64_t(a.n_seqs) * a.heads * (a.value_dim / scan_slice(int64_t(a.n_seqs) * a.heads, a.value_dim)) <=
      device_cus())
    return hipSuccess;
  int32_t* o = reinterpret_cast<int32_t*>(static_cast<unsigned char*>(a.workspace) + records);
  hipLaunchKernelGGL(seq_order_kernel, dim3(1), dim3(kSeqOrderMax), 0, stream, a.cu_seqlens, a.n_seqs, a.seq_len, o);
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) *order = o;  // the scan reads the order only when it was written
  return e;
}

template <int VARIANT, int K, typename OutT>
hipError_t launch_split_typed(const gdr_args& a, const gdr_prologue& pro, hipStream_t stream) {
  const int32_t* order;
  const hipError_t oe = launch_seq_order(a, slots_per_head(a) * a.heads * Rec<K>::bytes(a.value_dim), &order, stream);
  if (oe != hipSuccess) return oe;
  if (a.q.dtype == GDR_F16) {  // f16 q, k, v: f16 MFMA operands and records (plain op only)
    hipError_t e = launch_prep<VARIANT, K, 0, _Float16>(a, pro, stream);
    if (e != hipSuccess) return e;
    return launch_scan<VARIANT, K, OutT, kScanOut, _Float16>(a, nullptr, nullptr, stream, order);
  }
  hipError_t e;
  const bool conv = pro.flags & GDR_PRO_CONV;
  const bool any_width = conv && pro.conv_size != 4;  // widths other than 4: one kernel per mode for all of them
  if (!pro.flags) {
    e = launch_prep_plain<VARIANT, K>(a, stream);
  } else if constexpr (VARIANT == GDR_KDA || VARIANT == GDR_GLA) {
    if (pro.flags & GDR_PRO_GATE_LOWRANK)
      e = !conv ? launch_prep<VARIANT, K, 2>(a, pro, stream)
                : any_width ? launch_prep<VARIANT, K, 22>(a, pro, stream) : launch_prep<VARIANT, K, 6>(a, pro, stream);
    else
      e = !conv ? launch_prep<VARIANT, K, 1>(a, pro, stream)
                : any_width ? launch_prep<VARIANT, K, 21>(a, pro, stream) : launch_prep<VARIANT, K, 5>(a, pro, stream);
  } else {
    e = !conv ? launch_prep<VARIANT, K, 1>(a, pro, stream)
              : any_width ? launch_prep<VARIANT, K, 21>(a, pro, stream) : launch_prep<VARIANT, K, 5>(a, pro, stream);
  }
  if (e != hipSuccess) return e;
  return launch_scan<VARIANT, K, OutT, kScanOut>(a, nullptr, nullptr, stream, order);
}

template <int VARIANT, int K>
hipError_t launch_split_k(const gdr_args& a, const gdr_prologue& pro, hipStream_t stream) {
  switch (a.out.dtype) {
    case GDR_BF16: return launch_split_typed<VARIANT, K, __bf16>(a, pro, stream);
    case GDR_F16: return launch_split_typed<VARIANT, K, _Float16>(a, pro, stream);
    default: return launch_split_typed<VARIANT, K, float>(a, pro, stream);
  }
}

template <int VARIANT>
hipError_t launch_split_v(const gdr_args& a, const gdr_prologue& pro, hipStream_t stream) {
  return a.key_dim == 64 ? launch_split_k<VARIANT, 64>(a, pro, stream) : launch_split_k<VARIANT, 128>(a, pro, stream);
}

// Backward recompute: records into the backward workspace, then the scan in its states mode.
template <int VARIANT, int K>
hipError_t launch_states_typed(const gdr_args& fwd, const BwdLayout& L, unsigned char* ws, hipStream_t stream) {
  gdr_args a = fwd;
  a.workspace = ws + L.rec;
  a.ht = nullptr;
  hipError_t e = launch_prep_plain<VARIANT, K>(a, stream);
  if (e != hipSuccess) return e;
  return launch_scan<VARIANT, K, __bf16, kScanStates>(a, reinterpret_cast<__bf16*>(ws + L.states),
                                              reinterpret_cast<__bf16*>(ws + L.ubuf), stream);
}

// Forward for training: the records into the backward workspace, then the scan writing the output and the final
// state together with the states and u that the backward reads.
template <int VARIANT, int K>
hipError_t launch_train_typed(const gdr_args& fwd, const BwdLayout& L, unsigned char* ws, hipStream_t stream) {
  gdr_args a = fwd;
  a.workspace = ws + L.rec;
  hipError_t e = launch_prep_plain<VARIANT, K>(a, stream);
  if (e != hipSuccess) return e;
  __bf16* states = reinterpret_cast<__bf16*>(ws + L.states);
  __bf16* ubuf = reinterpret_cast<__bf16*>(ws + L.ubuf);
  return a.out.dtype == GDR_F32 ? launch_scan<VARIANT, K, float, kScanBoth>(a, states, ubuf, stream)
                                : launch_scan<VARIANT, K, __bf16, kScanBoth>(a, states, ubuf, stream);
}

template <int VARIANT>
hipError_t launch_train_v(const gdr_args& a, const BwdLayout& L, unsigned char* ws, hipStream_t stream) {
  return a.key_dim == 64 ? launch_train_typed<VARIANT, 64>(a, L, ws, stream)
                         : launch_train_typed<VARIANT, 128>(a, L, ws, stream);
}

template <int VARIANT>
hipError_t launch_states_v(const gdr_args& a, const BwdLayout& L, unsigned char* ws, hipStream_t stream) {
  return a.key_dim == 64 ? launch_states_typed<VARIANT, 64>(a, L, ws, stream)
                         : launch_states_typed<VARIANT, 128>(a, L, ws, stream);
}

}  // namespace

int64_t chunk_workspace_bytes(const gdr_args& a) {
  const int64_t rec = a.key_dim == 64 ? Rec<64>::bytes(a.value_dim) : Rec<128>::bytes(a.value_dim);
  return slots_per_head(a) * a.heads * rec + (seq_order_room(a) ? (int64_t(a.n_seqs) * 4 + 255) / 256 * 256 : 0);
}

hipError_t launch_chunk_states(const gdr_args& a, const BwdLayout& L, unsigned char* ws, hipStream_t stream) {
  switch (a.variant) {
    case GDR_KDA: return launch_states_v<GDR_KDA>(a, L, ws, stream);
    case GDR_GDN: return launch_states_v<GDR_GDN>(a, L, ws, stream);
    case GDR_GLA: return launch_states_v<GDR_GLA>(a, L, ws, stream);
    default: return launch_states_v<GDR_DELTANET>(a, L, ws, stream);
  }
}

hipError_t launch_chunk_train(const gdr_args& a, const BwdLayout& L, unsigned char* ws, hipStream_t stream) {
  switch (a.variant) {
    case GDR_KDA: return launch_train_v<GDR_KDA>(a, L, ws, stream);
    case GDR_GDN: return launch_train_v<GDR_GDN>(a, L, ws, stream);
    case GDR_GLA: return launch_train_v<GDR_GLA>(a, L, ws, stream);
    default: return launch_train_v<GDR_DELTANET>(a, L, ws, stream);
  }
}

hipError_t launch_chunk_split(const gdr_args& a, const gdr_prologue& pro, hipStream_t stream) {
  switch (a.variant) {
    case GDR_KDA: return launch_split_v<GDR_KDA>(a, pro, stream);
    case GDR_GDN: return launch_split_v<GDR_GDN>(a, pro, stream);
    case GDR_GLA: return launch_split_v<GDR_GLA>(a, pro, stream);
    default: return launch_split_v<GDR_DELTANET>(a, pro, stream);
  }
}

}  // namespace gdr
