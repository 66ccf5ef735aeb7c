// Device helpers shared by the causal attention forward (attention.hip) and backward (attention_bwd.hip): the MFMA
// of the two 16-bit operand types, operand concatenation, the swizzled [64][D] LDS tile fed by LDS DMA, and the
// transposing tile read that turns a tile's rows into the k dimension of an A operand.
#pragma once

#include "chunk_common.h"

namespace gdr {
namespace attn {

constexpr int kThreads = 256;  // four waves per workgroup
constexpr int kWaves = kThreads / kWave;
constexpr int kTile = 64;      // rows of a key/value (forward, dq) or query/dO (dk, dv) LDS tile

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short short4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Mma;
template <>
struct Mma<__bf16> {
  using v8 = bf16x8;
  using v4 = bf16x4;
  static __device__ __forceinline__ floatx4 run(v8 a, v8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ v4 pack(floatx4 x) { return chunk::pack4(x); }
};
template <>
struct Mma<_Float16> {
  using v8 = f16x8;
  using v4 = f16x4;
  static __device__ __forceinline__ floatx4 run(v8 a, v8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ v4 pack(floatx4 x) {
    return v4{static_cast<_Float16>(x[0]), static_cast<_Float16>(x[1]), static_cast<_Float16>(x[2]),
              static_cast<_Float16>(x[3])};
  }
};

template <typename V4, typename V8>
__device__ __forceinline__ V8 cat(V4 lo, V4 hi) {
  return V8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// A [kTile][D] tile in LDS with row r's 16-byte chunk c stored at chunk c ^ (r mod D/8), filled straight from global
// memory (global_load_lds_dwordx4: a lane's 16 bytes land at the wave-uniform LDS base + 16 * lane): each lane loads
// the global chunk that belongs at its slot.  GPW groups of 64 pieces per wave per tile.
template <int D>
struct TileDma {
  static constexpr int DC = D / 8;
  static constexpr int GPW = kTile * DC / kWave / kWaves;
  static_assert(GPW >= 1 && kTile * DC % (kWave * kWaves) == 0, "tile load split");
  int lrow[GPW], lcol[GPW];
  int uwave;
  __device__ __forceinline__ void init(int wave_uniform, int lane) {
    uwave = wave_uniform;
#pragma unroll
    for (int k = 0; k < GPW; ++k) {
      const int slot = kWave * (uwave + kWaves * k) + lane;
      lrow[k] = slot / DC;
      lcol[k] = (slot % DC) ^ (lrow[k] % DC);
    }
  }
  // Rows r0 .. r0 + kTile - 1 of `base` (row stride `stride` elements) into `tile`; rows at or past `len` read row
  // len - 1 (callers mask them).
  template <typename T>
  __device__ __forceinline__ void issue(const T* base, int64_t stride, int r0, int len, T* tile) const {
    const int lim = len - 1 - r0;
#pragma unroll
    for (int k = 0; k < GPW; ++k)
      chunk::lds_dma16(base + int64_t(r0 + min(lrow[k], lim)) * stride + 8 * lcol[k],
                       tile + kWave * 8 * (uwave + kWaves * k));
  }
};

// Element offset, inside a swizzled tile, of this lane's row fragment for k step ds of a 16x16x32 A (or B) operand:
// row l16 of the 16-row block, columns 32 ds + 8 g4 .. + 7 (add 16 t D for row block t).
template <int D>
__device__ __forceinline__ int row_frag(int ds, int l16, int g4) {
  return l16 * D + (((4 * ds + g4) ^ (l16 % (D / 8))) << 3);
}

// Element offset of this lane's address for the transposing read of column tile t (columns 16 t .. + 15): row
// 4 g4 + (l16 >> 2), columns 16 t + 4 (l16 & 3) .. + 3.  The swizzle of rows +16, +32, +48 is the same.
template <int D>
__device__ __forceinline__ int tr_frag(int t, int l16, int g4) {
  const int col = 16 * t + 4 * (l16 & 3), r0 = 4 * g4 + (l16 >> 2);
  return r0 * D + (((col >> 3) ^ (r0 % (D / 8))) << 3) + (col & 7);
}

// Four transposing reads (ds_read_b64_tr_b16) at LDS byte address `addr` and the rows 16, 32 and 48 below it.
// Within each 16-lane group, lane c slot r of read m receives tile[4 g4 + r + 16 m][16 t + c] for the address of
// tr_frag(t, ...), so reads 2 s2 and 2 s2 + 1 concatenated are the A operand X^T[16 t + l16][k] of a 16x16x32 MFMA
// whose k runs over the tile rows 32 s2 + {4 g4 + r, 16 + 4 g4 + r}: the order in which two 16-row blocks of a
// D-layout accumulator (lane: rows 4 g4 + r of column l16) concatenate into a B operand.  Issued as inline
// assembly: the compiler cannot tell these reads from LDS DMA still in flight into the other buffers and would
// otherwise wait for that DMA first; callers wait for the results with an explicit lgkmcnt.
template <int D>
__device__ __forceinline__ void tr_read4(uint32_t addr, short4 (&r)[4]) {
  asm volatile(
      "ds_read_b64_tr_b16 %0, %4\n\t"
      "ds_read_b64_tr_b16 %1, %4 offset:%5\n\t"
      "ds_read_b64_tr_b16 %2, %4 offset:%6\n\t"
      "ds_read_b64_tr_b16 %3, %4 offset:%7"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
      : "v"(addr), "i"(2 * 16 * D), "i"(2 * 32 * D), "i"(2 * 48 * D));
}

// LDS byte address of a generic pointer into the dynamic LDS array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>((uintptr_t)(__attribute__((address_space(3))) const unsigned char*)p);
}

}  // namespace attn
}  // namespace gdr
