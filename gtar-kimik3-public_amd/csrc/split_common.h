// Workspace record layout and small helpers shared by the two-launch prefill (chunk_split.hip) and the
// chunkwise backward (chunk_bwd.hip).
#pragma once

#include "chunk_common.h"
#include "varlen_index.h"

namespace gdr {
namespace chunk {

// Workspace record of one (chunk, head); byte offsets.  UT (U^T, [V][64]) closes the record.  Rows are unpadded;
// 16-byte chunks are XOR-swizzled within a row instead (chunk c of row r stored at chunk c ^ (r mod chunks per
// row)), which keeps every LDS read pattern of the scan kernel free of bank conflicts.
//   * W and Q e^B are A operands of 16x16x32 MFMAs whose B operand is the state in the two-tile k order: within
//     each 32-channel group, position 8 g + j holds channel 4 g + j (j < 4) or 16 + 4 g + j - 4 (j >= 4), so a lane
//     reads its 8 operands with one 16-byte LDS read.
//   * K e^{B_end - B} is row-major in natural order and read with the transposing LDS read.
template <int K>
struct Rec {
  static constexpr int W = 0;                                   // bf16 [64][K]   A diag(beta) K e^B (permuted)
  static constexpr int QD = W + 64 * K * 2;                     // bf16 [64][K]   scale Q e^B (permuted)
  static constexpr int KT = QD + 64 * K * 2;                    // bf16 [64][K]   K e^{B_end - B}
  static constexpr int SC = KT + 64 * K * 2;                    // bf16 [10][16][16] scale x gated scores, tile (i, j <= i)
  static constexpr int GAM = SC + 10 * 256 * 2;                 // fp32 [K] e^{B_end}
  static constexpr int FIX = ((GAM + K * 4 + 255) / 256) * 256;  // start of UT
  static constexpr int ut_slice(int cols) { return cols * 64 * 2; }  // bytes of `cols` rows of UT
  static int64_t bytes(int value_dim) { return FIX + ((int64_t(value_dim) * 64 * 2 + 255) / 256) * 256; }
  // element offsets of (row, column) in the swizzled [*][K] arrays and of (row, token) in UT
  static __device__ __forceinline__ int rk(int row, int col) {
    return row * K + (((col >> 3) ^ (row & (K / 8 - 1))) << 3) + (col & 7);
  }
  static __device__ __forceinline__ int rt(int row, int tok) { return row * 64 + (((tok >> 3) ^ (row & 7)) << 3) + (tok & 7); }
};

// Four consecutive outputs in one 8-byte (16-bit types) or 16-byte (fp32) store.
__device__ __forceinline__ void store4(__bf16* dst, floatx4 v) {
  *reinterpret_cast<bf16x4*>(dst) = bf16x4{bf(v[0]), bf(v[1]), bf(v[2]), bf(v[3])};
}
__device__ __forceinline__ void store4(_Float16* dst, floatx4 v) {
  typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 f16x4;
  *reinterpret_cast<f16x4*>(dst) = f16x4{static_cast<_Float16>(v[0]), static_cast<_Float16>(v[1]),
                                         static_cast<_Float16>(v[2]), static_cast<_Float16>(v[3])};
}
__device__ __forceinline__ void store4(float* dst, floatx4 v) {
  *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
}

// First workspace slot of packed sequence n (clamped offsets, one slot per chunk): floor(bos / 64) + n.
__device__ __forceinline__ int varlen_base(const int32_t* cu, int n, int T) { return packed_slot_base(cu, n, T, kChunk); }

}  // namespace chunk
}  // namespace gdr
