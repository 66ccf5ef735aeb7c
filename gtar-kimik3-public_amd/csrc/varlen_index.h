// Index arithmetic of packed variable-length sequences (cu_seqlens), shared by the kernels and compiled on the host
// by tests/test_varlen_index.py, which checks that every slot and row it yields stays in bounds.
//
// The offsets are device-resident and the kernels read them without a host-side check (one would need a
// synchronisation).  Every kernel therefore reads them through these functions, which clamp them to [0, T] with
// end >= begin: a call whose offsets break the contract (decreasing, negative or past T) computes undefined values
// but reads and writes only inside its tensors and its workspace.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define GDR_HD __host__ __device__ __forceinline__
#else
#define GDR_HD static inline
#endif

namespace gdr {

// First row of packed sequence n, clamped to [0, T].
GDR_HD int packed_begin(const int32_t* cu, int n, int T) {
  const int b = cu[n];
  return b < 0 ? 0 : (b > T ? T : b);
}

// One past the last row of packed sequence n, clamped to [packed_begin(n), T].
GDR_HD int packed_end(const int32_t* cu, int n, int T) {
  const int b = packed_begin(cu, n, T);
  const int e = cu[n + 1];
  return e < b ? b : (e > T ? T : e);
}

// First slot of packed sequence n when each sequence takes ceil(len / block) consecutive slots:
// floor(begin / block) + n.  With offsets that keep the contract the slots of consecutive sequences never overlap
// (floor(a + b) >= floor(a) + floor(b) and floor(len / block) + 1 >= ceil(len / block)); with any offsets every slot
// of sequence n, base + c for c < ceil(len / block), is below ceil(T / block) + n_seqs.
GDR_HD int packed_slot_base(const int32_t* cu, int n, int T, int block) { return packed_begin(cu, n, T) / block + n; }

// The sequence that slot `slot` belongs to: the largest n < n_seqs with packed_slot_base(n) <= slot (binary search;
// the bases are non-decreasing when the offsets are).  The caller still checks that the slot lies inside that
// sequence's slots.
GDR_HD int packed_slot_seq(const int32_t* cu, int n_seqs, int T, int block, int slot) {
  int lo = 0, hi = n_seqs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (packed_slot_base(cu, mid, T, block) <= slot) lo = mid; else hi = mid - 1;
  }
  return lo;
}

}  // namespace gdr
