// Host check of the packed-sequence index arithmetic the kernels use (csrc/varlen_index.h), built with g++ by
// test_varlen_index.py.  For seeded random offsets -- valid ones and ones that break the contract (negative, past T,
// decreasing) -- it walks every workgroup of the mappings the kernels use and checks that each slot and row stays
// in bounds; for valid offsets it also checks that the prep launch (slot -> sequence, chunk) and the scan launch
// (sequence, chunk -> slot) agree and that no two chunks share a slot.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "varlen_index.h"

using gdr::packed_begin;
using gdr::packed_end;
using gdr::packed_slot_base;
using gdr::packed_slot_seq;

static unsigned long long rng = 88172645463325252ull;
static int rnd(int lo, int hi) {  // inclusive
  rng ^= rng << 13; rng ^= rng >> 7; rng ^= rng << 17;
  return lo + int(rng % (unsigned long long)(hi - lo + 1));
}

static int fail(const char* what, int T, const std::vector<int32_t>& cu, int block, int a, int b) {
  std::printf("FAIL %s: T=%d block=%d (%d, %d) cu=", what, T, block, a, b);
  for (int x : cu) std::printf("%d ", x);
  std::printf("\n");
  return 1;
}

// One launch mapping with `block` rows per slot (64: the chunk prep and scan; 128: the attention query blocks).
static int check(const std::vector<int32_t>& cu, int T, int block, bool valid) {
  const int n_seqs = int(cu.size()) - 1;
  const int slots = (T + block - 1) / block + n_seqs;  // the launch's slot count per head
  std::vector<int> owner(slots, -1);
  // prep / attention: workgroup per slot
  for (int slot = 0; slot < slots; ++slot) {
    const int n = packed_slot_seq(cu.data(), n_seqs, T, block, slot);
    if (n < 0 || n >= n_seqs) return fail("slot -> sequence", T, cu, block, slot, n);
    const int bos = packed_begin(cu.data(), n, T), len = packed_end(cu.data(), n, T) - bos;
    const int c = slot - packed_slot_base(cu.data(), n, T, block);
    if (bos < 0 || len < 0 || bos + len > T) return fail("clamped span", T, cu, block, bos, len);
    if (c < 0 || c * block >= len) continue;  // gap slot: the workgroup returns
    const int r0 = bos + c * block, r1 = bos + (c + 1) * block < bos + len ? bos + (c + 1) * block : bos + len;
    if (r0 < 0 || r1 > T || r0 >= r1) return fail("prep rows", T, cu, block, r0, r1);
    if (valid) owner[slot] = n * 100000 + c;
  }
  // scan: workgroup per sequence, chunk loop
  for (int n = 0; n < n_seqs; ++n) {
    const int bos = packed_begin(cu.data(), n, T), len = packed_end(cu.data(), n, T) - bos;
    const int base = packed_slot_base(cu.data(), n, T, block);
    for (int c = 0; c * block < len; ++c) {
      if (base + c < 0 || base + c >= slots) return fail("scan slot", T, cu, block, n, c);
      if (bos + c * block >= T) return fail("scan rows", T, cu, block, n, c);
      if (valid && owner[base + c] != n * 100000 + c) return fail("prep / scan disagree", T, cu, block, n, c);
      if (valid) owner[base + c] = -2;  // each slot read once
    }
  }
  return 0;
}

int main() {
  int cases = 0;
  for (int trial = 0; trial < 20000; ++trial) {
    const int T = rnd(0, 700), n_seqs = rnd(1, 12);
    const bool valid = trial % 2 == 0;
    std::vector<int32_t> cu(n_seqs + 1);
    if (valid) {  // sorted cuts of [0, T], empty sequences included
      cu[0] = 0;
      cu[n_seqs] = T;
      for (int i = 1; i < n_seqs; ++i) cu[i] = rnd(0, T);
      for (int i = 1; i < n_seqs; ++i)
        for (int j = i + 1; j < n_seqs; ++j)
          if (cu[j] < cu[i]) { const int t = cu[i]; cu[i] = cu[j]; cu[j] = t; }
    } else {  // anything: negative, past T, decreasing
      for (auto& x : cu) x = rnd(-300, T + 300);
    }
    for (int block : {64, 128}) {
      if (check(cu, T, block, valid)) return 1;
      ++cases;
    }
  }
  std::printf("ok %d cases\n", cases);
  return 0;
}
