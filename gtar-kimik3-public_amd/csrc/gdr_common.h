// Shared device helpers for the gfx950 gated delta-rule kernels: scalar conversions, dtype-dispatched loads and
// stores, MFMA operand vector types and wavefront shuffles.  Everything here is header-only device code.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gdr.h"

namespace gdr {

constexpr int kWave = 64;  // CDNA wavefront width

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4;

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t x) { return __uint_as_float(uint32_t(x) << 16); }
__device__ __forceinline__ float f16_bits_to_f32(uint16_t x) {
  _Float16 h;
  __builtin_memcpy(&h, &x, 2);
  return float(h);
}

// Load element `i` of a tensor whose dtype is only known at run time (uniform branch per launch).
__device__ __forceinline__ float load_any(const void* p, int64_t i, int dtype) {
  if (dtype == GDR_BF16) return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  if (dtype == GDR_F16) return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  return static_cast<const float*>(p)[i];
}

__device__ __forceinline__ void store_any(void* p, int64_t i, int dtype, float x) {
  if (dtype == GDR_BF16) {
    static_cast<__bf16*>(p)[i] = static_cast<__bf16>(x);
  } else if (dtype == GDR_F16) {
    static_cast<_Float16*>(p)[i] = static_cast<_Float16>(x);
  } else {
    static_cast<float*>(p)[i] = x;
  }
}

// e^x through the hardware 2^x instruction (v_exp_f32) with a log2(e) pre-scale.
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// SiLU x / (1 + e^-x) of the short convolutions, with the hardware reciprocal (v_rcp_f32, 1 ulp) in place of an IEEE
// division (about ten instructions): the standalone and the in-kernel convolutions share it, so their results agree
// bit for bit.
__device__ __forceinline__ float silu_rcp(float x) {
  return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}

__device__ __forceinline__ float shfl_xor(float x, int mask) { return __shfl_xor(x, mask, kWave); }

// x + x[lane ^ m] in every lane (m a power of two below 64, constant after unrolling), formed on the VALU where one
// lane move gives exactly that partner: quad_perm for 1 and 2, the 16-lane row rotated by 8 for 8, and the gfx950
// permlane swaps of two copies of x for 16 and 32 (whose two results hold the partner rows' values, so every lane
// adds the same pair).  m = 4 goes through ds_bpermute.  Bit-identical to x + shfl_xor(x, m).
__device__ __forceinline__ float xor_sum(float x, int m) {
  const int xi = __float_as_int(x);
  if (m == 1) return x + __int_as_float(__builtin_amdgcn_update_dpp(0, xi, 0xB1, 0xf, 0xf, false));   // [1,0,3,2]
  if (m == 2) return x + __int_as_float(__builtin_amdgcn_update_dpp(0, xi, 0x4E, 0xf, 0xf, false));   // [2,3,0,1]
  if (m == 8) return x + __int_as_float(__builtin_amdgcn_update_dpp(0, xi, 0x128, 0xf, 0xf, false));  // row_ror:8
  if (m == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if (m == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  return x + shfl_xor(x, m);
}

// max(x, x[lane ^ m]) for m = 16 or 32 through the permlane swaps (bit-identical to the shuffle form), else a shuffle.
__device__ __forceinline__ float xor_max(float x, int m) {
  if (m == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  if (m == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  return fmaxf(x, shfl_xor(x, m));
}

}  // namespace gdr
