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

__device__ __forceinline__ float shfl_xor(float x, int mask) { return __shfl_xor(x, mask, kWave); }

}  // namespace gdr
