// Shared helpers for the gfx950 kernels of the paged-attention path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "auto_infer_amd.h"

namespace aia {

// Records a message for aia_last_error() (thread local) and returns `code`.
int fail(int code, const char* fmt, ...);
// Maps a HIP status to AIA_ERR_HIP with the runtime's message.
int check_hip(hipError_t err, const char* what);

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// bf16 <- f32, round to nearest even (inputs here are finite).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16 pair, round to nearest even (gfx950 converts a
// pair in one instruction, v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// Reductions over lanes l, l^16, l^32, l^48 (the 4 lane groups of an MFMA
// 16-row fragment) with gfx950's VALU lane swaps instead of ds_bpermute's
// LDS crossbar round trip.  Given the same value in both operands,
// v_permlane16_swap / v_permlane32_swap leave each lane holding x[l] and
// x[l ^ 16] (resp. x[l ^ 32]) in its two results, so max or sum of the pair
// equals the xor-shuffle step bit for bit (both operations commute).
__device__ __forceinline__ float group4_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float group4_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

}  // namespace aia
