// Device helpers for the MFMA attention kernels (gfx950): bf16 fragment types, the
// 32x32x16 bf16 MFMA, bf16 packing, lane-half exchanges and the transposing LDS read.
#pragma once

#include "common.hpp"

namespace orator_hip {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8_t, u); }

__device__ __forceinline__ f32x16_t mfma32(bf16x8_t a, bf16x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Two fp32 -> two RNE bf16 in one dword (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t cvt_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Sum of the two bf16 halves of w, added to acc (v_dot2_f32_bf16 against (1, 1)).
__device__ __forceinline__ float add_bf16x2(uint32_t w, float acc) {
  const bf16x2_t ones = __builtin_bit_cast(bf16x2_t, 0x3f803f80u);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), ones, acc, false);
}

// Value of the lane 32 apart combined with this lane's.
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives element (i & 3) of the
// 8 bytes addressed by lane 4k + (i >> 2), for k = 0..3.  With lane s of the group pointing at
// row r0 + (s >> 2), columns c0 + 4 (s & 3) .. +3 of a row-major bf16 tile, lane i therefore
// gets column c0 + i of rows r0 .. r0 + 3: a transposed 4 x 16 block.
typedef short s16x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t* p) {
  typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
  const s16x4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p));
  return __builtin_bit_cast(uint2, r);
}

}  // namespace orator_hip
