// Device-side helpers shared by the gfx950 kernels: bf16 bit conversions, wave64
// DPP/shuffle reductions and the paged-KV row addressing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace orator_hip {

constexpr int kWave = 64;

// ---- bf16 <-> fp32 (bf16 is the high half of an fp32; RNE on the way down) ----
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  uint32_t u = __float_as_uint(x);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
// Packs two fp32 into one dword of two RNE bf16 (lo in bits 0..15).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

// ---- DPP lane exchanges (gfx9 encodings) ----
// quad_perm [1,0,3,2] = 0xB1 (xor 1), [2,3,0,1] = 0x4E (xor 2),
// row_half_mirror = 0x141, row_mirror = 0x140.
template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}

__device__ __forceinline__ float quad_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  return v;
}

__device__ __forceinline__ float quad_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  return v;
}

// All-lane reductions over the full wave64.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// 16-byte streaming load with the non-temporal hint: data read exactly once (K/V rows)
// should not displace reused lines; on gfx950 this also raised plain streaming read
// bandwidth from ~6.1 to ~6.8 TB/s.
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_nt(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Orders LDS traffic between the lanes of ONE wave (wave-private LDS regions): the fences
// make the compiler wait for this wave's LDS writes and keep later LDS reads after them.
// Waves may run different trip counts, so a workgroup barrier would not be safe there.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Workgroup barrier for an LDS hand-off between waves that does NOT wait for outstanding
// global loads: __syncthreads() also waits for vmcnt(0), which would drain every register
// prefetch in flight at the barrier.  Only LDS traffic (lgkmcnt) is completed; the asm's
// memory clobber keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Raw v_exp_f32 (2^x); 2^-inf = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// (float)(1 / sqrt((double)x)) for x > 0 -- the RMSNorm factor the oracle forms (a correctly
// rounded double rounded to float) -- by two fp64 Newton steps y += y/2 (1 - x y^2) from the
// fp32 estimate v_rsq_f32: from a 1-ulp start the double is within a few of its ulps of the
// exact value, so its rounding to float agrees with the double formula's except within ~2^-28
// of a float rounding boundary (no mismatch in 3e8 sampled inputs against the formula), in 4
// fp64 FMAs and 2 multiplies where the correctly rounded fp64 sqrt and division expand to ~30
// instructions on a dependent chain.
__device__ __forceinline__ float rsqrt_via_f64(float x) {
  const double xd = static_cast<double>(x);
  double y = static_cast<double>(__builtin_amdgcn_rsqf(x));
  if (!(y < static_cast<double>(INFINITY))) return static_cast<float>(1.0 / sqrt(xd));  // x = 0
#pragma unroll
  for (int i = 0; i < 2; ++i) y = __builtin_fma(0.5 * y, __builtin_fma(-xd * y, y, 1.0), y);
  return static_cast<float>(y);
}

// ---- KV addressing ----
// A cache is a pool of rows [row][Hkv][Dh].  Paged: absolute position j lives in page
// page_table[j >> page_shift], row (page << page_shift) | (j & mask).  Contiguous:
// row j of the stream's own cache.  With an identity page table the two coincide, which
// is how the reference's [max_seq_len][Hkv][Dh] layout is a special case of the pool.
struct KvMap {
  const int* page_table;  // nullptr => contiguous
  int page_shift;
  long stream_base;       // element offset of this stream's cache (contiguous only)

  __device__ __forceinline__ long row_offset(int j, int Hkv, int kvh, int dh) const {
    long row;
    if (page_table) {
      const long page = page_table[j >> page_shift];
      row = (page << page_shift) | (j & ((1 << page_shift) - 1));
    } else {
      row = j;
    }
    return stream_base + (row * Hkv + kvh) * static_cast<long>(dh);
  }
};

}  // namespace orator_hip
