// bf16-weight linear layers of the decoder (gfx950): out[M,N] = act(bf16(in)[M,K] W[N,K]^T
// + bias), fp32 accumulation.
//
// Replaces asr_gemm::Linear / LinearPre (include/model/asr_gemm.h:27-38,
// src/model/asr_gemm.cu:160-208) and gemm::LaunchBf16Gemm (include/model/gemm.cuh:384-501):
// activation 0 none, 1 exact-erf GELU, 2 ReLU (gemm.cuh:289-293).
//
//  * M == 1 (decode step) is HBM-bound: a weight stream of N*K*2 bytes.  One wave computes
//    4 output rows; each lane reads 16 contiguous bytes of each row per step, so a wave
//    instruction moves one contiguous 1 KB piece of a row, and the k loop is unrolled so a
//    lane keeps 16 such loads in flight.  x (4-12 KB) is read through the caches.
//  * M > 1 (prefill) is MFMA-bound: this library's bf16 GEMM (gemm_bf16.hip).
//  * K not a multiple of 8, or operands not 16-byte aligned (the audio tower's first conv as
//    a GEMM has K = 9, asr_audio_tower.cu:417-445): the GEMM with element loads, M = 1 too.
#include "common.hpp"
#include "internal.hpp"

namespace orator_hip {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float apply_act(float v, int act) {
  if (act == 1) return 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f));
  if (act == 2) return fmaxf(v, 0.0f);
  return v;
}

// ------------------------------------------------------------------- GEMV (M = 1) ----
constexpr int kGemvRows = 4;    // output rows per wave
constexpr int kGemvWaves = 4;   // waves per workgroup
constexpr int kGemvUnroll = 4;  // 512-element k steps per loop iteration

__device__ __forceinline__ float dot8(const u32x4_t w, const u32x4_t x) {
  float d = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    d = fmaf(bf16_lo(w[j]), bf16_lo(x[j]), d);
    d = fmaf(bf16_hi(w[j]), bf16_hi(x[j]), d);
  }
  return d;
}

__global__ __launch_bounds__(64 * kGemvWaves) void gemv_bf16_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ W,
    const float* __restrict__ bias, float* __restrict__ out, int K, int N, int act) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * kGemvWaves + wave) * kGemvRows;
  if (row0 >= N) return;
  const int nchunk = K >> 3;  // 16-byte chunks per row
  const u32x4_t* xv = reinterpret_cast<const u32x4_t*>(x);
  const u32x4_t* wr[kGemvRows];
#pragma unroll
  for (int r = 0; r < kGemvRows; ++r)
    wr[r] = reinterpret_cast<const u32x4_t*>(W + static_cast<long>(min(row0 + r, N - 1)) * K);
  float acc[kGemvRows] = {};
  int c = lane;
  for (; c + 64 * (kGemvUnroll - 1) < nchunk; c += 64 * kGemvUnroll) {
    u32x4_t wv[kGemvUnroll][kGemvRows], xx[kGemvUnroll];
#pragma unroll
    for (int u = 0; u < kGemvUnroll; ++u) {
      xx[u] = xv[c + 64 * u];
#pragma unroll
      for (int r = 0; r < kGemvRows; ++r) wv[u][r] = __builtin_nontemporal_load(wr[r] + c + 64 * u);
    }
#pragma unroll
    for (int u = 0; u < kGemvUnroll; ++u)
#pragma unroll
      for (int r = 0; r < kGemvRows; ++r) acc[r] += dot8(wv[u][r], xx[u]);
  }
  for (; c < nchunk; c += 64) {
    const u32x4_t xx = xv[c];
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r) acc[r] += dot8(__builtin_nontemporal_load(wr[r] + c), xx);
  }
#pragma unroll
  for (int r = 0; r < kGemvRows; ++r) acc[r] = wave_sum(acc[r]);
  if (lane < kGemvRows && row0 + lane < N) {
    float v = acc[0];
#pragma unroll
    for (int r = 1; r < kGemvRows; ++r)
      if (lane == r) v = acc[r];
    if (bias) v += bias[row0 + lane];
    out[row0 + lane] = apply_act(v, act);
  }
}

// ------------------------------------------------------ fused decode-step GEMV ----
// out[n] (=, or += with ACC) sum_k xb[k] W[n,k] for one input row, where the bf16 row xb is
// built in LDS by the workgroup from the fp32 producer of the decode step:
//   kGemvInF32      xb = bf16(x)                                 (F32ToBf16 + LinearPre)
//   kGemvInRmsNorm  xb = bf16(x * rsqrt(mean(x^2) + eps) * w)     (RmsNorm + F32ToBf16)
//   kGemvInSwiglu   xb = bf16(silu(g) * u), g = x, u = aux        (SwiGLU + F32ToBf16)
// so one launch replaces three of asr_text_decoder.cu:398-429; ACC folds the residual add
// (AddResidualKernel) into the store.  PAIR computes the fused gate|up projection's rows n and
// N + n in the same wave and stores silu(gate) * up (the SwiGLU that follows it, :424), N
// outputs from 2N weight rows.  The per-element arithmetic is the standalone kernels'; only
// the order of the RMSNorm sum of squares differs.  The row's loads, then the first batch of
// weight loads (U 16-byte chunks per lane and row: U = 4 holds a 2048-wide row, 12 a 6144-wide
// one), are issued before the row is built, so the prologue runs under the weights' HBM
// latency; longer rows ping-pong two batches.
template <int MODE, int R, bool ACC, int U, bool PAIR, int NWV = 4>
__global__ __launch_bounds__(64 * NWV) void gemv_fused_kernel(const float* x, const float* aux,
                                                         float eps,
                                                         const uint16_t* __restrict__ W,
                                                         float* __restrict__ out, int K, int N) {
#pragma clang fp contract(off)
  constexpr int RO = PAIR ? R / 2 : R;  // outputs per wave
  static_assert(!PAIR || R % 2 == 0, "paired rows");
  __shared__ __align__(16) uint16_t xs[kFusedMaxK];
  static_assert(NWV == 4 || NWV == 8, "4 or 8 waves per workgroup");
  constexpr int XS = 4 * 64 * NWV;  // input elements per pass of the workgroup (4 per thread)
  __shared__ float red[NWV];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int row0 = (blockIdx.x * NWV + wave) * RO;
  const int nchunk = K >> 3;
  const u32x4_t* wr[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int o = min(row0 + (r % RO), N - 1);
    const long row = PAIR && r >= RO ? static_cast<long>(N) + o : o;
    wr[r] = reinterpret_cast<const u32x4_t*>(W + row * K);
  }
  // The input row (and the RMSNorm gain or the SwiGLU up values) is read into registers
  // before the first batch of weight loads: loads return in issue order, so the row issued
  // after the weights would wait out their HBM latency before the prologue could start.
  constexpr int NX = (U == 4 ? 2048 : 6144) / XS;  // float4 per thread held: K <= 2048 / 6144
  constexpr bool kAux = MODE == kGemvInRmsNorm || MODE == kGemvInSwiglu;
  // Both the row and the weights are loaded without branches (indices clamped in range; the
  // values past the end are never used): a branch per load leaves the wait before the
  // prologue unable to count the loads in flight, and it then waits for the weights too.
  float4 xr[NX], ar[NX];
#pragma unroll
  for (int i = 0; i < NX; ++i) {
    const int d = min(4 * tid + XS * i, K - 4);
    xr[i] = *reinterpret_cast<const float4*>(x + d);
    if constexpr (kAux) ar[i] = *reinterpret_cast<const float4*>(aux + d);
  }
  // ACC: the residual this lane adds its output to, read now (only this launch writes these
  // rows, at its end): read after the reduction it was one more memory round trip at the end
  // of every o / down projection
  float res = 0.0f;
  if constexpr (ACC) res = out[min(row0 + min(lane, RO - 1), N - 1)];

  // the row's loads go out before the weights' (x and aux are not __restrict__, so this
  // fence also keeps the compiler from sinking them to their uses)
  asm volatile("" ::: "memory");
  u32x4_t A[U][R], Bb[U][R];
  auto load = [&](u32x4_t(&dst)[U][R], int base) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = base + 64 * u + lane;
#pragma unroll
      for (int r = 0; r < R; ++r) dst[u][r] = __builtin_nontemporal_load(wr[r] + min(c, nchunk - 1));
    }
  };
  load(A, 0);

  // ---- the bf16 input row, in LDS ----
  if constexpr (MODE == kGemvInRmsNorm) {
    float local = 0.0f;
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      const int d = 4 * tid + XS * i;
      if (d < K) {
        const float4 v = xr[i];
        local += v.x * v.x;
        local += v.y * v.y;
        local += v.z * v.z;
        local += v.w * v.w;
      }
    }
    for (int d = 4 * tid + XS * NX; d < K; d += XS) {
      const float4 v = *reinterpret_cast<const float4*>(x + d);
      local += v.x * v.x;
      local += v.y * v.y;
      local += v.z * v.z;
      local += v.w * v.w;
    }
    const float ws = wave_sum(local);
    if (lane == 0) red[wave] = ws;
    lds_barrier();
    float sum = (red[0] + red[1]) + (red[2] + red[3]);
    if constexpr (NWV == 8) sum += (red[4] + red[5]) + (red[6] + red[7]);
    const float ms = sum / static_cast<float>(K) + eps;
    const float inv = rsqrt_via_f64(ms);
    auto put = [&](int d, float4 v, float4 g) {
      *reinterpret_cast<uint2*>(xs + d) =
          make_uint2(pack_bf16x2(v.x * inv * g.x, v.y * inv * g.y),
                     pack_bf16x2(v.z * inv * g.z, v.w * inv * g.w));
    };
#pragma unroll
    for (int i = 0; i < NX; ++i)
      if (4 * tid + XS * i < K) put(4 * tid + XS * i, xr[i], ar[i]);
    for (int d = 4 * tid + XS * NX; d < K; d += XS)
      put(d, *reinterpret_cast<const float4*>(x + d), *reinterpret_cast<const float4*>(aux + d));
  } else {
    auto put = [&](int d, float4 v, float4 u) {
      if constexpr (MODE == kGemvInSwiglu) {
        *reinterpret_cast<uint2*>(xs + d) =
            make_uint2(pack_bf16x2((v.x / (1.0f + expf(-v.x))) * u.x,
                                   (v.y / (1.0f + expf(-v.y))) * u.y),
                       pack_bf16x2((v.z / (1.0f + expf(-v.z))) * u.z,
                                   (v.w / (1.0f + expf(-v.w))) * u.w));
      } else {
        *reinterpret_cast<uint2*>(xs + d) =
            make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
      }
    };
#pragma unroll
    for (int i = 0; i < NX; ++i)
      if (4 * tid + XS * i < K) put(4 * tid + XS * i, xr[i], ar[i]);
    for (int d = 4 * tid + XS * NX; d < K; d += XS)
      put(d, *reinterpret_cast<const float4*>(x + d),
          kAux ? *reinterpret_cast<const float4*>(aux + d) : make_float4(0.0f, 0.0f, 0.0f, 0.0f));
  }
  lds_barrier();

  float acc[R] = {};
  const u32x4_t* xv = reinterpret_cast<const u32x4_t*>(xs);
  auto comp = [&](const u32x4_t(&src)[U][R], int base) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = base + 64 * u + lane;
      if (c < nchunk) {
        const u32x4_t xx = xv[c];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] += dot8(src[u][r], xx);
      }
    }
  };
  constexpr int kStep = 64 * U;
  int base = 0;
  while (true) {
    if (base + kStep < nchunk) load(Bb, base + kStep);
    comp(A, base);
    base += kStep;
    if (base >= nchunk) break;
    if (base + kStep < nchunk) load(A, base + kStep);
    comp(Bb, base);
    base += kStep;
    if (base >= nchunk) break;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
  if (lane < RO && row0 + lane < N) {
    float v = acc[0], up = PAIR ? acc[RO] : 0.0f;
#pragma unroll
    for (int r = 1; r < RO; ++r)
      if (lane == r) {
        v = acc[r];
        if constexpr (PAIR) up = acc[RO + r];
      }
    if constexpr (PAIR) v = (v / (1.0f + expf(-v))) * up;
    if constexpr (ACC) v = res + v;
    out[row0 + lane] = v;
  }
}

template <int MODE, bool ACC, int U>
int launch_fused_u(const float* x, const float* aux, float eps, const uint16_t* W, float* out,
                   int K, int N, bool pair, hipStream_t s) {
  // Rows per wave and waves per workgroup: enough waves to cover the chip, one input-row
  // rebuild per workgroup.  8-wave workgroups halve the rebuilds (each re-reads the fp32 row
  // and, for RMSNorm, its gain through L2) and give the one-row waves more company per CU;
  // measured against 4-wave ones on the decode step (same box, alternating runs): qkv / o
  // 1.062 -> 1.055 ms per token, lm_head 1.056 -> 1.051, down (one 6144-wide row per wave
  // instead of two) 1.051 -> 1.038, gate|up (one gate/up pair per wave instead of two)
  // 1.038 -> 1.026.
  if (pair && U == 4) {
    // the 6144-pair gate|up projection: one pair per wave, 768 workgroups of 8 waves
    hipLaunchKernelGGL((gemv_fused_kernel<MODE, 2, ACC, U, true, 8>), dim3((N + 7) / 8),
                       dim3(512), 0, s, x, aux, eps, W, out, K, N);
  } else if (pair) {
    hipLaunchKernelGGL((gemv_fused_kernel<MODE, 2, ACC, U, true>), dim3((N + 3) / 4), dim3(256),
                       0, s, x, aux, eps, W, out, K, N);
  } else if (N >= 32768) {
    // the vocabulary-sized projection: 4 rows per wave, 32 rows per workgroup
    hipLaunchKernelGGL((gemv_fused_kernel<MODE, 4, ACC, U, false, 8>), dim3((N + 31) / 32),
                       dim3(512), 0, s, x, aux, eps, W, out, K, N);
  } else if (N >= 8192) {
    hipLaunchKernelGGL((gemv_fused_kernel<MODE, 2, ACC, U, false>), dim3((N + 7) / 8), dim3(256),
                       0, s, x, aux, eps, W, out, K, N);
  } else {
    // one row per wave, 8 rows per workgroup: the 2048-wide qkv and o projections, and the
    // 6144-wide rows of the down projection
    hipLaunchKernelGGL((gemv_fused_kernel<MODE, 1, ACC, U, false, 8>), dim3((N + 7) / 8),
                       dim3(512), 0, s, x, aux, eps, W, out, K, N);
  }
  return check_launch("gemv_fused_kernel");
}

template <int MODE, bool ACC>
int launch_fused_mode(const float* x, const float* aux, float eps, const uint16_t* W, float* out,
                      int K, int N, bool pair, hipStream_t s) {
  // one batch per row where it fits: K <= 2048 -> 4 chunks per lane, else 12 (K <= 6144)
  if (K > 2048) return launch_fused_u<MODE, ACC, 12>(x, aux, eps, W, out, K, N, pair, s);
  return launch_fused_u<MODE, ACC, 4>(x, aux, eps, W, out, K, N, pair, s);
}

// Argument checks shared by the bf16 linear entry points.  Returns the status; *generic is set
// when K is not a multiple of 8 or `in` / W are not 16-byte aligned: the GEMM then loads
// element by element (any K, as the reference's generic fallback, gemm.cuh:461-501; operands
// need only the 2-byte alignment of their element type).
int check_linear(const void* in, const uint16_t* W, const float* out, int K, int act,
                 const char* who, bool* generic) {
  if (!in || !W || !out) return fail(ORATOR_ERR_INVALID, std::string(who) + ": null pointer");
  if (act < 0 || act > 2) return fail(ORATOR_ERR_INVALID, std::string(who) + ": act must be 0-2");
  const uintptr_t al = reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(W);
  if (al & 1u)
    return fail(ORATOR_ERR_INVALID, std::string(who) + ": in and W must be 2-byte aligned");
  *generic = (K % 8) != 0 || (al & 15u) != 0;
  return ORATOR_OK;
}

}  // namespace

int launch_bf16_gemm(const uint16_t* in, const uint16_t* W, const float* bias, float* out, int M,
                     int K, int N, int act, hipStream_t stream) {
  if (M <= 0 || K <= 0 || N <= 0) return ORATOR_OK;  // reference no-op
  bool generic = false;
  if (int rc = check_linear(in, W, out, K, act, "bf16_gemm", &generic)) return rc;
  if (M == 1 && !generic) {  // one row: the weight-streaming GEMV
    const int per_wg = kGemvRows * kGemvWaves;
    hipLaunchKernelGGL(gemv_bf16_kernel, dim3((N + per_wg - 1) / per_wg), dim3(64 * kGemvWaves), 0,
                       stream, in, W, bias, out, K, N, act);
    return check_launch("gemv_bf16_kernel");
  }
  return launch_gemm_bf16_nt(in, W, bias, out, M, K, N, act, false, stream, generic);
}

int launch_gemv_fused(int mode, const float* x, const float* aux, float eps, const uint16_t* W,
                      float* out, int K, int N, bool accumulate, hipStream_t s, bool pair) {
  if (K <= 0 || N <= 0) return ORATOR_OK;
  if (!x || !W || !out || (mode != kGemvInF32 && !aux))
    return fail(ORATOR_ERR_INVALID, "gemv_fused: null pointer");
  if (K % 8 || K > kFusedMaxK)
    return fail(ORATOR_ERR_UNSUPPORTED, "gemv_fused: K must be a multiple of 8, at most 8192");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(W) |
       reinterpret_cast<uintptr_t>(aux)) & 15u)
    return fail(ORATOR_ERR_INVALID, "gemv_fused: x, aux and W must be 16-byte aligned");
  switch (mode) {
    case kGemvInF32:
      return accumulate ? launch_fused_mode<kGemvInF32, true>(x, aux, eps, W, out, K, N, pair, s)
                        : launch_fused_mode<kGemvInF32, false>(x, aux, eps, W, out, K, N, pair, s);
    case kGemvInRmsNorm:
      return accumulate
                 ? launch_fused_mode<kGemvInRmsNorm, true>(x, aux, eps, W, out, K, N, pair, s)
                 : launch_fused_mode<kGemvInRmsNorm, false>(x, aux, eps, W, out, K, N, pair, s);
    case kGemvInSwiglu:
      return accumulate
                 ? launch_fused_mode<kGemvInSwiglu, true>(x, aux, eps, W, out, K, N, pair, s)
                 : launch_fused_mode<kGemvInSwiglu, false>(x, aux, eps, W, out, K, N, pair, s);
    default:
      return fail(ORATOR_ERR_INVALID, "gemv_fused: unknown input mode");
  }
}

int launch_linear_pre(const uint16_t* in, const uint16_t* W, const float* bias, float* out, int M,
                      int K, int N, int act, hipStream_t stream) {
  return launch_bf16_gemm(in, W, bias, out, M, K, N, act, stream);
}

int launch_linear_pre_acc(const uint16_t* in, const uint16_t* W, float* out, int M, int K, int N,
                          float* tmp, hipStream_t stream) {
  if (M <= 0 || K <= 0 || N <= 0) return ORATOR_OK;
  bool generic = false;
  if (int rc = check_linear(in, W, out, K, 0, "linear_acc", &generic)) return rc;
  if (M > 1) return launch_gemm_bf16_nt(in, W, nullptr, out, M, K, N, 0, true, stream, generic);
  if (int rc = launch_bf16_gemm(in, W, nullptr, tmp, M, K, N, 0, stream)) return rc;
  return orator_add_residual(out, tmp, static_cast<long>(M) * N, stream);
}

}  // namespace orator_hip

using namespace orator_hip;

extern "C" {

int orator_linear_pre(const uint16_t* in_bf16, const uint16_t* W_bf16, const float* bias,
                      float* out, int M, int K, int N, int act, void* stream) {
  return launch_linear_pre(in_bf16, W_bf16, bias, out, M, K, N, act,
                           static_cast<hipStream_t>(stream));
}

int orator_linear_pre_swiglu(const uint16_t* in_bf16, const uint16_t* W_gateup,
                             uint16_t* out_bf16, int M, int K, int I, void* stream) {
  if (M <= 0 || K <= 0 || I <= 0) return ORATOR_OK;
  if (!out_bf16) return fail(ORATOR_ERR_INVALID, "linear_pre_swiglu: null pointer");
  if (I % 4) return fail(ORATOR_ERR_UNSUPPORTED, "linear_pre_swiglu: I must be a multiple of 4");
  bool generic = false;
  if (int rc = check_linear(in_bf16, W_gateup, reinterpret_cast<const float*>(out_bf16), K, 0,
                            "linear_pre_swiglu", &generic))
    return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  // the fp32 gate|up block is materialised (in the stream's workspace) only by the M = 1,
  // any-K and short-grid paths
  if (M == 1 || generic) {
    float* tmp =
        static_cast<float*>(workspace(s, 2 * static_cast<size_t>(M) * I * sizeof(float)));
    if (!tmp) return ORATOR_ERR_HIP;
    if (int rc = launch_bf16_gemm(in_bf16, W_gateup, nullptr, tmp, M, K, 2 * I, 0, s)) return rc;
    return launch_swiglu_bf16(tmp, out_bf16, M, I, s);
  }
  return launch_gemm_bf16_swiglu(in_bf16, W_gateup, out_bf16, nullptr, M, K, I, s);
}

int orator_linear(const float* in_f32, const uint16_t* W_bf16, const float* bias, float* out,
                  int M, int K, int N, int act, void* stream) {
  if (M <= 0 || K <= 0 || N <= 0) return ORATOR_OK;
  if (!in_f32) return fail(ORATOR_ERR_INVALID, "linear: null pointer");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const long n = static_cast<long>(M) * K;
  uint16_t* in_bf16 = static_cast<uint16_t*>(workspace(s, n * sizeof(uint16_t)));
  if (!in_bf16) return ORATOR_ERR_HIP;
  if (int rc = orator_f32_to_bf16(in_f32, in_bf16, n, stream)) return rc;
  return launch_linear_pre(in_bf16, W_bf16, bias, out, M, K, N, act, s);
}

int orator_bf16_gemm(const uint16_t* in_bf16, const uint16_t* W_bf16, const float* bias,
                     float* out, int M, int K, int N, int act, void* stream) {
  return launch_bf16_gemm(in_bf16, W_bf16, bias, out, M, K, N, act,
                          static_cast<hipStream_t>(stream));
}

}  // extern "C"
