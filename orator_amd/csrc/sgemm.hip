// fp32 GEMM on fp32 MFMA (gfx950): out[M,N] = act(sum_k in[m,k] * W[n,k] (+ bias[n])).
//
// Replaces gemm::LaunchSgemm / LaunchSgemmBatched (include/model/gemm.cuh:47-268): the same
// nn.Linear "NT" contract (both operands K-contiguous), activation codes 0 none, 1 SiLU,
// 2 ReLU, 3 sigmoid (gemm.cuh:38-45), strided batches, arbitrary M/N/K and alignment
// (guarded loads, as SgemmBatchedKernel).  Products are exact fp32 and accumulate in fp32
// on v_mfma_f32_32x32x2_f32, so results stay within fp32 rounding of the reference's
// k-sequential FMA chains.
//
// Products of at least 32 rows run on hipBLASLt (blaslt_gemm.cpp; fp32 compute, bias and
// activation in one pass after it); the kernel below serves smaller products and shapes the
// library has no plan for.
//
// Tiling: a workgroup of 4 wave64s computes a 64x64 output tile (2x2 waves of 32x32);
// 64x16 slices of both operands are staged through padded LDS (row stride 17 floats, so
// the 32 rows an MFMA operand load touches fall in distinct banks).
#include "common.hpp"
#include "internal.hpp"

namespace orator_hip {
namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kTile = 64;
constexpr int kBK = 16;

__device__ __forceinline__ float apply_act(float v, int act) {
  if (act == 1) return v / (1.0f + expf(-v));
  if (act == 2) return fmaxf(v, 0.0f);
  if (act == 3) return 1.0f / (1.0f + expf(-v));
  return v;
}

__global__ __launch_bounds__(256) void sgemm_nt_kernel(const float* __restrict__ in,
                                                       const float* __restrict__ W,
                                                       const float* __restrict__ bias,
                                                       float* __restrict__ out, int M, int K,
                                                       int N, int act, long stride_in,
                                                       long stride_w, long stride_out) {
  __shared__ float As[kTile][kBK + 1];
  __shared__ float Bs[kTile][kBK + 1];
  const int b = blockIdx.z;
  const float* A = in + b * stride_in;
  const float* Bm = W + b * stride_w;
  float* C = out + b * stride_out;
  const int m0 = blockIdx.y * kTile;
  const int n0 = blockIdx.x * kTile;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lrow = tid >> 2;        // 0..63: tile row this thread stages
  const int lk = (tid & 3) * 4;     // 4 consecutive k
  const bool vec = (K & 3) == 0 && ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(Bm)) & 15) == 0;

  f32x16_t acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.0f;

  for (int k0 = 0; k0 < K; k0 += kBK) {
    float av[4], bv[4];
    const int gm = m0 + lrow, gn = n0 + lrow, gk = k0 + lk;
    if (vec && gk + 3 < K) {
      const float4 a4 = gm < M ? *reinterpret_cast<const float4*>(A + static_cast<long>(gm) * K + gk)
                               : make_float4(0, 0, 0, 0);
      const float4 b4 = gn < N ? *reinterpret_cast<const float4*>(Bm + static_cast<long>(gn) * K + gk)
                               : make_float4(0, 0, 0, 0);
      av[0] = a4.x; av[1] = a4.y; av[2] = a4.z; av[3] = a4.w;
      bv[0] = b4.x; bv[1] = b4.y; bv[2] = b4.z; bv[3] = b4.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        av[e] = (gm < M && gk + e < K) ? A[static_cast<long>(gm) * K + gk + e] : 0.0f;
        bv[e] = (gn < N && gk + e < K) ? Bm[static_cast<long>(gn) * K + gk + e] : 0.0f;
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      As[lrow][lk + e] = av[e];
      Bs[lrow][lk + e] = bv[e];
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 2) {
      const float a = As[32 * wm + (lane & 31)][kk + (lane >> 5)];
      const float bb = Bs[32 * wn + (lane & 31)][kk + (lane >> 5)];
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, bb, acc, 0, 0, 0);
    }
    __syncthreads();
  }
  // accumulator layout: acc[4i + j] -> row 8i + 4*(lane/32) + j, column lane % 32
  const int n = n0 + 32 * wn + (lane & 31);
  if (n >= N) return;
  const float bn = bias ? bias[n] : 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + 32 * wm + 8 * i + 4 * (lane >> 5) + j;
      if (m < M) {
        float v = acc[4 * i + j];
        if (bias) v += bn;
        C[static_cast<long>(m) * N + n] = apply_act(v, act);
      }
    }
}

// out_b[m][n] = act(out_b[m][n] + bias[n]) after a library GEMM.
__global__ __launch_bounds__(256) void sgemm_bias_act_kernel(float* __restrict__ out,
                                                             const float* __restrict__ bias,
                                                             int M, int N, int act, long per,
                                                             long stride_out, long total) {
  const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const long b = i / per, r = i - b * per;
  float* o = out + b * stride_out + r;
  const float v = *o + (bias ? bias[r % N] : 0.0f);
  *o = apply_act(v, act);
}

}  // namespace

int launch_sgemm(const float* in, const float* W, const float* bias, float* out, int M, int K,
                 int N, int act, int batch, long stride_in, long stride_w, long stride_out,
                 hipStream_t stream) {
  if (M <= 0 || N <= 0 || K <= 0 || batch <= 0) return ORATOR_OK;
  if (!in || !W || !out) return fail(ORATOR_ERR_INVALID, "sgemm: null pointer");
  if (act < 0 || act > 3) return fail(ORATOR_ERR_INVALID, "sgemm: act must be 0..3");
  // Products of at least kLibMinM rows: the GEMM library (exact fp32 products), then bias and
  // activation in one pass; shapes it has no plan for run the kernel above.
  if (M >= kLibMinM && bf16_gemm_lib_enabled()) {
    const long s_in = batch > 1 ? stride_in : 0, s_w = batch > 1 ? stride_w : 0,
               s_out = batch > 1 ? stride_out : 0;
    const int rc = launch_f32_gemm_lib(in, W, out, M, K, N, batch, s_in, s_w, s_out, stream);
    if (rc == ORATOR_OK) {
      if (!bias && act == 0) return ORATOR_OK;
      const long per = static_cast<long>(M) * N, total = per * batch;
      hipLaunchKernelGGL(sgemm_bias_act_kernel, dim3(static_cast<unsigned>((total + 255) / 256)),
                         dim3(256), 0, stream, out, bias, M, N, act, per,
                         batch > 1 ? stride_out : per, total);
      return check_launch("sgemm_bias_act");
    }
    if (rc != ORATOR_ERR_UNSUPPORTED) return rc;
  }
  const dim3 grid((N + kTile - 1) / kTile, (M + kTile - 1) / kTile, batch);
  hipLaunchKernelGGL(sgemm_nt_kernel, grid, dim3(256), 0, stream, in, W, bias, out, M, K, N, act,
                     stride_in, stride_w, stride_out);
  return check_launch("sgemm");
}

}  // namespace orator_hip

using namespace orator_hip;

extern "C" {

int orator_sgemm(const float* in, const float* W, const float* bias, float* out, int M, int K,
                 int N, int act, void* stream) {
  return launch_sgemm(in, W, bias, out, M, K, N, act, 1, 0, 0, 0, static_cast<hipStream_t>(stream));
}

int orator_sgemm_batched(const float* in, const float* W, float* out, int M, int K, int N, int act,
                         int batch, long stride_in, long stride_w, long stride_out, void* stream) {
  return launch_sgemm(in, W, nullptr, out, M, K, N, act, batch, stride_in, stride_w, stride_out,
                      static_cast<hipStream_t>(stream));
}

}  // extern "C"
