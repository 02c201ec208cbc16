// bf16 GEMM with fp32 accumulation and output for prompt-sized products, gfx950:
// out[M][N] (=|+=) act(in[M][K] W[N][K]^T + bias).
//
// Replaces the tiled tensor-core GEMM behind gemm::LaunchBf16Gemm and asr_gemm::LinearPre for
// M > 1 (include/model/gemm.cuh:384-501, src/model/asr_gemm.cu:175-208).  Both operands are
// K-contiguous, which is the fragment order of v_mfma_f32_32x32x16_bf16 (lane = row, 8
// consecutive k per lane), so tiles go from HBM to LDS row by row and back out as fragments
// without any transpose.
//
// Workgroup = BM x BN output tile, 4 waves in a 2 x 2 grid, each wave (BM/2) x (BN/2) =
// (BM/64) x (BN/64) blocks of 32 x 32 accumulators.  K advances 64 at a time through two LDS
// buffers (rows padded to 72 elements = 144 bytes, which puts the 16 rows a quarter-wave reads
// on 16 distinct 16-byte bank groups); the next K tile is loaded into registers while the
// current one is multiplied and stored after it, one barrier per step.  Larger wave tiles
// reuse each fragment read from LDS for more MFMAs (128 x 128 per wave: 8 fragment reads per
// 16 MFMAs); the tile shape is chosen per problem so the grid covers the 256 CUs.
#include <stdlib.h>

#include <algorithm>
#include <string>

#include "common.hpp"
#include "internal.hpp"

namespace orator_hip {
namespace {

typedef __bf16 gb_bf16x8_t __attribute__((ext_vector_type(8)));
typedef float gb_f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t gb_u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBK = 64;        // K per step
constexpr int kLdk = kBK + 8;  // padded LDS row (bf16 elements)

__device__ __forceinline__ float gb_act(float v, int act) {
  if (act == 1) return 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f));
  if (act == 2) return fmaxf(v, 0.0f);
  return v;
}

template <int BM, int BN, int WGM, int WGN>
__global__ __launch_bounds__(64 * WGM * WGN, 1) void gemm_bf16_nt_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ W,
    const float* __restrict__ bias, float* __restrict__ C, int M, int K, int N, int act,
    int accumulate, float* __restrict__ part, int k_split) {
  constexpr int NT = 64 * WGM * WGN;               // threads
  constexpr int TM = BM / WGM, TN = BN / WGN;      // wave tile
  constexpr int FM = TM / 32, FN = TN / 32;        // 32 x 32 blocks per wave
  constexpr int RPI = NT / 8;                      // rows per load instruction
  constexpr int LA = BM / RPI, LW = BN / RPI;      // 16-byte loads per thread per K step
  __shared__ __align__(16) uint16_t sA[2][BM][kLdk];
  __shared__ __align__(16) uint16_t sW[2][BN][kLdk];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  // Tile order: workgroups are handed to the 8 XCDs in turn, so workgroup b runs on XCD b % 8.
  // Give each XCD a contiguous range of a row-grouped tile order (groups of 4 tile rows, down
  // the rows then across), so the tiles sharing one XCD's L2 share their A rows and W rows.
  const int tiles_n = gridDim.x, tiles_m = gridDim.y;
  const int total = tiles_n * tiles_m;
  int L = blockIdx.x + tiles_n * blockIdx.y;
  if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
  constexpr int kGroup = 4;
  const int group = L / (kGroup * tiles_n);
  const int first_m = group * kGroup;
  const int gm = min(tiles_m - first_m, kGroup);
  const int in_group = L - group * kGroup * tiles_n;
  const int m0 = (first_m + in_group % gm) * BM, n0 = (in_group / gm) * BN;
  // loader: 32 rows x 128 bytes per instruction, thread = (row tid / 8, 16-byte chunk tid % 8)
  const int lr = tid >> 3, lc = tid & 7;
  gb_u32x4_t ra[LA], rw[LW];
  const long ld = K;  // row stride of A and W (elements)
  int k_lim = K;      // set below for the split
  auto load = [&](int k0) {
    const int kk = k0 + 8 * lc;
    const bool k_ok = kk < k_lim;
#pragma unroll
    for (int i = 0; i < LA; ++i) {
      const int m = m0 + RPI * i + lr;
      ra[i] = (m < M && k_ok) ? *reinterpret_cast<const gb_u32x4_t*>(A + m * ld + kk)
                              : gb_u32x4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < LW; ++i) {
      const int n = n0 + RPI * i + lr;
      rw[i] = (n < N && k_ok) ? *reinterpret_cast<const gb_u32x4_t*>(W + n * ld + kk)
                              : gb_u32x4_t{0, 0, 0, 0};
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < LA; ++i)
      *reinterpret_cast<gb_u32x4_t*>(&sA[buf][RPI * i + lr][8 * lc]) = ra[i];
#pragma unroll
    for (int i = 0; i < LW; ++i)
      *reinterpret_cast<gb_u32x4_t*>(&sW[buf][RPI * i + lr][8 * lc]) = rw[i];
  };

  gb_f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int fr = lane & 31, fk = 8 * (lane >> 5);
  // split-K: workgroup z covers k in [z * k_split, (z + 1) * k_split) (k_split a multiple of
  // kBK) and leaves its raw partial sums in part[z]
  const int kb = blockIdx.z * k_split;
  const int n_k = (min(K, kb + k_split) - kb + kBK - 1) / kBK;
  A += kb;
  W += kb;
  k_lim = min(K - kb, k_split);
  load(0);
  store(0);
  lds_barrier();
  for (int t = 0; t < n_k; ++t) {
    const int buf = t & 1;
    if (t + 1 < n_k) load((t + 1) * kBK);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      // the next tile's rows go to the other buffer half way through (its loads have long
      // arrived; nobody reads that buffer during this step)
      if (ks == kBK / 32 && t + 1 < n_k) store(buf ^ 1);
      gb_bf16x8_t fa[FM], fb[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        fa[i] = __builtin_bit_cast(
            gb_bf16x8_t, *reinterpret_cast<const gb_u32x4_t*>(
                             &sA[buf][wm * TM + 32 * i + fr][16 * ks + fk]));
#pragma unroll
      for (int j = 0; j < FN; ++j)
        fb[j] = __builtin_bit_cast(
            gb_bf16x8_t, *reinterpret_cast<const gb_u32x4_t*>(
                             &sW[buf][wn * TN + 32 * j + fr][16 * ks + fk]));
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    lds_barrier();
  }

  // block (i, j): lane holds column n = 32 j + lane % 32 and rows 8 (e / 4) + 4 (lane / 32) +
  // e % 4 of the block
  if (part) {
    float* P = part + static_cast<long>(blockIdx.z) * M * N;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = n0 + wn * TN + 32 * j + fr;
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m0 + wm * TM + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
          if (m < M) P[static_cast<long>(m) * N + n] = acc[i][j][e];
        }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int n = n0 + wn * TN + 32 * j + fr;
    if (n >= N) continue;
    const float bv = bias ? bias[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * TM + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        if (m < M) {
          float* o = C + static_cast<long>(m) * N + n;
          const float v = gb_act(acc[i][j][e] + bv, act);
          *o = accumulate ? *o + v : v;
        }
      }
  }
}

// out[m][n] (= or +=) act(sum_z part[z][m][n] + bias[n]), z ascending (a fixed order).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part,
                                                            int splits, const float* __restrict__ bias,
                                                            float* __restrict__ out, long MN, int N,
                                                            int act, int accumulate) {
  const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= MN) return;
  float v = part[i];
  for (int z = 1; z < splits; ++z) v += part[z * MN + i];
  v = gb_act(v + (bias ? bias[i % N] : 0.0f), act);
  out[i] = accumulate ? out[i] + v : v;
}

template <int BM, int BN, int WGM, int WGN>
int launch_tile(const uint16_t* in, const uint16_t* W, const float* bias, float* out, int M,
                int K, int N, int act, bool accumulate, int splits, hipStream_t s) {
  const int k_split = splits > 1 ? ((K + splits - 1) / splits + kBK - 1) / kBK * kBK : K;
  if (splits > 1) splits = (K + k_split - 1) / k_split;
  float* part = nullptr;
  const long MN = static_cast<long>(M) * N;
  if (splits > 1) {
    part = static_cast<float*>(
        workspace(s, static_cast<size_t>(splits) * MN * sizeof(float), kWsGemm));
    if (!part) return ORATOR_ERR_HIP;
  }
  const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM, splits);
  hipLaunchKernelGGL((gemm_bf16_nt_kernel<BM, BN, WGM, WGN>), grid, dim3(64 * WGM * WGN), 0, s,
                     in, W, bias, out, M, K, N, act, accumulate ? 1 : 0, part, k_split);
  if (int rc = check_launch("gemm_bf16_nt_kernel")) return rc;
  if (splits == 1) return ORATOR_OK;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(static_cast<unsigned>((MN + 255) / 256)),
                     dim3(256), 0, s, part, splits, bias, out, MN, N, act, accumulate ? 1 : 0);
  return check_launch("splitk_reduce_kernel");
}

}  // namespace

// Tile shape by grid size: 8 waves per workgroup (two per SIMD) on the largest tile whose grid
// still gives every CU a workgroup; when even 128 x 128 tiles leave CUs idle and K is long, K
// is split over workgroups (partials reduced in a fixed order: deterministic).
int launch_gemm_bf16_nt(const uint16_t* in, const uint16_t* W, const float* bias, float* out,
                        int M, int K, int N, int act, bool accumulate, hipStream_t s) {
  if (M <= 0 || K <= 0 || N <= 0) return ORATOR_OK;
  const long cus = device_cu_count() > 0 ? device_cu_count() : 256;
  auto tiles = [&](int bm, int bn) {
    return static_cast<long>((M + bm - 1) / bm) * ((N + bn - 1) / bn);
  };
  if (tiles(256, 256) >= cus)
    return launch_tile<256, 256, 2, 4>(in, W, bias, out, M, K, N, act, accumulate, 1, s);
  if (tiles(256, 128) >= cus)
    return launch_tile<256, 128, 4, 2>(in, W, bias, out, M, K, N, act, accumulate, 1, s);
  const long t = tiles(128, 128);
  int splits = 1;
  if (t < cus) splits = static_cast<int>(std::min<long>((cus + t - 1) / t, std::max(1, K / 512)));
  return launch_tile<128, 128, 2, 4>(in, W, bias, out, M, K, N, act, accumulate, splits, s);
}

}  // namespace orator_hip
