// bf16 GEMM with fp32 accumulation and output for prompt-sized products, gfx950:
// out[M][N] (=|+=) act(in[M][K] W[N][K]^T + bias).
//
// Replaces the tiled tensor-core GEMM behind gemm::LaunchBf16Gemm and asr_gemm::LinearPre for
// M > 1 (include/model/gemm.cuh:384-501, src/model/asr_gemm.cu:175-208).  Both operands are
// K-contiguous, which is the fragment order of v_mfma_f32_32x32x16_bf16 (lane = row, 8
// consecutive k per lane), so tiles go from HBM to LDS row by row and back out as fragments
// without any transpose.
//
// Workgroup = BM x BN output tile, 4 waves (one per SIMD) in a WGM x WGN grid, each wave
// (BM/WGM) x (BN/WGN) = FM x FN blocks of 32 x 32 accumulators, two workgroups per CU (73.7 KB
// of LDS each), so one workgroup's epilogue and barrier waits overlap the other's MFMAs.  K
// advances 64 at a time through two LDS buffers (rows padded to 72 elements = 144 bytes,
// which puts the 16 rows a quarter-wave reads on 16 distinct 16-byte bank groups); the next K
// tile is loaded into registers during the current step and stored to the other buffer
// before the step's last MFMAs, the next 16-deep fragments are read from LDS under the
// current ones' MFMAs, one barrier per step.  Rows past M / N load the last valid row (their
// outputs are never stored) and k chunks past K are zeroed by a mask on the last step, so the
// loads carry no branches.  128 x 128 tiles when they give every CU two workgroups, else
// 128 x 64, with K split over workgroups when even those leave CUs idle.  (Measured
// alternatives: 256 x 256 and 256 x 128 tiles with 8 waves, one workgroup per CU, were
// 25-55 % slower at the decoder's prompt shapes: their grids quantize badly on 256 CUs and
// their epilogue is not overlapped; K = 32 steps with 3-4 workgroups per CU were 10-35 %
// slower.)
#include <stdlib.h>

#include <algorithm>
#include <string>
#include <type_traits>

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

// Epilogues: raw split-K partials, out = acc (no bias), out += acc + bias, the general
// out (= or +=) act(acc + bias), and SwiGLU: W holds gate rows [0, I) then up rows [I, 2I)
// (N = 2I); a tile takes BN/2 gate rows and the matching BN/2 up rows, and stores
// bf16(silu(gate) * up) for its BN/2 columns of the [M][I] bf16 output.
constexpr int kEpiPartial = 0, kEpiStore = 1, kEpiAccumulate = 2, kEpiAct = 3, kEpiSwiglu = 4;

template <int BM, int BN, int WGM, int WGN, int MINW, int EPI, bool GEN = false>
__global__ __launch_bounds__(64 * WGM * WGN, MINW) void gemm_bf16_nt_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ W,
    const float* __restrict__ bias, float* __restrict__ C, int M, int K, int N, int act,
    int accumulate, float* __restrict__ part, int k_split) {
  constexpr int NT = 64 * WGM * WGN;               // threads
  constexpr int TM = BM / WGM, TN = BN / WGN;      // wave tile
  constexpr int FM = TM / 32, FN = TN / 32;        // 32 x 32 blocks per wave
  constexpr int RPI = NT / 8;                      // rows per load instruction
  constexpr int LA = BM / RPI, LW = BN / RPI;      // 16-byte loads per thread per K step
  constexpr int KS = kBK / 16;                     // MFMA k-steps per K step
  // LDS: the double-buffered A and W tiles during the K loop, then the fp32 output tile (rows
  // padded by 8 floats: lanes 0-31 and 32-63 of an accumulator store, 4 rows apart, land 32
  // banks apart)
  constexpr int kCLd = BN + 8;
  constexpr int kTileBytes = 2 * (BM + BN) * kLdk * 2;
  constexpr int kOutBytes = BM * kCLd * 4;
  __shared__ __align__(16) unsigned char smem[kTileBytes > kOutBytes ? kTileBytes : kOutBytes];
  auto sA = reinterpret_cast<uint16_t(*)[BM][kLdk]>(smem);
  auto sW = reinterpret_cast<uint16_t(*)[BN][kLdk]>(smem + 2 * BM * kLdk * 2);
  auto sC = reinterpret_cast<float(*)[kCLd]>(smem);

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

  // split-K: workgroup z covers k in [z * k_split, (z + 1) * k_split) (k_split a multiple of
  // kBK) and leaves its raw partial sums in part[z]
  const int kb = blockIdx.z * k_split;
  const int k_lim = min(K - kb, k_split);  // a multiple of 8 unless GEN
  const int n_k = (k_lim + kBK - 1) / kBK;
  A += kb;
  W += kb;
  // loader: 32 rows x 128 bytes per instruction, thread = (row tid / 8, 16-byte chunk tid % 8);
  // rows clamped into range, chunks past k_lim read in range and masked to zero
  const int lr = tid >> 3, lc = tid & 7;
  const long ld = K;  // row stride of A and W (elements)
  const uint16_t* arow[LA];
  const uint16_t* wrow[LW];
#pragma unroll
  for (int i = 0; i < LA; ++i) arow[i] = A + min(m0 + RPI * i + lr, M - 1) * ld;
#pragma unroll
  for (int i = 0; i < LW; ++i) {
    const int j = RPI * i + lr;  // tile row
    long row;
    if constexpr (EPI == kEpiSwiglu) {
      const int I = N / 2, c0 = (n0 / BN) * (BN / 2);
      row = j < BN / 2 ? min(c0 + j, I - 1) : I + min(c0 + j - BN / 2, I - 1);
    } else {
      row = min(n0 + j, N - 1);
    }
    wrow[i] = W + row * ld;
  }
  gb_u32x4_t ra[LA], rw[LW];
  uint32_t keep = 0;  // mask of the chunk in flight; applied at the LDS store, and only on the
                      // last K step when k_lim is not a multiple of kBK (a uniform branch)
  // GEN (any K, rows at any 2-byte alignment): the chunk's 8 elements are loaded one by one,
  // elements past k_lim read as zero, so nothing is masked at the store.
  auto load8 = [&](const uint16_t* row, int kk) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t lo = kk + 2 * e < k_lim ? row[kk + 2 * e] : 0u;
      const uint32_t hi = kk + 2 * e + 1 < k_lim ? row[kk + 2 * e + 1] : 0u;
      w[e] = lo | (hi << 16);
    }
    return gb_u32x4_t{w[0], w[1], w[2], w[3]};
  };
  auto load = [&](int k0) {
    const int kk = k0 + 8 * lc;
    if constexpr (GEN) {
#pragma unroll
      for (int i = 0; i < LA; ++i) ra[i] = load8(arow[i], kk);
#pragma unroll
      for (int i = 0; i < LW; ++i) rw[i] = load8(wrow[i], kk);
    } else {
      const int kc = min(kk, k_lim - 8);
      keep = kk < k_lim ? 0xffffffffu : 0u;
#pragma unroll
      for (int i = 0; i < LA; ++i) ra[i] = *reinterpret_cast<const gb_u32x4_t*>(arow[i] + kc);
#pragma unroll
      for (int i = 0; i < LW; ++i) rw[i] = *reinterpret_cast<const gb_u32x4_t*>(wrow[i] + kc);
    }
  };
  const bool ragged = !GEN && (k_lim % kBK) != 0;
  auto store = [&](int buf, bool masked) {
    if (masked) {
#pragma unroll
      for (int i = 0; i < LA; ++i) ra[i] &= keep;
#pragma unroll
      for (int i = 0; i < LW; ++i) rw[i] &= keep;
    }
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
  load(0);
  store(0, ragged && n_k == 1);
  lds_barrier();
  for (int t = 0; t < n_k; ++t) {
    const int buf = t & 1;
    if (t + 1 < n_k) load((t + 1) * kBK);
    gb_bf16x8_t fa[2][FM], fb[2][FN];
    auto read = [&](int ks, int s) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
        fa[s][i] = __builtin_bit_cast(
            gb_bf16x8_t, *reinterpret_cast<const gb_u32x4_t*>(
                             &sA[buf][wm * TM + 32 * i + fr][16 * ks + fk]));
#pragma unroll
      for (int j = 0; j < FN; ++j)
        fb[s][j] = __builtin_bit_cast(
            gb_bf16x8_t, *reinterpret_cast<const gb_u32x4_t*>(
                             &sW[buf][wn * TN + 32 * j + fr][16 * ks + fk]));
    };
    read(0, 0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int s = ks & 1;
      if (ks + 1 < KS) read(ks + 1, s ^ 1);
      // the next tile's rows go to the other buffer before the last k-step's MFMAs (nobody
      // reads that buffer during this step)
      if (ks == KS - 1 && t + 1 < n_k) store(buf ^ 1, ragged && t + 2 == n_k);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[s][i], fb[s][j], acc[i][j], 0, 0, 0);
    }
    lds_barrier();
  }

  // Plain stores (no bias) and split-K partials: straight from the accumulators (block (i, j):
  // lane holds column 32 j + lane % 32 and rows 8 (e / 4) + 4 (lane / 32) + e % 4 of the
  // block); nothing is loaded, so the stores never wait.
  if constexpr (EPI == kEpiStore || EPI == kEpiPartial) {
    float* out = C;
    if constexpr (EPI == kEpiPartial) out = part + static_cast<long>(blockIdx.z) * M * N;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = n0 + wn * TN + 32 * j + fr;
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m0 + wm * TM + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
          if (m < M) out[static_cast<long>(m) * N + n] = acc[i][j][e];
        }
    }
    return;
  }
  // Bias, activation or accumulate: through LDS.  The accumulators go to the fp32 tile in LDS
  // (same lane mapping), then the workgroup writes the tile out row by row in 16-byte pieces.  An accumulating
  // epilogue loads all its old values before its first store: stores count against the same
  // wait counter as loads, so a load issued behind stores would wait for them too.
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        sC[wm * TM + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)][wn * TN + 32 * j + fr] =
            acc[i][j][e];
  __syncthreads();

  if constexpr (EPI == kEpiSwiglu) {
    // 4 output columns per thread: gate from tile column c, up from column BN/2 + c; the
    // arithmetic of the standalone SwiGLU + cast (silu(g) * u in fp32, bf16 round to nearest
    // even), so the result is bit-identical to GEMM -> SwiGLU -> F32ToBf16
    const int I = N / 2, c0 = (n0 / BN) * (BN / 2);
    uint16_t* ob = reinterpret_cast<uint16_t*>(C);
    constexpr int TPRs = BN / 8;  // threads per output row
    constexpr int RPIs = NT / TPRs;
    const int srow = tid / TPRs, scol = 4 * (tid % TPRs);
    const int col = c0 + scol;
    const bool vec8 = (I % 4) == 0 && (reinterpret_cast<uintptr_t>(ob) & 7) == 0;
#pragma unroll
    for (int p = 0; p < BM / RPIs; ++p) {
      const int r = RPIs * p + srow;
      const int m = m0 + r;
      const float4 g = *reinterpret_cast<const float4*>(&sC[r][scol]);
      const float4 u = *reinterpret_cast<const float4*>(&sC[r][BN / 2 + scol]);
      const float y0 = (g.x / (1.0f + expf(-g.x))) * u.x, y1 = (g.y / (1.0f + expf(-g.y))) * u.y;
      const float y2 = (g.z / (1.0f + expf(-g.z))) * u.z, y3 = (g.w / (1.0f + expf(-g.w))) * u.w;
      if (m >= M) continue;
      uint16_t* dst = ob + static_cast<long>(m) * I + col;
      if (vec8 && col + 3 < I) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(y0, y1), pack_bf16x2(y2, y3));
      } else {
        const float y[4] = {y0, y1, y2, y3};
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (col + q < I) dst[q] = f32_to_bf16(y[q]);
      }
    }
    return;
  }
  float* out = C;
  constexpr int TPRo = BN / 4;            // threads per output row (4 floats each)
  constexpr int RPIo = NT / TPRo;         // rows per pass
  constexpr int PASSES = BM / RPIo;
  const int orow = tid / TPRo, ocol = 4 * (tid % TPRo);
  const int n = n0 + ocol;
  const bool vec = (N % 4) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  const bool add_old = EPI == kEpiAccumulate || (EPI == kEpiAct && accumulate);
  float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (bias) {
#pragma unroll
    for (int q = 0; q < 4; ++q) bv[q] = bias[min(n + q, N - 1)];
  }
  float old[PASSES][4];
  if (add_old) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const float* src = out + static_cast<long>(min(m0 + RPIo * p + orow, M - 1)) * N;
#pragma unroll
      for (int q = 0; q < 4; ++q) old[p][q] = src[min(n + q, N - 1)];
    }
  }
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int r = RPIo * p + orow;
    const int m = m0 + r;
    const float4 c = *reinterpret_cast<const float4*>(&sC[r][ocol]);
    float v[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[q] += bv[q];
      if constexpr (EPI == kEpiAct) v[q] = gb_act(v[q], act);
      if (add_old) v[q] += old[p][q];
    }
    if (m >= M) continue;
    float* dst = out + static_cast<long>(m) * N + n;
    if (vec && n + 3 < N) {
      *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (n + q < N) dst[q] = v[q];
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

template <int BM, int BN, int WGM, int WGN, int MINW, bool GEN>
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
  const dim3 block(64 * WGM * WGN);
  const int acc = accumulate ? 1 : 0;
  if (splits > 1)
    hipLaunchKernelGGL((gemm_bf16_nt_kernel<BM, BN, WGM, WGN, MINW, kEpiPartial, GEN>), grid,
                       block, 0, s, in, W, bias, out, M, K, N, act, acc, part, k_split);
  else if (act != 0 || (bias && !accumulate))
    hipLaunchKernelGGL((gemm_bf16_nt_kernel<BM, BN, WGM, WGN, MINW, kEpiAct, GEN>), grid, block,
                       0, s, in, W, bias, out, M, K, N, act, acc, part, k_split);
  else if (accumulate)
    hipLaunchKernelGGL((gemm_bf16_nt_kernel<BM, BN, WGM, WGN, MINW, kEpiAccumulate, GEN>), grid,
                       block, 0, s, in, W, bias, out, M, K, N, act, acc, part, k_split);
  else
    hipLaunchKernelGGL((gemm_bf16_nt_kernel<BM, BN, WGM, WGN, MINW, kEpiStore, GEN>), grid, block,
                       0, s, in, W, bias, out, M, K, N, act, acc, part, k_split);
  if (int rc = check_launch("gemm_bf16_nt_kernel")) return rc;
  if (splits == 1) return ORATOR_OK;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(static_cast<unsigned>((MN + 255) / 256)),
                     dim3(256), 0, s, part, splits, bias, out, MN, N, act, acc);
  return check_launch("splitk_reduce_kernel");
}

}  // namespace

// out[M][I] bf16 = bf16(silu(in W_gate^T) * (in W_up^T)), W = [gate; up] of 2I rows: the
// gate|up projection with SwiGLU and the bf16 cast in its epilogue.  Grids too short for the
// CUs (small M) take the plain GEMM (split K) into `tmp` ([M][2I] fp32; the stream's workspace
// when null) and the standalone SwiGLU pass instead: the same values either way.
int launch_gemm_bf16_swiglu(const uint16_t* in, const uint16_t* W, uint16_t* out, float* tmp,
                            int M, int K, int I, hipStream_t s) {
  if (M <= 0 || K <= 0 || I <= 0) return ORATOR_OK;
  const long cus = device_cu_count() > 0 ? device_cu_count() : 256;
  const long tiles = static_cast<long>((M + 127) / 128) * ((I + 63) / 64);
  if (tiles < cus) {
    if (!tmp) tmp = static_cast<float*>(workspace(s, static_cast<size_t>(M) * 2 * I * sizeof(float)));
    if (!tmp) return ORATOR_ERR_HIP;
    if (int rc = launch_gemm_bf16_nt(in, W, nullptr, tmp, M, K, 2 * I, 0, false, s)) return rc;
    return launch_swiglu_bf16(tmp, out, M, I, s);
  }
  const dim3 grid(static_cast<unsigned>((I + 63) / 64), static_cast<unsigned>((M + 127) / 128), 1);
  hipLaunchKernelGGL((gemm_bf16_nt_kernel<128, 128, 2, 2, 2, kEpiSwiglu>), grid, dim3(256), 0, s,
                     in, W, nullptr, reinterpret_cast<float*>(out), M, K, 2 * I, 0, 0, nullptr, K);
  return check_launch("gemm_bf16_nt_kernel (swiglu)");
}

// Tile shape by grid size: 128 x 128 when that grid gives every CU two workgroups, else
// 128 x 64 (always for `generic`: K not a multiple of 8 or rows not 16-byte aligned, loaded
// element by element); when even that leaves CUs idle and K is long, K is split over workgroups (partials
// reduced in a fixed order: deterministic).  Measured at the 503-row prompt shapes: 128 x 64 unsplit
// beats a K split whenever its grid covers the CUs (qkv, 21.7 vs 23.7 us); below that, splits
// to two workgroups per CU beat one (down projection, 28.4 vs 36.8 us).
int launch_gemm_bf16_nt(const uint16_t* in, const uint16_t* W, const float* bias, float* out,
                        int M, int K, int N, int act, bool accumulate, hipStream_t s,
                        bool generic) {
  if (M <= 0 || K <= 0 || N <= 0) return ORATOR_OK;
  const long cus = device_cu_count() > 0 ? device_cu_count() : 256;
  auto tiles = [&](int bm, int bn) {
    return static_cast<long>((M + bm - 1) / bm) * ((N + bn - 1) / bn);
  };
  // 128 x 128 only when every CU gets two of them (one workgroup per CU leaves its epilogue
  // exposed: the decoder's 2048 x 2048 -> 2048 projections ran 2 % faster on 128 x 64)
  if (!generic && tiles(128, 128) >= 2 * cus)
    return launch_tile<128, 128, 2, 2, 2, false>(in, W, bias, out, M, K, N, act, accumulate, 1, s);
  // when even 128 x 64 tiles leave CUs idle, split K until the grid gives every CU two
  // workgroups (K / 512 splits at most)
  const long t = tiles(128, 64);
  int splits = 1;
  if (t < cus)
    splits = static_cast<int>(std::min<long>((2 * cus + t - 1) / t, std::max(1, K / 512)));
  if (generic)
    return launch_tile<128, 64, 4, 1, 2, true>(in, W, bias, out, M, K, N, act, accumulate, splits,
                                               s);
  return launch_tile<128, 64, 4, 1, 2, false>(in, W, bias, out, M, K, N, act, accumulate, splits,
                                              s);
}

}  // namespace orator_hip
