// fp32 GEMM on fp32 MFMA (gfx950): out[M,N] = act(sum_k in[m,k] * W[n,k] (+ bias[n])).
//
// Replaces gemm::LaunchSgemm / LaunchSgemmBatched (include/model/gemm.cuh:47-268): the same
// nn.Linear "NT" contract (both operands K-contiguous), activation codes 0 none, 1 SiLU,
// 2 ReLU, 3 sigmoid (gemm.cuh:38-45), strided batches, arbitrary M/N/K and alignment
// (guarded loads, as SgemmBatchedKernel).  Products are exact fp32 and accumulate in fp32
// on v_mfma_f32_32x32x2_f32, so results stay within fp32 rounding of the reference's
// k-sequential FMA chains.
//
// Workgroup = 64 x 64 tile of one batch entry, 4 waves of one 32 x 32 block each, four
// workgroups per CU (fp32 MFMA is 16x slower per flop than bf16, so these small products are
// latency-bound and want many resident waves, not big tiles: 128 x 128 tiles measured 1.6-2.8x
// slower at the Conformer's shapes).  K advances 32 floats at a time through two LDS buffers
// (rows padded to 36 floats = 144 bytes: the 16 rows a quarter-wave reads land on distinct
// 16-byte bank groups).  MFMA k-step j takes k = 2j from the lower half-wave and 2j + 1 from
// the upper (the pairs in k order, as a k-sequential chain adds them); LDS rows hold the even k
// then the odd k, so one ds_read_b128 per lane still feeds four MFMAs.  The next K tile is
// loaded into registers while the current one is multiplied and stored before the step's last
// MFMAs, the next fragments are read under the current ones; one barrier per step.  When the
// grid leaves CUs idle and K is long, K is split over workgroups and the partials are summed
// in a fixed order.
#include <stdint.h>

#include <algorithm>

#include "common.hpp"
#include "internal.hpp"

namespace orator_hip {
namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kSK = 32;        // K per step (floats)
constexpr int kSLd = kSK + 4;  // padded LDS row

__device__ __forceinline__ float apply_act(float v, int act) {
  if (act == 1) return v / (1.0f + expf(-v));
  if (act == 2) return fmaxf(v, 0.0f);
  if (act == 3) return 1.0f / (1.0f + expf(-v));
  return v;
}

struct SgemmArgs {
  const float* in;
  const float* W;
  const float* bias;
  float* out;
  float* part;  // split-K partials [splits][batch][M][N], or nullptr
  int M, K, N, act, k_split;
  int batch, splits;  // blockIdx.z = split * batch + batch entry
  long s_in, s_w, s_out;
  bool vec;  // K % 32 == 0 and 16-byte aligned operands: 16-byte loads
  // Grouped products (group > 0): `group` problems share `in`; problem z uses weight Wg[z],
  // bias bg[z] and output og[z] (batch = group, blockIdx.z selects the problem).
  int group;
  const float* Wg[3];
  const float* bg[3];
  float* og[3];
  // Residual update (residual != 0): out = out + res_scale * (in W^T + bias), act 0.
  int residual;
  float res_scale;
  // GLU (the kSEpiGlu epilogue): W has 2 glu_c rows (value rows, then gate rows); out[m][c] =
  // a * (1 / (1 + exp(-b))) with a, b the value and gate outputs (bias added), 0 for rows
  // m >= glu_valid; out is [M][glu_c].
  int glu_c, glu_valid;
  // LayerNorm of the updated rows (ln_g non-null; split-K reduce only): ln_out[m] =
  // (x - mean) rsqrt(var + eps) g + b over the row's N values x = out[m] after the residual
  // update; ln_out == out writes the normalised row only.
  const float* ln_g;
  const float* ln_b;
  float* ln_out;
  float ln_eps;
  // fp16 outputs: bit z set stores problem z's output (group products; bit 0 otherwise) as
  // fp16, each value rounded to nearest even once; unsplit products without residual only.
  int h16;
};

// Epilogues: raw split-K partials, out = acc (no bias, act 0), and through LDS out =
// act(acc + bias) or the residual update out += res_scale * (acc + bias), or the GLU of a
// tile's value and gate halves.  out = acc and out = act(acc + bias) may be stored as fp16 (h16).
constexpr int kSEpiPartial = 0, kSEpiStore = 1, kSEpiAct = 2, kSEpiGlu = 3;

template <int BM, int BN, int WGM, int WGN, int MINW, bool VEC, int EPI>
__global__ __launch_bounds__(64 * WGM * WGN, MINW) void sgemm_nt_kernel(SgemmArgs a) {
  constexpr int NT = 64 * WGM * WGN;
  constexpr int TM = BM / WGM, TN = BN / WGN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int RPI = NT / 8;  // rows per load instruction (8 threads x 16 bytes per row)
  // load instructions per thread per K step; a tile side that is not a multiple of RPI (96 x 64
  // tiles: 48 rows per instruction) loads clamped rows past it and does not store them
  constexpr int LA = (BM + RPI - 1) / RPI, LW = (BN + RPI - 1) / RPI;
  // LDS: the double-buffered tiles during the K loop, then (bias / activation epilogue) the
  // fp32 output tile, rows padded by 8 floats
  constexpr int kCLd = BN + 8;
  constexpr int kTileBytes = 2 * (BM + BN) * kSLd * 4;
  constexpr int kOutBytes = BM * kCLd * 4;
  __shared__ __align__(16) unsigned char smem[kTileBytes > kOutBytes ? kTileBytes : kOutBytes];
  auto sA = reinterpret_cast<float(*)[BM][kSLd]>(smem);
  auto sW = reinterpret_cast<float(*)[BN][kSLd]>(smem + 2 * BM * kSLd * 4);
  auto sC = reinterpret_cast<float(*)[kCLd]>(smem);

  const int batch = blockIdx.z % a.batch;
  const int split = blockIdx.z / a.batch;
  const float* A = a.in + batch * a.s_in;
  const float* B = a.group ? a.Wg[batch] : a.W + batch * a.s_w;
  const int M = a.M, N = a.N, K = a.K;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int kb = split * a.k_split;
  const int k_end = min(K, kb + a.k_split);
  const int lr = tid >> 3, lc = tid & 7;
  // 16-byte loads (VEC: K a multiple of the 32-float step, 16-byte aligned operands, so every
  // split is whole steps): rows clamped into range (their outputs are never stored), no
  // branches.  Otherwise guarded scalar loads.
  const float* arow[LA];
  const float* wrow[LW];
#pragma unroll
  for (int i = 0; i < LA; ++i) arow[i] = A + static_cast<long>(min(m0 + RPI * i + lr, M - 1)) * K;
#pragma unroll
  for (int i = 0; i < LW; ++i) {
    if constexpr (EPI == kSEpiGlu) {  // tile rows: BN/2 value rows, then the matching gate rows
      const int t = RPI * i + lr, c = blockIdx.x * (BN / 2) + (t % (BN / 2));
      wrow[i] = B + static_cast<long>((t < BN / 2 ? 0 : a.glu_c) + min(c, a.glu_c - 1)) * K;
    } else {
      wrow[i] = B + static_cast<long>(min(n0 + RPI * i + lr, N - 1)) * K;
    }
  }
  float4 ra[LA], rw[LW];
  auto load_guarded = [&](const float* base, int row, int rows, int k) -> float4 {
    if (row >= rows) return make_float4(0.f, 0.f, 0.f, 0.f);
    const float* p = base + static_cast<long>(row) * K + k;
    float4 v;
    v.x = k < k_end ? p[0] : 0.f;
    v.y = k + 1 < k_end ? p[1] : 0.f;
    v.z = k + 2 < k_end ? p[2] : 0.f;
    v.w = k + 3 < k_end ? p[3] : 0.f;
    return v;
  };
  auto load = [&](int k0) {
    const int k = k0 + 4 * lc;
    if constexpr (VEC) {
#pragma unroll
      for (int i = 0; i < LA; ++i) ra[i] = *reinterpret_cast<const float4*>(arow[i] + k);
#pragma unroll
      for (int i = 0; i < LW; ++i) rw[i] = *reinterpret_cast<const float4*>(wrow[i] + k);
    } else {
#pragma unroll
      for (int i = 0; i < LA; ++i) ra[i] = load_guarded(A, m0 + RPI * i + lr, M, k);
#pragma unroll
      for (int i = 0; i < LW; ++i) rw[i] = load_guarded(B, n0 + RPI * i + lr, N, k);
    }
  };
  // LDS row = [even k | odd k]: k = 4c..4c+3 of a 16-byte load go to slots 2c, 2c+1 of each
  // half, so a lane of half h reading slots 4q..4q+3 of half h gets k = 2j + h, j = 4q..4q+3
  auto put = [&](float* row, float4 v) {
    *reinterpret_cast<float2*>(row + 2 * lc) = make_float2(v.x, v.z);
    *reinterpret_cast<float2*>(row + 16 + 2 * lc) = make_float2(v.y, v.w);
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < LA; ++i)
      if (BM % RPI == 0 || RPI * i + lr < BM) put(&sA[buf][RPI * i + lr][0], ra[i]);
#pragma unroll
    for (int i = 0; i < LW; ++i)
      if (BN % RPI == 0 || RPI * i + lr < BN) put(&sW[buf][RPI * i + lr][0], rw[i]);
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int fr = lane & 31, fk = 16 * (lane >> 5);
  const int n_k = (k_end - kb + kSK - 1) / kSK;
  load(kb);
  store(0);
  lds_barrier();
  for (int t = 0; t < n_k; ++t) {
    const int buf = t & 1;
    if (t + 1 < n_k) load(kb + (t + 1) * kSK);
    float4 fa[2][FM], fb[2][FN];
    auto read = [&](int q, int s) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
        fa[s][i] = *reinterpret_cast<const float4*>(&sA[buf][wm * TM + 32 * i + fr][fk + 4 * q]);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        fb[s][j] = *reinterpret_cast<const float4*>(&sW[buf][wn * TN + 32 * j + fr][fk + 4 * q]);
    };
    read(0, 0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int s = q & 1;
      if (q + 1 < 4) read(q + 1, s ^ 1);  // next fragments under this q's MFMAs
      // the next tile goes to the other (idle) buffer before the step's last MFMAs
      if (q == 3 && t + 1 < n_k) store(buf ^ 1);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] =
                __builtin_amdgcn_mfma_f32_32x32x2f32(fa[s][i][e], fb[s][j][e], acc[i][j], 0, 0, 0);
    }
    lds_barrier();
  }

  // block (i, j): lane holds column 32 j + lane % 32 and rows 8 (e / 4) + 4 (lane / 32) + e % 4
  // of the block.  Plain stores and partials go straight out (nothing is loaded, so no store
  // waits); bias / activation go through LDS with the bias loaded before the first store
  // (stores count against the same wait counter as loads).
  if constexpr (EPI == kSEpiPartial || EPI == kSEpiStore) {
    float* C = EPI == kSEpiPartial
                   ? a.part + (static_cast<long>(split) * a.batch + batch) * M * N
                   : (a.group ? a.og[batch] : a.out + batch * a.s_out);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = n0 + wn * TN + 32 * j + fr;
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m0 + wm * TM + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
          if (m >= M) continue;
          if (EPI == kSEpiStore && (a.h16 & 1))  // ungrouped: bit 0
            reinterpret_cast<_Float16*>(C)[static_cast<long>(m) * N + n] =
                static_cast<_Float16>(acc[i][j][e]);
          else
            C[static_cast<long>(m) * N + n] = acc[i][j][e];
        }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        sC[wm * TM + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)][wn * TN + 32 * j + fr] =
            acc[i][j][e];
  __syncthreads();
  if constexpr (EPI == kSEpiGlu) {
    // columns [0, BN/2) of the tile are the value outputs of channels c0 .., [BN/2, BN) the
    // gate outputs of the same channels; the same fp32 values and formula as a plain product
    // followed by the GLU pass (its bias added, then a * (1 / (1 + exp(-b))))
    constexpr int HB = BN / 2, TPRg = HB / 4, RPIg = NT / TPRg, PASSES_G = BM / RPIg;
    const int Cg = a.glu_c, c0 = blockIdx.x * HB;
    const int orow = tid / TPRg, j = 4 * (tid % TPRg);
    float ba[4] = {0.f, 0.f, 0.f, 0.f}, bg[4] = {0.f, 0.f, 0.f, 0.f};
    if (a.bias) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        ba[q] = a.bias[min(c0 + j + q, Cg - 1)];
        bg[q] = a.bias[Cg + min(c0 + j + q, Cg - 1)];
      }
    }
    const bool vec_out = (Cg % 4) == 0 && ((reinterpret_cast<uintptr_t>(a.out)) & 15) == 0;
#pragma unroll
    for (int p = 0; p < PASSES_G; ++p) {
      const int r = RPIg * p + orow;
      const int m = m0 + r;
      const float4 va = *reinterpret_cast<const float4*>(&sC[r][j]);
      const float4 vg = *reinterpret_cast<const float4*>(&sC[r][HB + j]);
      const float av[4] = {va.x, va.y, va.z, va.w}, gv[4] = {vg.x, vg.y, vg.z, vg.w};
      float o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float x = av[q] + ba[q], g = gv[q] + bg[q];
        o[q] = m < a.glu_valid ? x * (1.0f / (1.0f + __expf(-g))) : 0.0f;
      }
      if (m >= M) continue;
      float* dst = a.out + static_cast<long>(m) * Cg + c0 + j;
      if (vec_out && c0 + j + 3 < Cg) {
        *reinterpret_cast<float4*>(dst) = make_float4(o[0], o[1], o[2], o[3]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (c0 + j + q < Cg) dst[q] = o[q];
      }
    }
    return;
  }
  float* C = a.group ? a.og[batch] : a.out + batch * a.s_out;
  const float* bias = a.group ? a.bg[batch] : a.bias;
  const bool h16 = (a.h16 >> (a.group ? batch : 0)) & 1;
  constexpr int TPRo = BN / 4, RPIo = NT / TPRo, PASSES = BM / RPIo;
  const int orow = tid / TPRo, ocol = 4 * (tid % TPRo);
  const int n = n0 + ocol;
  const bool vec_out = (N % 4) == 0 && ((reinterpret_cast<uintptr_t>(C)) & 15) == 0;
  const bool vec_h16 = (N % 4) == 0 && ((reinterpret_cast<uintptr_t>(C)) & 7) == 0;
  float bv[4] = {0.f, 0.f, 0.f, 0.f};
  if (bias) {
#pragma unroll
    for (int q = 0; q < 4; ++q) bv[q] = bias[min(n + q, N - 1)];
  }
  // the residual's old values, all loaded before the first store
  float old[PASSES][4];
  if (a.residual) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const float* src = C + static_cast<long>(min(m0 + RPIo * p + orow, M - 1)) * N;
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
      v[q] = apply_act(v[q] + bv[q], a.act);
      if (a.residual) v[q] = fmaf(a.res_scale, v[q], old[p][q]);
    }
    if (m >= M) continue;
    if (h16) {
      _Float16* dst = reinterpret_cast<_Float16*>(C) + static_cast<long>(m) * N + n;
      if (vec_h16 && n + 3 < N) {
        typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
        const h4_t hv = {static_cast<_Float16>(v[0]), static_cast<_Float16>(v[1]),
                         static_cast<_Float16>(v[2]), static_cast<_Float16>(v[3])};
        *reinterpret_cast<h4_t*>(dst) = hv;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (n + q < N) dst[q] = static_cast<_Float16>(v[q]);
      }
      continue;
    }
    float* dst = C + static_cast<long>(m) * N + n;
    if (vec_out && n + 3 < N) {
      *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (n + q < N) dst[q] = v[q];
    }
  }
}

// out_b[m][n] = act(sum_z part[z][b][m][n] + bias[n]), z ascending (a fixed order).
__global__ __launch_bounds__(256) void sgemm_splitk_reduce_kernel(const float* __restrict__ part,
                                                                  int splits, int batch,
                                                                  const float* __restrict__ bias,
                                                                  float* __restrict__ out, int M,
                                                                  int N, int act, long s_out,
                                                                  int residual, float res_scale) {
  const long MN = static_cast<long>(M) * N;
  const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= MN * batch) return;
  const long b = i / MN, r = i - b * MN;
  const long per_split = MN * batch;
  float v = part[i];
  for (int z = 1; z < splits; ++z) v += part[z * per_split + i];
  v = apply_act(v + (bias ? bias[r % N] : 0.0f), act);
  if (residual) v = fmaf(res_scale, v, out[b * s_out + r]);
  out[b * s_out + r] = v;
}

// The split-K reduce with the residual update, then a LayerNorm of each updated row: one wave
// per row, lane l holding columns l, l + 64, ... (N <= 64 PER).  Per element the same
// arithmetic as sgemm_splitk_reduce_kernel (partials in split order, bias, residual fmaf);
// the normalisation is layer_norm_kernel's (lane-order sums, the wave sum, contraction off),
// so x and LN(x) carry the same bits as the reduce followed by the LayerNorm pass.
constexpr int kMaxLnSplits = 8;  // the split count run_sgemm chooses is at most 8

template <int PER, int MAXS>
__global__ __launch_bounds__(256) void sgemm_splitk_reduce_ln_kernel(
    const float* __restrict__ part, int splits, const float* __restrict__ bias, float* out,
    int M, int N, float res_scale, const float* __restrict__ g, const float* __restrict__ b,
    float* ln_out, float eps) {
#pragma clang fp contract(off)
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const long MN = static_cast<long>(M) * N;
  const long base = static_cast<long>(row) * N;
  // every partial of the lane's columns is loaded at once (one memory round trip: a wave per
  // row leaves few waves per CU); the sum keeps split order, terms past `splits` selected away
  float p[PER][MAXS], old[PER], bv[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int n = min(lane + 64 * i, N - 1);
#pragma unroll
    for (int z = 0; z < MAXS; ++z) p[i][z] = part[min(z, splits - 1) * MN + base + n];
    old[i] = out[base + n];
    bv[i] = bias ? bias[n] : 0.0f;
  }
  float v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    float x = p[i][0];
#pragma unroll
    for (int z = 1; z < MAXS; ++z) x = z < splits ? x + p[i][z] : x;
    x = x + bv[i];
    v[i] = fmaf(res_scale, x, old[i]);
  }
  const bool in_place = ln_out == out;
#pragma unroll
  for (int i = 0; i < PER; ++i)
    if (!in_place && lane + 64 * i < N) out[base + lane + 64 * i] = v[i];
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; ++i)
    if (lane + 64 * i < N) sum += v[i];
  const float mean = wave_sum(sum) / static_cast<float>(N);
  float sq = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const float t = v[i] - mean;
    if (lane + 64 * i < N) sq += t * t;
  }
  const float inv = rsqrtf(wave_sum(sq) / static_cast<float>(N) + eps);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int n = lane + 64 * i;
    if (n < N) ln_out[base + n] = (v[i] - mean) * inv * g[n] + b[n];
  }
}

template <int BM, int BN, int WGM, int WGN, int MINW, bool VEC>
int launch_sg(SgemmArgs a, int batch, int splits, hipStream_t s) {
  a.k_split = a.K;
  a.part = nullptr;
  if (splits > 1) {
    a.k_split = ((a.K + splits - 1) / splits + kSK - 1) / kSK * kSK;
    splits = (a.K + a.k_split - 1) / a.k_split;
  }
  a.batch = batch;
  a.splits = splits;
  const long MN = static_cast<long>(a.M) * a.N;
  if (splits > 1) {
    a.part = static_cast<float*>(
        workspace(s, static_cast<size_t>(splits) * batch * MN * sizeof(float), kWsGemm));
    if (!a.part) return ORATOR_ERR_HIP;
  }
  const dim3 grid((a.N + BN - 1) / BN, (a.M + BM - 1) / BM, batch * splits);
  const dim3 block(64 * WGM * WGN);
  if (splits > 1)
    hipLaunchKernelGGL((sgemm_nt_kernel<BM, BN, WGM, WGN, MINW, VEC, kSEpiPartial>), grid, block,
                       0, s, a);
  else if (a.bias || a.act || a.residual || a.group)
    hipLaunchKernelGGL((sgemm_nt_kernel<BM, BN, WGM, WGN, MINW, VEC, kSEpiAct>), grid, block, 0,
                       s, a);
  else
    hipLaunchKernelGGL((sgemm_nt_kernel<BM, BN, WGM, WGN, MINW, VEC, kSEpiStore>), grid, block,
                       0, s, a);
  if (int rc = check_launch("sgemm_nt_kernel")) return rc;
  if (splits == 1) {
    if (!a.ln_g) return ORATOR_OK;
    return launch_layer_norm(a.out, a.ln_g, a.ln_b, a.ln_out, a.M, a.N, a.ln_eps, s);
  }
  if (a.ln_g && a.N <= 1024 && splits <= kMaxLnSplits) {  // batch 1, act 0, residual
    const dim3 rgrid((a.M + 3) / 4);
    auto go = [&](auto kern) {
      hipLaunchKernelGGL(kern, rgrid, dim3(256), 0, s, a.part, splits, a.bias, a.out, a.M, a.N,
                         a.res_scale, a.ln_g, a.ln_b, a.ln_out, a.ln_eps);
    };
    if (a.N <= 512)
      splits <= 2 ? go(sgemm_splitk_reduce_ln_kernel<8, 2>) : go(sgemm_splitk_reduce_ln_kernel<8, 8>);
    else
      splits <= 2 ? go(sgemm_splitk_reduce_ln_kernel<16, 2>) : go(sgemm_splitk_reduce_ln_kernel<16, 8>);
    return check_launch("sgemm_splitk_reduce_ln");
  }
  const long total = MN * batch;
  hipLaunchKernelGGL(sgemm_splitk_reduce_kernel, dim3(static_cast<unsigned>((total + 255) / 256)),
                     dim3(256), 0, s, a.part, splits, batch, a.bias, a.out, a.M, a.N, a.act,
                     batch > 1 ? a.s_out : MN, a.residual, a.res_scale);
  if (int rc = check_launch("sgemm_splitk_reduce")) return rc;
  if (!a.ln_g) return ORATOR_OK;
  return launch_layer_norm(a.out, a.ln_g, a.ln_b, a.ln_out, a.M, a.N, a.ln_eps, s);
}

// 64 x 64 tiles, 4 waves of one 32 x 32 block each, four workgroups per CU.  K is split over
// workgroups only when the grid leaves more than half the CUs idle.  Measured at the
// Conformer's shapes: 717 x 2048 -> 512 takes 25 us with 8 splits against 45.9 unsplit;
// 1433 x 512 -> 512 (184 tiles) 13.6 unsplit against 19.1 with 2 splits.  Grouped products
// are never split.  Two tiles on one CU are
// MFMA-bound together (each takes twice as long), so an unsplit grid that would give some CUs
// two 64 x 64 tiles takes 96 x 64 tiles (6 waves) when that needs fewer rounds of work and K
// is long enough for the tiles to be MFMA-bound: 717 x 512 -> 2048 (384 tiles -> 256) 28.3 ->
// 24.5 us, -> 1536 (288 -> 192) 27.5 -> 23.5 us; at K = 64 (8 x 717 x 64 -> 717) 96-row tiles
// were slower, 16.1 against 12.9 us.
int run_sgemm(SgemmArgs a, int batch, hipStream_t stream) {
  const int M = a.M, N = a.N, K = a.K;
  const long cus = device_cu_count() > 0 ? device_cu_count() : 256;
  const long t = static_cast<long>((M + 63) / 64) * ((N + 63) / 64) * batch;
  int splits = 1;
  if (2 * t <= cus && K >= 512 && !a.group && !a.h16) {
    // the split count with the least work per CU in whole rounds, ceil(t s / cus) / s (ties to
    // fewer splits), K / 256 and 8 at most: 717 x 2048 -> 512 (96 tiles) takes 8 splits (768
    // workgroups, 3 rounds of 1/8): 24.7-25.9 us, against 25.9-27.4 with 5 and 27.5-28.9 with 6
    long best_num = 1, best_den = 1;  // 1 round of the whole K
    for (long sp = 2; sp <= std::min<long>(8, K / 256); ++sp) {
      const long rounds = (t * sp + cus - 1) / cus;
      if (rounds * best_den < best_num * sp) {
        best_num = rounds;
        best_den = sp;
      }
    }
    splits = static_cast<int>(best_den);
  }
  if (static_cast<long>(batch) * splits > 65535) splits = 1;
  if (splits == 1 && t > cus && K >= 256) {  // short K: latency-bound tiles, more is better
    const long t96 = static_cast<long>((M + 95) / 96) * ((N + 63) / 64) * batch;
    const long r64 = (t + cus - 1) / cus, r96 = (t96 + cus - 1) / cus;
    if (2 * r64 > 3 * r96) {  // rounds of 64 x 64 work: r64 against 1.5 r96
      if (a.vec) return launch_sg<96, 64, 3, 2, 2, true>(a, batch, 1, stream);
      return launch_sg<96, 64, 3, 2, 2, false>(a, batch, 1, stream);
    }
  }
  if (a.vec) return launch_sg<64, 64, 2, 2, 4, true>(a, batch, splits, stream);
  return launch_sg<64, 64, 2, 2, 4, false>(a, batch, splits, stream);
}

}  // namespace

int launch_sgemm(const float* in, const float* W, const float* bias, float* out, int M, int K,
                 int N, int act, int batch, long stride_in, long stride_w, long stride_out,
                 hipStream_t stream) {
  if (M <= 0 || N <= 0 || K <= 0 || batch <= 0) return ORATOR_OK;
  if (!in || !W || !out) return fail(ORATOR_ERR_INVALID, "sgemm: null pointer");
  if (act < 0 || act > 3) return fail(ORATOR_ERR_INVALID, "sgemm: act must be 0..3");
  if (batch > 65535) return fail(ORATOR_ERR_UNSUPPORTED, "sgemm: at most 65535 batches");
  SgemmArgs a{};
  a.in = in;
  a.W = W;
  a.bias = bias;
  a.out = out;
  a.M = M;
  a.K = K;
  a.N = N;
  a.act = act;
  a.s_in = batch > 1 ? stride_in : 0;
  a.s_w = batch > 1 ? stride_w : 0;
  a.s_out = batch > 1 ? stride_out : 0;
  a.vec = (K % kSK) == 0 && ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(W) |
                            (batch > 1 ? (stride_in | stride_w) * 4 : 0)) & 15) == 0;
  return run_sgemm(a, batch, stream);
}

int launch_sgemm_residual(const float* in, const float* W, const float* bias, float* out, int M,
                          int K, int N, float res_scale, hipStream_t stream) {
  if (M <= 0 || N <= 0 || K <= 0) return ORATOR_OK;
  if (!in || !W || !out) return fail(ORATOR_ERR_INVALID, "sgemm: null pointer");
  SgemmArgs a{};
  a.in = in;
  a.W = W;
  a.bias = bias;
  a.out = out;
  a.M = M;
  a.K = K;
  a.N = N;
  a.residual = 1;
  a.res_scale = res_scale;
  a.vec = (K % kSK) == 0 &&
          ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(W)) & 15) == 0;
  return run_sgemm(a, 1, stream);
}

int launch_sgemm_residual_ln(const float* in, const float* W, const float* bias, float* out,
                             int M, int K, int N, float res_scale, const float* ln_g,
                             const float* ln_b, float* ln_out, float eps, hipStream_t stream) {
  if (M <= 0 || N <= 0 || K <= 0) return ORATOR_OK;
  if (!in || !W || !out || !ln_g || !ln_b || !ln_out)
    return fail(ORATOR_ERR_INVALID, "sgemm_residual_ln: null pointer");
  SgemmArgs a{};
  a.in = in;
  a.W = W;
  a.bias = bias;
  a.out = out;
  a.M = M;
  a.K = K;
  a.N = N;
  a.residual = 1;
  a.res_scale = res_scale;
  a.ln_g = ln_g;
  a.ln_b = ln_b;
  a.ln_out = ln_out;
  a.ln_eps = eps;
  a.vec = (K % kSK) == 0 &&
          ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(W)) & 15) == 0;
  return run_sgemm(a, 1, stream);
}

int launch_sgemm_glu(const float* in, const float* W, const float* bias, float* out, int M, int K,
                     int C, int valid, hipStream_t stream) {
  if (M <= 0 || C <= 0 || K <= 0) return ORATOR_OK;
  if (!in || !W || !out) return fail(ORATOR_ERR_INVALID, "sgemm_glu: null pointer");
  if ((K % kSK) != 0 ||
      ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(W)) & 15) != 0)
    return ORATOR_ERR_UNSUPPORTED;  // no 16-byte loads: the caller takes the two-pass path
  SgemmArgs a{};
  a.in = in;
  a.W = W;
  a.bias = bias;
  a.out = out;
  a.M = M;
  a.K = K;
  a.N = 2 * C;
  a.k_split = K;
  a.batch = 1;
  a.splits = 1;
  a.vec = true;
  a.glu_c = C;
  a.glu_valid = valid;
  const dim3 grid((C + 31) / 32, (M + 63) / 64, 1);
  hipLaunchKernelGGL((sgemm_nt_kernel<64, 64, 2, 2, 4, true, kSEpiGlu>), grid, dim3(256), 0, stream,
                     a);
  return check_launch("sgemm_nt_kernel (glu)");
}

int launch_sgemm_group3(const float* in, const float* const W[3], const float* const bias[3],
                        void* const out[3], int M, int K, int N, int h16_mask,
                        hipStream_t stream) {
  if (M <= 0 || N <= 0 || K <= 0) return ORATOR_OK;
  if (!in) return fail(ORATOR_ERR_INVALID, "sgemm: null pointer");
  SgemmArgs a{};
  a.in = in;
  a.M = M;
  a.K = K;
  a.N = N;
  a.group = 3;
  a.h16 = h16_mask & 7;
  uintptr_t align = reinterpret_cast<uintptr_t>(in);
  for (int g = 0; g < 3; ++g) {
    if (!W[g] || !out[g]) return fail(ORATOR_ERR_INVALID, "sgemm: null pointer");
    a.Wg[g] = W[g];
    a.bg[g] = bias[g];
    a.og[g] = static_cast<float*>(out[g]);
    align |= reinterpret_cast<uintptr_t>(W[g]);
  }
  a.W = a.Wg[0];
  a.vec = (K % kSK) == 0 && (align & 15) == 0;
  return run_sgemm(a, 3, stream);
}

int launch_sgemm_f16_out(const float* in, const float* W, void* out, int M, int K, int N,
                         hipStream_t stream) {
  if (M <= 0 || N <= 0 || K <= 0) return ORATOR_OK;
  if (!in || !W || !out) return fail(ORATOR_ERR_INVALID, "sgemm: null pointer");
  SgemmArgs a{};
  a.in = in;
  a.W = W;
  a.out = static_cast<float*>(out);
  a.M = M;
  a.K = K;
  a.N = N;
  a.h16 = 1;
  a.vec = (K % kSK) == 0 &&
          ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(W)) & 15) == 0;
  return run_sgemm(a, 1, stream);
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
