// Masked multi-head self-attention with a small head dimension (the Sortformer decoder's
// transformer layers: H = 8, Dk = 24), fp32 throughout.
//
// Replaces the GEMM-decomposed MHA of src/model/sortformer_decoder.cu:280-298 (head-major
// gathers, QK^T batched SGEMM, ScaleMaskScoresKernel, AttnSoftmaxKernel, PV batched SGEMM,
// scatter): scores = (q_i . k_j) * scale, keys j >= valid_len scored -1e30, row softmax, then
// ctx = P . V, written back in the [T, H, Dk] layout linear_out reads.  No [H, T, T] score
// matrix: one workgroup owns 64 queries of one head, one query per lane; its waves (16 for
// Dk <= 32, 8 above: 717 queries x 8 heads is only 96 workgroups, so the keys are split
// finely to occupy the SIMDs) split the keys, each keeps an online softmax (a running max per
// 8-key block), and the partials are merged in LDS.  When those workgroups leave CUs idle,
// the keys are also split over grid z (Z workgroups per query tile and head): each writes its
// unnormalised (max, sum, P.V) to a workspace and a second kernel merges the Z partials per
// (query, head) (717 x 8 heads on 256 CUs: Z = 2, half the keys per workgroup).  K and V rows are wave-uniform, so they arrive through scalar
// loads and feed the FMAs as scalar operands: the kernel is VALU-bound at ~2 Dk FMAs per
// (query, key), with no LDS traffic in the key loop.
#include "common.hpp"
#include "internal.hpp"

namespace orator_hip {
namespace {

constexpr int kQ = 64;       // queries per workgroup (one per lane)
constexpr int kKB = 8;       // keys per softmax block

// key ranges (waves) per workgroup; the merge area [waves][64][DK + 2] floats fits the LDS
template <int DK>
constexpr int mha_waves() {
  return DK <= 32 ? 16 : 8;
}

template <int DK, int kWaves = mha_waves<DK>()>
__global__ __launch_bounds__(kQ * kWaves) void mha_small_kernel(const float* __restrict__ q,
                                                                const float* __restrict__ k,
                                                                const float* __restrict__ v,
                                                                float* __restrict__ out, int T,
                                                                int H, int valid, float scale,
                                                                int nsplit,
                                                                float* __restrict__ ws) {
  __shared__ float part[kWaves][kQ][DK + 2];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = blockIdx.y;
  const int i = blockIdx.x * kQ + lane;
  const int ic = min(i, T - 1);
  const long hs = static_cast<long>(H) * DK;  // elements between tokens

  // Keys attended: [0, valid); with no valid key every score is -1e30 in the reference and the
  // softmax is uniform over all T keys, which score 0 reproduces.
  const bool uniform = valid <= 0;
  const int nk = uniform ? T : min(valid, T);
  const int ranges = nsplit * kWaves;  // key ranges of one query tile: (split z, wave)
  const int per = ((nk + ranges - 1) / ranges + kKB - 1) / kKB * kKB;
  const int j0 = min((static_cast<int>(blockIdx.z) * kWaves + wave) * per, nk);
  const int j1 = min(j0 + per, nk);

  float qr[DK];
  const float* qp = q + ic * hs + static_cast<long>(h) * DK;
#pragma unroll
  for (int d = 0; d < DK; d += 4) {
    const float4 x = *reinterpret_cast<const float4*>(qp + d);
    qr[d] = x.x;
    qr[d + 1] = x.y;
    qr[d + 2] = x.z;
    qr[d + 3] = x.w;
  }
  float m = -INFINITY, l = 0.0f, acc[DK];
#pragma unroll
  for (int d = 0; d < DK; ++d) acc[d] = 0.0f;

  const float* kh = k + static_cast<long>(h) * DK;
  const float* vh = v + static_cast<long>(h) * DK;
  for (int jb = j0; jb < j1; jb += kKB) {
    float s[kKB];
    float bm = -INFINITY;
#pragma unroll
    for (int u = 0; u < kKB; ++u) {
      const int j = jb + u;
      if (j < j1) {
        const float* kr = kh + j * hs;
        float dot = 0.0f;
#pragma unroll
        for (int d = 0; d < DK; ++d) dot = fmaf(qr[d], kr[d], dot);
        s[u] = uniform ? 0.0f : dot * scale;
      } else {
        s[u] = -INFINITY;
      }
      bm = fmaxf(bm, s[u]);
    }
    const float mn = fmaxf(m, bm);  // finite: key jb is in range
    const float corr = __expf(m - mn);
    l *= corr;
#pragma unroll
    for (int d = 0; d < DK; ++d) acc[d] *= corr;
#pragma unroll
    for (int u = 0; u < kKB; ++u) {
      const int j = jb + u;
      if (j < j1) {
        const float p = __expf(s[u] - mn);
        l += p;
        const float* vr = vh + j * hs;
#pragma unroll
        for (int d = 0; d < DK; ++d) acc[d] = fmaf(p, vr[d], acc[d]);
      }
    }
    m = mn;
  }

  // ---- merge the key ranges ----
  float* mine = part[wave][lane];
  mine[0] = m;
  mine[1] = l;
#pragma unroll
  for (int d = 0; d < DK; ++d) mine[2 + d] = acc[d];
  __syncthreads();
  if (wave != 0) return;
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) M = fmaxf(M, part[w][lane][0]);
  float L = 0.0f, o[DK];
#pragma unroll
  for (int d = 0; d < DK; ++d) o[d] = 0.0f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const float* pw = part[w][lane];
    const float c = pw[0] == -INFINITY ? 0.0f : __expf(pw[0] - M);  // empty range: weight 0
    L = fmaf(c, pw[1], L);
#pragma unroll
    for (int d = 0; d < DK; ++d) o[d] = fmaf(c, pw[2 + d], o[d]);
  }
  if (i >= T) return;
  if (nsplit > 1) {
    // ws[z][h][c][i], c = max, sum, P.V[0..DK): consecutive lanes write consecutive floats
    float* wp = ws + (static_cast<long>(blockIdx.z) * H + h) * (DK + 2) * T + i;
    wp[0] = M;
    wp[T] = L;
#pragma unroll
    for (int d = 0; d < DK; ++d) wp[static_cast<long>(2 + d) * T] = o[d];
    return;
  }
  const float inv = 1.0f / L;
  float* op = out + i * hs + static_cast<long>(h) * DK;
#pragma unroll
  for (int d = 0; d < DK; d += 4)
    *reinterpret_cast<float4*>(op + d) =
        make_float4(o[d] * inv, o[d + 1] * inv, o[d + 2] * inv, o[d + 3] * inv);
}

// out[i][h] = sum_z c_z o_z / sum_z c_z l_z, c_z = exp(m_z - max_z m_z) (0 for a split with no
// keys, m_z = -inf): the Z key-split partials of one (query, head), one thread each; one wave
// per workgroup, so the ~90 workgroups of T = 717 x 8 heads spread their loads over as many
// CUs.
template <int DK>
__global__ __launch_bounds__(64) void mha_small_merge_kernel(const float* __restrict__ ws,
                                                              float* __restrict__ out, int T,
                                                              int H, int nsplit) {
  const long idx = static_cast<long>(blockIdx.x) * 64 + threadIdx.x;
  if (idx >= static_cast<long>(T) * H) return;
  const int i = static_cast<int>(idx % T), h = static_cast<int>(idx / T);
  const long zs = static_cast<long>(H) * (DK + 2) * T;  // floats between splits
  const float* wp = ws + static_cast<long>(h) * (DK + 2) * T + i;
  float M = -INFINITY;
  for (int z = 0; z < nsplit; ++z) M = fmaxf(M, wp[z * zs]);
  float L = 0.0f, o[DK];
#pragma unroll
  for (int d = 0; d < DK; ++d) o[d] = 0.0f;
  for (int z = 0; z < nsplit; ++z) {
    const float* pz = wp + z * zs;
    const float m = pz[0];
    const float c = m == -INFINITY ? 0.0f : __expf(m - M);
    L = fmaf(c, pz[T], L);
#pragma unroll
    for (int d = 0; d < DK; ++d) o[d] = fmaf(c, pz[static_cast<long>(2 + d) * T], o[d]);
  }
  const float inv = 1.0f / L;
  float* op = out + (static_cast<long>(i) * H + h) * DK;
#pragma unroll
  for (int d = 0; d < DK; d += 4)
    *reinterpret_cast<float4*>(op + d) =
        make_float4(o[d] * inv, o[d + 1] * inv, o[d + 2] * inv, o[d + 3] * inv);
}

template <int DK>
int launch(const float* q, const float* k, const float* v, float* out, int T, int H, int valid,
           float scale, hipStream_t s) {
  constexpr int kWaves = mha_waves<DK>();
  // Key splits over grid z: as many as the CUs take one workgroup each (the merge area holds
  // a CU's LDS to one workgroup), at most 8, and at least one 8-key block per wave each.
  const int tiles = (T + kQ - 1) / kQ;
  const long wgs = static_cast<long>(tiles) * H;
  const long cus = device_cu_count() > 0 ? device_cu_count() : 256;
  const int nk = valid <= 0 ? T : (valid < T ? valid : T);
  long z = std::min<long>(8, cus / wgs);
  z = std::min<long>(z, nk / (kWaves * kKB));
  const int nsplit = z > 1 ? static_cast<int>(z) : 1;
  float* ws = nullptr;
  if (nsplit > 1) {
    ws = static_cast<float*>(
        workspace(s, static_cast<size_t>(nsplit) * H * (DK + 2) * T * sizeof(float), kWsMha));
    if (!ws) return ORATOR_ERR_HIP;
  }
  hipLaunchKernelGGL(mha_small_kernel<DK>, dim3(tiles, H, nsplit), dim3(kQ * kWaves), 0, s, q, k,
                     v, out, T, H, valid, scale, nsplit, ws);
  if (nsplit == 1) return check_launch("mha_small_kernel");
  if (int rc = check_launch("mha_small_kernel")) return rc;
  hipLaunchKernelGGL(mha_small_merge_kernel<DK>,
                     dim3(static_cast<unsigned>((static_cast<long>(T) * H + 63) / 64)),
                     dim3(64), 0, s, ws, out, T, H, nsplit);
  return check_launch("mha_small_merge_kernel");
}

}  // namespace
}  // namespace orator_hip

using namespace orator_hip;

extern "C" {

int orator_masked_mha(const float* q, const float* k, const float* v, float* out, int T, int H,
                      int Dk, int valid_len, float scale, void* stream) {
  if (T <= 0 || H <= 0 || Dk <= 0) return ORATOR_OK;
  if (!q || !k || !v || !out) return fail(ORATOR_ERR_INVALID, "masked_mha: null pointer");
  if (!(Dk == 24 || Dk == 32 || Dk == 64))
    return fail(ORATOR_ERR_UNSUPPORTED, "masked_mha: Dk must be 24, 32 or 64");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
       reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(out)) & 15u)
    return fail(ORATOR_ERR_INVALID, "masked_mha: q, k, v, out must be 16-byte aligned");
  if (H > 65535) return fail(ORATOR_ERR_UNSUPPORTED, "masked_mha: at most 65535 heads");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (Dk == 24) return launch<24>(q, k, v, out, T, H, valid_len, scale, s);
  if (Dk == 32) return launch<32>(q, k, v, out, T, H, valid_len, scale, s);
  return launch<64>(q, k, v, out, T, H, valid_len, scale, s);
}

}  // extern "C"
