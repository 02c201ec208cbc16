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
// 8-key block), and the partials are merged in LDS.  K and V rows are wave-uniform, so they arrive through scalar
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
                                                                int H, int valid, float scale) {
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
  const int per = ((nk + kWaves - 1) / kWaves + kKB - 1) / kKB * kKB;
  const int j0 = min(wave * per, nk);
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
  const float inv = 1.0f / L;
  float* op = out + i * hs + static_cast<long>(h) * DK;
#pragma unroll
  for (int d = 0; d < DK; d += 4)
    *reinterpret_cast<float4*>(op + d) =
        make_float4(o[d] * inv, o[d + 1] * inv, o[d + 2] * inv, o[d + 3] * inv);
}

template <int DK>
void launch(const float* q, const float* k, const float* v, float* out, int T, int H, int valid,
            float scale, hipStream_t s) {
  hipLaunchKernelGGL(mha_small_kernel<DK>, dim3((T + kQ - 1) / kQ, H), dim3(kQ * mha_waves<DK>()),
                     0, s, q, k, v, out, T, H, valid, scale);
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
  if (Dk == 24) launch<24>(q, k, v, out, T, H, valid_len, scale, s);
  else if (Dk == 32) launch<32>(q, k, v, out, T, H, valid_len, scale, s);
  else launch<64>(q, k, v, out, T, H, valid_len, scale, s);
  return check_launch("mha_small_kernel");
}

}  // extern "C"
