// Generic fp32 GQA self-attention for the shapes the split-K decode kernel is not built for.
//
// asr_ops::GqaAttention (include/model/asr_ops.cuh:50-56, src/model/asr_ops.cu:113-195,
// 237-295) accepts any power-of-two head_dim up to 1024 and any Hq that is a multiple of Hkv.
// The common shapes (Dh 64 / 128, Hq / Hkv in {1, 2, 4}) run on the split-K kernel; every
// other one runs here.  Semantics as the reference: query row i of head h attends keys
// [0, i] (causal) or [0, T) of kv head h / (Hq / Hkv), fp32 scores scaled after the dot,
// online softmax, out = acc / l (0 when l = 0).
//
// One workgroup = (query row, q head), 4 wave64s striding over the keys.  A key is covered by
// L = min(Dh, 64) lanes holding Dh / L elements each (element d = e * L + lane: coalesced
// rows), so a wave takes 64 / L keys per step; each key slot keeps its own online-softmax
// state, merged across slots and waves in LDS at the end.
#include <math.h>

#include "common.hpp"
#include "internal.hpp"

namespace orator_hip {
namespace {

constexpr int kGenWaves = 4;

template <int DH>
__global__ __launch_bounds__(64 * kGenWaves) void gqa_attention_generic_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ out, int T, int Hq, int Hkv, float scale_log2e, int causal) {
  constexpr int L = DH < kWave ? DH : kWave;  // lanes per key
  constexpr int KPI = kWave / L;              // keys per wave step
  constexpr int E = DH / L;                   // elements per lane
  constexpr int NS = kGenWaves * KPI;         // key slots per workgroup
  __shared__ float s_ml[NS][2];
  __shared__ float s_o[NS][DH];

  const int i = blockIdx.x;
  const int h = blockIdx.y;
  const int kvh = h / (Hq / Hkv);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane / L;  // key slot within the wave
  const int li = lane % L;
  const int slot = wave * KPI + sub;

  float qr[E];
  const float* qp = q + (static_cast<long>(i) * Hq + h) * DH;
#pragma unroll
  for (int e = 0; e < E; ++e) qr[e] = qp[e * L + li];
  const int S = causal ? i + 1 : T;
  float m = -INFINITY, l = 0.0f, acc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.0f;
  const long rs = static_cast<long>(Hkv) * DH;
  for (int j0 = wave * KPI; j0 < S; j0 += NS) {
    const int j = j0 + sub;
    const bool valid = j < S;
    const int jr = valid ? j : S - 1;  // in-bounds row; its weight is 0
    const float* kr = k + jr * rs + static_cast<long>(kvh) * DH;
    const float* vr = v + jr * rs + static_cast<long>(kvh) * DH;
    float d = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) d = fmaf(qr[e], kr[e * L + li], d);
#pragma unroll
    for (int off = 1; off < L; off <<= 1) d += __shfl_xor(d, off);
    const float s = valid ? d * scale_log2e : -INFINITY;
    const float mn = fmaxf(m, s);
    const float mr = mn == -INFINITY ? 0.0f : mn;
    const float corr = fast_exp2(m - mr);
    const float p = fast_exp2(s - mr);
    l = l * corr + p;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = fmaf(p, vr[e * L + li], acc[e] * corr);
    m = mn;
  }
  if (li == 0) {
    s_ml[slot][0] = m;
    s_ml[slot][1] = l;
  }
#pragma unroll
  for (int e = 0; e < E; ++e) s_o[slot][e * L + li] = acc[e];
  __syncthreads();
  for (int d = threadIdx.x; d < DH; d += 64 * kGenWaves) {
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < NS; ++t) mx = fmaxf(mx, s_ml[t][0]);
    const float mr = mx == -INFINITY ? 0.0f : mx;
    float ov = 0.0f, lv = 0.0f;
#pragma unroll
    for (int t = 0; t < NS; ++t) {
      const float wt = fast_exp2(s_ml[t][0] - mr);  // empty slots: 2^-inf = 0
      ov = fmaf(wt, s_o[t][d], ov);
      lv = fmaf(wt, s_ml[t][1], lv);
    }
    out[(static_cast<long>(i) * Hq + h) * DH + d] = lv > 0.0f ? ov * (1.0f / lv) : 0.0f;
  }
}

template <int DH>
int launch_dh(const float* q, const float* k, const float* v, float* out, int T, int Hq, int Hkv,
              float scale, bool causal, hipStream_t s) {
  hipLaunchKernelGGL(gqa_attention_generic_kernel<DH>, dim3(T, Hq), dim3(64 * kGenWaves), 0, s,
                     q, k, v, out, T, Hq, Hkv, scale * 1.4426950408889634f, causal ? 1 : 0);
  return check_launch("gqa_attention_generic_kernel");
}

}  // namespace

int launch_gqa_attention_generic(const float* q, const float* k, const float* v, float* out,
                                 int T, int Hq, int Hkv, int Dh, float scale, bool causal,
                                 hipStream_t s) {
  if (Hq > 65535) return fail(ORATOR_ERR_UNSUPPORTED, "gqa_attention: at most 65535 q heads");
  switch (Dh) {
    case 1: return launch_dh<1>(q, k, v, out, T, Hq, Hkv, scale, causal, s);
    case 2: return launch_dh<2>(q, k, v, out, T, Hq, Hkv, scale, causal, s);
    case 4: return launch_dh<4>(q, k, v, out, T, Hq, Hkv, scale, causal, s);
    case 8: return launch_dh<8>(q, k, v, out, T, Hq, Hkv, scale, causal, s);
    case 16: return launch_dh<16>(q, k, v, out, T, Hq, Hkv, scale, causal, s);
    case 32: return launch_dh<32>(q, k, v, out, T, Hq, Hkv, scale, causal, s);
    case 64: return launch_dh<64>(q, k, v, out, T, Hq, Hkv, scale, causal, s);
    case 128: return launch_dh<128>(q, k, v, out, T, Hq, Hkv, scale, causal, s);
    case 256: return launch_dh<256>(q, k, v, out, T, Hq, Hkv, scale, causal, s);
    case 512: return launch_dh<512>(q, k, v, out, T, Hq, Hkv, scale, causal, s);
    case 1024: return launch_dh<1024>(q, k, v, out, T, Hq, Hkv, scale, causal, s);
    default:
      return fail(ORATOR_ERR_UNSUPPORTED, "gqa_attention: Dh must be a power of two <= 1024");
  }
}

}  // namespace orator_hip
