// Self-attention over per-query key ranges, fp32 throughout, on fp32 MFMA (gfx950).
//
// Serves two small fp32 self-attentions over [N, H, Dk] rows:
//  * the audio tower's windowed attention (WindowAttnKernel, src/model/asr_audio_tower.cu:
//    204-258): query i attends keys [seg_start[i], seg_end[i]), clamped into [0, N); zeros for
//    an empty window;
//  * the Sortformer decoder's masked MHA (src/model/sortformer_decoder.cu:280-298): every query
//    attends keys [0, valid_len); with valid_len <= 0 every key gets the reference's score
//    -1e30, so the softmax is uniform over all N keys (score 0 here).
// Scores (q . k) * scale, online softmax, out = (P V) * (1 / sum P).
//
// Workgroup = (32-query block, head), NW waves.  The block's queries attend the union of their
// ranges, cut into 32-key tiles; wave w takes tiles w, w + NW, ..., keeps an online softmax per
// query and the waves merge (max, sum, P V) through LDS at the end.  Per tile, on
// v_mfma_f32_32x32x2_f32:
//   S^T[j][i] = K[j] . q_i        k-step s pairs dims s (lower half-wave) and DK/2 + s
//                                  (upper): a lane reads DK/2 contiguous floats of one key
//                                  row, and of its query row for the other operand;
//   O^T[d][i] += V^T[d][j] P^T[j][i]   k-step kp pairs keys 8 (kp / 4) + kp % 4 and that + 4,
//                                  the keys of score register kp in the two half-waves, so the
//                                  weights go from the score registers straight into the
//                                  MFMA, and the V^T operand is one float per lane (128
//                                  contiguous bytes of a key row per half-wave).
// Each lane therefore owns one query column of both products: the maximum, the sum and the
// rescale of O^T are in-lane, plus one exchange of the two half-waves' maxima.  Products are
// exact fp32 and accumulate in fp32.  The weights are exp2((score - max) * log2(e)) of the
// scaled scores: the difference is formed in the reference's units, so the one extra rounding
// (the product with log2(e)) scales with score - max, small for the weights that matter; on the
// parity cases this sits as close to the fp64 value as OCML's expf does (1.70x / 1.74x the
// oracle's distance at worst) in fewer instructions, where exp2 of log2(e)-prescaled scores
// (a rounding proportional to the score itself) measured 2.25x.  Each wave computes its tiles
// in turn (a tile's loads, then its products); the waves of a SIMD overlap one another's.
#include <climits>

#include "common.hpp"
#include "internal.hpp"

namespace orator_hip {
namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));
constexpr float kLog2e = 1.4426950408889634f;

struct RangeArgs {
  const float* q;
  const float* k;
  const float* v;
  float* out;
  const int* seg_start;  // per-query ranges, or nullptr: keys [0, valid)
  const int* seg_end;
  int N, H;
  int valid;  // without ranges: keys [0, valid); <= 0: uniform softmax over all N keys
  float scale;
};

__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) v = min(v, __shfl_xor(v, d));
  return v;
}
__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) v = max(v, __shfl_xor(v, d));
  return v;
}

// One 32-key tile as the two MFMA products read it: K row (tile key lane % 32), dims
// (lane / 32) * DK / 2 + 0 .. DK / 2 - 1; V[key of score register kp in this half-wave]
// [32 db + lane % 32] (0 past DK).
template <int DK>
struct RangeTile {
  static constexpr int KQ = DK / 8;           // float4 per lane of a K (or q) row half
  static constexpr int NB = (DK + 31) / 32;   // 32-dim blocks of the output
  float4 k[KQ];
  float v[16][NB];
};

template <int DK>
__device__ __forceinline__ void load_tile(RangeTile<DK>& t, const float* kh, const float* vh,
                                          long rs, int k0, int klast, int j32, int hf) {
  using T = RangeTile<DK>;
  const float* kr = kh + static_cast<long>(min(k0 + j32, klast)) * rs + hf * (DK / 2);
#pragma unroll
  for (int f = 0; f < T::KQ; ++f) t.k[f] = *reinterpret_cast<const float4*>(kr + 4 * f);
#pragma unroll
  for (int kp = 0; kp < 16; ++kp) {
    const float* vr =
        vh + static_cast<long>(min(k0 + 8 * (kp >> 2) + 4 * hf + (kp & 3), klast)) * rs;
#pragma unroll
    for (int db = 0; db < T::NB; ++db) {
      // branch-free: every lane loads (dims past DK clamped), lanes past DK then hold 0
      const int d = 32 * db + j32;
      const float x = vr[min(d, DK - 1)];
      t.v[kp][db] = DK % 32 == 0 || d < DK ? x : 0.0f;
    }
  }
}

template <int DK>
__device__ __forceinline__ float kq_elem(const float4 (&x)[DK / 8], int s) {
  const float4 w = x[s >> 2];
  return (s & 3) == 0 ? w.x : (s & 3) == 1 ? w.y : (s & 3) == 2 ? w.z : w.w;
}

template <int DK, int NW, bool PP>
__global__ __launch_bounds__(64 * NW) void range_attn_kernel(RangeArgs a) {
  using T = RangeTile<DK>;
  constexpr int NB = T::NB;
  constexpr int NT = 64 * NW;
  __shared__ float s_o[NW][NB * 32][33];  // [wave][dim][query], padded against bank conflicts
  __shared__ float s_ml[NW][2][32];

  const int h = blockIdx.y;
  const int q0 = blockIdx.x * 32;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j32 = lane & 31, hf = lane >> 5;
  const int N = a.N;
  const long rs = static_cast<long>(a.H) * DK;  // floats between rows

  // ---- this lane's query and key range; the block's union ----
  const int qi = q0 + j32;
  const bool uniform = !a.seg_start && a.valid <= 0;
  int lo, hi;
  if (a.seg_start) {
    const int qc = min(qi, N - 1);
    lo = min(max(a.seg_start[qc], 0), N);
    hi = min(max(a.seg_end[qc], lo), N);
  } else {
    lo = 0;
    hi = a.valid > 0 ? min(a.valid, N) : N;
  }
  if (qi >= N) hi = lo;  // no query: no keys
  const bool any = lo < hi;
  const int ulo = wave_min_i(any ? lo : INT_MAX);
  const int uhi = wave_max_i(any ? hi : INT_MIN);
  const int n_tiles = ulo < uhi ? (uhi - ulo + 31) / 32 : 0;
  const int klast = max(uhi - 1, 0);

  // q^T: the S product's B operand, DK / 2 dims of this lane's query row
  float4 qf[T::KQ];
  {
    const float* qr = a.q + static_cast<long>(min(qi, N - 1)) * rs + static_cast<long>(h) * DK +
                      hf * (DK / 2);
#pragma unroll
    for (int f = 0; f < T::KQ; ++f) qf[f] = *reinterpret_cast<const float4*>(qr + 4 * f);
  }
  const float* kh = a.k + static_cast<long>(h) * DK;
  const float* vh = a.v + static_cast<long>(h) * DK;

  float m = -INFINITY, lsum = 0.0f;
  f32x16_t o[NB];
#pragma unroll
  for (int db = 0; db < NB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[db][e] = 0.0f;

  auto compute = [&](const T& t, int k0) {
    f32x16_t s;
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < DK / 2; ++ks)
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kq_elem<DK>(t.k, ks), kq_elem<DK>(qf, ks), s, 0,
                                               0, 0);
    // scores of keys k0 + 8 (e / 4) + 4 hf + e % 4 for query qi
    float tmax = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int key = k0 + 8 * (e >> 2) + 4 * hf + (e & 3);
      const float x = uniform ? 0.0f : s[e] * a.scale;
      s[e] = key >= lo && key < hi ? x : -INFINITY;
      tmax = fmaxf(tmax, s[e]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float mn = fmaxf(m, tmax);
    const float corr = m == mn ? 1.0f : fast_exp2((m - mn) * kLog2e);  // m = -inf: nothing yet
    float psum = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      s[e] = s[e] == -INFINITY ? 0.0f : fast_exp2((s[e] - mn) * kLog2e);
      psum += s[e];
    }
    lsum = fmaf(lsum, corr, psum);
    m = mn;
    if (__builtin_amdgcn_ballot_w64(corr != 1.0f)) {
#pragma unroll
      for (int db = 0; db < NB; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[db][e] *= corr;
    }
#pragma unroll
    for (int kp = 0; kp < 16; ++kp)
#pragma unroll
      for (int db = 0; db < NB; ++db)
        o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(t.v[kp][db], s[kp], o[db], 0, 0, 0);
  };

  const int n_my = wave < n_tiles ? (n_tiles - wave + NW - 1) / NW : 0;
  if constexpr (PP) {  // the next tile's loads in flight while the current one is computed
    // (needs a second tile's registers: fewer waves per workgroup; not faster at the callers'
    // shapes, where a wave has one or two tiles)
    if (n_my > 0) {
      T A, B;
      load_tile<DK>(A, kh, vh, rs, ulo + 32 * wave, klast, j32, hf);
      for (int i = 0;;) {
        const int k0 = ulo + 32 * (wave + NW * i);
        if (i + 1 < n_my) load_tile<DK>(B, kh, vh, rs, k0 + 32 * NW, klast, j32, hf);
        compute(A, k0);
        if (++i >= n_my) break;
        const int k1 = k0 + 32 * NW;
        if (i + 1 < n_my) load_tile<DK>(A, kh, vh, rs, k1 + 32 * NW, klast, j32, hf);
        compute(B, k1);
        if (++i >= n_my) break;
      }
    }
  } else {
    for (int i = 0; i < n_my; ++i) {
      const int k0 = ulo + 32 * (wave + NW * i);
      T A;
      load_tile<DK>(A, kh, vh, rs, k0, klast, j32, hf);
      compute(A, k0);
    }
  }

  // ---- merge the waves' partials through LDS ----
  const float L = lsum + __shfl_xor(lsum, 32);  // the half-waves summed different keys
  if (hf == 0) {
    s_ml[wave][0][j32] = m;
    s_ml[wave][1][j32] = L;
  }
#pragma unroll
  for (int db = 0; db < NB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e)
      s_o[wave][32 * db + 8 * (e >> 2) + 4 * hf + (e & 3)][j32] = o[db][e];
  __syncthreads();
  for (int idx = tid; idx < 32 * DK; idx += NT) {
    const int d = idx % DK, qq = idx / DK;
    const int qo = q0 + qq;
    if (qo >= N) break;  // idx / DK only grows
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s_ml[w][0][qq]);
    float ov = 0.0f, lv = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float mw = s_ml[w][0][qq];
        const float wt = mw == -INFINITY ? 0.0f : fast_exp2((mw - M) * kLog2e);
        ov = fmaf(wt, s_o[w][d][qq], ov);
        lv = fmaf(wt, s_ml[w][1][qq], lv);
      }
    }
    a.out[static_cast<long>(qo) * rs + static_cast<long>(h) * DK + d] =
        lv > 0.0f ? ov * (1.0f / lv) : 0.0f;
  }
}

template <int DK, int NW, bool PP>
int launch_range(const RangeArgs& a, hipStream_t s) {
  const dim3 grid((a.N + 31) / 32, a.H);
  hipLaunchKernelGGL((range_attn_kernel<DK, NW, PP>), grid, dim3(64 * NW), 0, s, a);
  return check_launch("range_attn_kernel");
}

}  // namespace

int launch_range_attention(const float* q, const float* k, const float* v, float* out,
                           const int* seg_start, const int* seg_end, int N, int H, int Dk,
                           int valid, float scale, hipStream_t s) {
  if (N <= 0 || H <= 0) return ORATOR_OK;
  if (!(Dk == 24 || Dk == 32 || Dk == 64))
    return fail(ORATOR_ERR_UNSUPPORTED, "range_attention: Dk must be 24, 32 or 64");
  if (H > 65535) return fail(ORATOR_ERR_UNSUPPORTED, "range_attention: at most 65535 heads");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
       reinterpret_cast<uintptr_t>(v)) & 15u)
    return fail(ORATOR_ERR_INVALID, "range_attention: q, k, v must be 16-byte aligned");
  RangeArgs a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.seg_start = seg_start;
  a.seg_end = seg_end;
  a.N = N;
  a.H = H;
  a.valid = valid;
  a.scale = scale;
  // waves per workgroup: as many as the registers of a double-buffered tile allow unspilled
  // (256 per lane at 2 waves per SIMD for Dk <= 32; Dk = 64 needs ~230 + addresses: 1 wave)
  if (Dk == 24) return launch_range<24, 16, false>(a, s);
  if (Dk == 32) return launch_range<32, 16, false>(a, s);
  return launch_range<64, 8, false>(a, s);
}

}  // namespace orator_hip

using namespace orator_hip;

extern "C" {

// The Sortformer decoder's self-attention (src/model/sortformer_decoder.cu:280-298).
int orator_masked_mha(const float* q, const float* k, const float* v, float* out, int T, int H,
                      int Dk, int valid_len, float scale, void* stream) {
  if (T <= 0 || H <= 0 || Dk <= 0) return ORATOR_OK;
  if (!q || !k || !v || !out) return fail(ORATOR_ERR_INVALID, "masked_mha: null pointer");
  return launch_range_attention(q, k, v, out, nullptr, nullptr, T, H, Dk, valid_len, scale,
                                static_cast<hipStream_t>(stream));
}

}  // extern "C"
