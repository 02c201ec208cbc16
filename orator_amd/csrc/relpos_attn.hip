// FastConformer relative-position MHSA core (Transformer-XL u/v biases), gfx950.
//
// Replaces the attention block of ConformerLayer::Forward (src/model/conformer_layer.cu:405-444):
//   AC[h,i,j] = (q_i + u_h) . k_j,   BD[h,i,m] = (q_i + v_h) . p_m  (m over 2T-1 rel. positions)
//   score[h,i,j] = (AC[h,i,j] + BD[h,i,T-1-i+j]) * scale   for j < valid, else -1e30
//   out[i,h,:] = softmax_j(score[h,i,:]) . v
// q, k, v [T,H,Dk], p [2T-1,H,Dk] (linear_pos output), u, v_bias [H,Dk]; out [T,H,Dk]
// (the context before linear_out).  BD[h,i,T-1-i+j] is the closed form of the reference's
// rel_shift index arithmetic (RelShiftScoresKernel, :130-155).
//
// fp32 mode keeps the reference's decomposition -- head-major gathers, batched fp32 GEMMs
// for AC, BD and the context -- so its arithmetic is the reference's up to summation
// order; the rel-shift, mask, scale and row softmax are fused into one row kernel.
#include "common.hpp"
#include "internal.hpp"

namespace orator_hip {
namespace {

// qu[h,t,d] = q[t,h,d] + u[h,d]; qv likewise with v_bias; kh[h,t,d] = k[t,h,d];
// ph[h,m,d] = p[m,h,d]; vt[h,d,t] = v[t,h,d].
__global__ __launch_bounds__(256) void relpos_gather_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ p, const float* __restrict__ u, const float* __restrict__ vb,
    float* __restrict__ qu, float* __restrict__ qv, float* __restrict__ kh,
    float* __restrict__ ph, float* __restrict__ vt, int T, int H, int Dk) {
  const long n = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int P = 2 * T - 1;
  const long ntd = static_cast<long>(H) * T * Dk;
  const long npd = static_cast<long>(H) * P * Dk;
  if (n < ntd) {
    const int d = static_cast<int>(n % Dk);
    const int t = static_cast<int>((n / Dk) % T);
    const int h = static_cast<int>(n / (static_cast<long>(Dk) * T));
    const long src = (static_cast<long>(t) * H + h) * Dk + d;
    const float qq = q[src];
    qu[n] = qq + u[h * Dk + d];
    qv[n] = qq + vb[h * Dk + d];
    kh[n] = k[src];
    vt[(static_cast<long>(h) * Dk + d) * T + t] = v[src];
  }
  if (n < npd) {
    const int d = static_cast<int>(n % Dk);
    const int m = static_cast<int>((n / Dk) % P);
    const int h = static_cast<int>(n / (static_cast<long>(Dk) * P));
    ph[n] = p[(static_cast<long>(m) * H + h) * Dk + d];
  }
}

// One workgroup per (h, i) row: score = (AC + BD[T-1-i+j]) * scale (j < valid), softmax in
// place over the row, AttnSoftmaxKernel's max / exp / 1/sum order (:158-192).
__global__ __launch_bounds__(256) void relpos_softmax_kernel(float* __restrict__ ac,
                                                             const float* __restrict__ bd, int T,
                                                             int valid, float scale) {
  __shared__ float red[4];
  const int row = blockIdx.x;  // h*T + i
  const int i = row % T;
  const int P = 2 * T - 1;
  float* s = ac + static_cast<long>(row) * T;
  const float* bdr = bd + static_cast<long>(row) * P + (T - 1 - i);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float mx = -1e30f;
  for (int j = tid; j < T; j += 256) {
    const float x = j < valid ? (s[j] + bdr[j]) * scale : -1e30f;
    s[j] = x;
    mx = fmaxf(mx, x);
  }
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sum = 0.0f;
  for (int j = tid; j < T; j += 256) {
    const float e = expf(s[j] - mx);
    s[j] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  const float inv = 1.0f / (red[0] + red[1] + red[2] + red[3]);
  for (int j = tid; j < T; j += 256) s[j] *= inv;
}

// out[t,h,d] = ctx[h,t,d]
__global__ __launch_bounds__(256) void relpos_scatter_kernel(const float* __restrict__ ctx,
                                                             float* __restrict__ out, int T, int H,
                                                             int Dk) {
  const long n = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (n >= static_cast<long>(H) * T * Dk) return;
  const int d = static_cast<int>(n % Dk);
  const int t = static_cast<int>((n / Dk) % T);
  const int h = static_cast<int>(n / (static_cast<long>(Dk) * T));
  out[(static_cast<long>(t) * H + h) * Dk + d] = ctx[n];
}

inline int blocks(long n) { return static_cast<int>((n + 255) / 256); }

int relpos_fp32(const float* q, const float* k, const float* v, const float* p, const float* u,
                const float* vb, float* out, int T, int H, int Dk, int valid, float scale,
                hipStream_t stream) {
  const int P = 2 * T - 1;
  const size_t td = static_cast<size_t>(H) * T * Dk, pd = static_cast<size_t>(H) * P * Dk;
  const size_t tt = static_cast<size_t>(H) * T * T, tp = static_cast<size_t>(H) * T * P;
  const size_t floats = 4 * td + pd + td /*vt*/ + tt + tp;
  float* ws = static_cast<float*>(workspace(stream, floats * sizeof(float)));
  if (!ws) return ORATOR_ERR_HIP;
  float* qu = ws;
  float* qv = qu + td;
  float* kh = qv + td;
  float* ctx = kh + td;
  float* vt = ctx + td;
  float* ph = vt + td;
  float* ac = ph + pd;
  float* bd = ac + tt;
  hipLaunchKernelGGL(relpos_gather_kernel, dim3(blocks(static_cast<long>(pd > td ? pd : td))),
                     dim3(256), 0, stream, q, k, v, p, u, vb, qu, qv, kh, ph, vt, T, H, Dk);
  int rc = check_launch("relpos_gather");
  if (rc) return rc;
  rc = launch_sgemm(qu, kh, nullptr, ac, T, Dk, T, 0, H, static_cast<long>(T) * Dk,
                    static_cast<long>(T) * Dk, static_cast<long>(T) * T, stream);
  if (rc) return rc;
  rc = launch_sgemm(qv, ph, nullptr, bd, T, Dk, P, 0, H, static_cast<long>(T) * Dk,
                    static_cast<long>(P) * Dk, static_cast<long>(T) * P, stream);
  if (rc) return rc;
  hipLaunchKernelGGL(relpos_softmax_kernel, dim3(H * T), dim3(256), 0, stream, ac, bd, T, valid,
                     scale);
  rc = check_launch("relpos_softmax");
  if (rc) return rc;
  rc = launch_sgemm(ac, vt, nullptr, ctx, T, T, Dk, 0, H, static_cast<long>(T) * T,
                    static_cast<long>(Dk) * T, static_cast<long>(T) * Dk, stream);
  if (rc) return rc;
  hipLaunchKernelGGL(relpos_scatter_kernel, dim3(blocks(static_cast<long>(td))), dim3(256), 0,
                     stream, ctx, out, T, H, Dk);
  return check_launch("relpos_scatter");
}

}  // namespace
}  // namespace orator_hip

using namespace orator_hip;

extern "C" {

int orator_relpos_attention(const float* q, const float* k, const float* v, const float* p,
                            const float* pos_bias_u, const float* pos_bias_v, float* out, int T,
                            int H, int Dk, int valid_len, float scale, void* stream) {
  if (T <= 0 || H <= 0 || Dk <= 0) return ORATOR_OK;
  if (!q || !k || !v || !p || !pos_bias_u || !pos_bias_v || !out)
    return fail(ORATOR_ERR_INVALID, "relpos_attention: null pointer");
  if (valid_len > T) valid_len = T;
  return relpos_fp32(q, k, v, p, pos_bias_u, pos_bias_v, out, T, H, Dk, valid_len, scale,
                     static_cast<hipStream_t>(stream));
}

}  // extern "C"

// ===================================================================== fused fp16 path
//
// One workgroup = one (head, 32-query tile); its 8 wave64s split the key range (tiles of 32
// keys, wave w takes tiles w, w+8, ...) and merge (max, sum, acc) through LDS at the end.
// Per key tile and wave, on v_mfma_f32_32x32x16_f16 (S^T orientation, so the softmax
// state is per lane = per query column):
//   AC^T[j][i] = K[j] . (q_i + u)                  4 MFMAs
//   R[r][i]    = P[base + r] . (q_i + v), r < 64   8 MFMAs, base = T-1-(i0+31)+j0
//   BD^T[j][i] = R[j - i + 31][i]                  (the rel shift: R goes through LDS)
//   O^T[d][i] += V^T[d][j] P^T[j][i]               4 MFMAs, V^T staged through LDS
// so the BD band costs 2x the MFMA work of AC instead of a [H,T,2T-1] GEMM through HBM.
// Inputs fp16 (or fp32 converted on load), u/v biases fp32, output fp32.
namespace orator_hip {
namespace {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kRpDk = 64;
constexpr int kRpWaves = 8;
constexpr int kVRowH = 64 + 32;  // row-major V tile row (halves): 192 bytes, so the 4 rows
                                 // of a half-wave's transposing read start 48 banks apart
constexpr int kRtRow = 64 + 2;   // R^T row (floats): the diagonal band reads [c][jl - c + 31]
                                 // then fall on distinct banks across the 32 columns
constexpr int kStRow = 64 + 8;   // staged K / P / q row (halves): 144 bytes, so the A-fragment
                                 // reads of 16 lanes (rows r, 16 bytes each) hit distinct banks

__device__ __forceinline__ f16x8_t as_f16x8(uint4 u) { return __builtin_bit_cast(f16x8_t, u); }

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  const _Float16 ha = static_cast<_Float16>(a), hb = static_cast<_Float16>(b);
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, ha)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hb)) << 16);
}

// 8 consecutive elements as fp16 bits (converting fp32 input).
template <typename IN>
__device__ __forceinline__ uint4 load8_h(const IN* p) {
  if constexpr (sizeof(IN) == 2) {
    return *reinterpret_cast<const uint4*>(p);
  } else {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    return make_uint4(pack_h2(a.x, a.y), pack_h2(a.z, a.w), pack_h2(b.x, b.y), pack_h2(b.z, b.w));
  }
}

template <typename IN>
__device__ __forceinline__ void load8_f(const IN* p, float (&x)[8]) {
  if constexpr (sizeof(IN) == 2) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[e] & 0xffffu)));
      x[2 * e + 1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[e] >> 16)));
    }
  } else {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  }
}

// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives element (i & 3) of the
// 8 bytes addressed by lane 4k + (i >> 2), k = 0..3; with lane s pointing at row r0 + (s >> 2),
// columns c0 + 4 (s & 3) of a row-major 16-bit tile, lane i gets column c0 + i of rows
// r0 .. r0 + 3.
typedef short rp_s16x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t* p) {
  typedef __attribute__((address_space(3))) rp_s16x4_t lds_s16x4_t;
  const rp_s16x4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p));
  return __builtin_bit_cast(uint2, r);
}

// Inline-asm v_mfma_f32_32x32x16_f16 for the score products.  The hardware does not interlock
// them with other instructions; the wait states are placed by hand: s_nop 1 before each (an
// operand written by a VALU instruction needs 2 wait states before an MFMA reads it), and
// rp_mfma_result_guard() (12 wait states for an 8-pass MFMA) between the last of them and
// the first VALU or LDS read of their results.  A chain accumulating into the same registers
// needs none.
typedef unsigned rp_u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void rp_mfma0(f32x16_t& d, uint4 a, uint4 b) {
  const rp_u32x4_t x = __builtin_bit_cast(rp_u32x4_t, a), y = __builtin_bit_cast(rp_u32x4_t, b);
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(d) : "v"(x), "v"(y));
}
__device__ __forceinline__ void rp_mfma(f32x16_t& d, uint4 a, uint4 b) {
  const rp_u32x4_t x = __builtin_bit_cast(rp_u32x4_t, a), y = __builtin_bit_cast(rp_u32x4_t, b);
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(d) : "v"(x), "v"(y));
}
__device__ __forceinline__ void rp_mfma_result_guard() { asm volatile("s_nop 7\n\ts_nop 4" ::); }

struct RelPosArgs {
  const void *q, *k, *v, *p;
  const float *u, *vb;
  float* out;
  int T, H, valid;
  float scale_log2e;
  int uniform;  // every key masked (valid_len <= 0): all T scores equal, softmax = mean of V
};

// QT: the q rows' type; IN: the k, v and p rows' type (fp32 or fp16 bits).
template <typename QT, typename IN>
__global__ __launch_bounds__(64 * kRpWaves) void relpos_fused_kernel(RelPosArgs a) {
  // Each wave's LDS area holds, per key tile, first the tile's K rows and P window (row-major,
  // padded; the MFMA A fragments are read back from them), then the V tile and R^T; after the
  // key loop its R^T part holds the wave's partial output [dim][query] for the merge.  Before
  // the loop the workgroup's (q + u), (q + v) rows are staged at the start of the areas.
  constexpr int kVBytes = 32 * kVRowH * 2;
  constexpr int kWaveBytes = kVBytes + 32 * kRtRow * 4;
  static_assert((32 + 64) * kStRow * 2 <= kWaveBytes, "K / P staging fits a wave's area");
  static_assert(2 * 32 * kStRow * 2 <= kRpWaves * kWaveBytes, "q staging fits");
  static_assert(kRpDk * 33 * 4 <= kWaveBytes - kVBytes, "the merge area fits a wave's R^T area");
  __shared__ __align__(16) unsigned char lds[kRpWaves * kWaveBytes];
  __shared__ float mo_lds[kRpWaves][2][32];
  auto o_lds = [&](int w, int d, int c) -> float& {
    return reinterpret_cast<float*>(lds + w * kWaveBytes + kVBytes)[d * 33 + c];
  };

  const int h = blockIdx.x % a.H;
  const int i0 = (blockIdx.x / a.H) * 32;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar tile offsets
  const int col = lane & 31, h2 = lane >> 5;
  const int T = a.T, H = a.H;
  const long rs = static_cast<long>(H) * kRpDk;  // elements per token row
  const QT* qp = static_cast<const QT*>(a.q);
  const IN* kp = static_cast<const IN*>(a.k);
  const IN* vp = static_cast<const IN*>(a.v);
  const IN* pp = static_cast<const IN*>(a.p);

  unsigned char* wl = lds + wave * kWaveBytes;
  uint16_t* const kst = reinterpret_cast<uint16_t*>(wl);  // staged K rows [32][kStRow]
  uint16_t* const pst = kst + 32 * kStRow;                 // staged P window [64][kStRow]
  uint16_t* const vt = reinterpret_cast<uint16_t*>(wl);   // V tile [32][kVRowH]
  float* const rt = reinterpret_cast<float*>(wl + kVBytes);  // R^T [32][kRtRow]

  const int n_tiles = (a.valid + 31) / 32;
  const int P = 2 * T - 1;

  // One tile's global operands, row-contiguous (8 lanes per 128-byte row): V and K rows
  // j0 .. j0+31 and the P window base .. base+63.  Loaded through buffer resources whose
  // range is the tensor: rows outside [0, T) / [0, P) read as zeros with no branch, so the
  // compiler can count the next tile's loads and wait only for the current one's.
  constexpr int kES = sizeof(IN);
  const int row_bytes = static_cast<int>(rs) * kES;
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<IN*>(kp), 0, T * row_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<IN*>(vp), 0, T * row_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t prs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<IN*>(pp), 0, P * row_bytes, 0x00020000);
  struct Tile {
    uint4 v[4], k[4], p[8];
  };
  const int dcv = lane & 7, rv = lane >> 3;
  const int lane_off = rv * row_bytes + (h * kRpDk + 8 * dcv) * kES;
  auto bload8 = [&](__amdgpu_buffer_rsrc_t r, int off) -> uint4 {
    if constexpr (kES == 2) {
      return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
    } else {
      const float4 x = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
      const float4 y = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, 0));
      return make_uint4(pack_h2(x.x, x.y), pack_h2(x.z, x.w), pack_h2(y.x, y.y), pack_h2(y.z, y.w));
    }
  };
  auto load_kp = [&](Tile& t, int n) {
    const int j0 = 32 * n;
    const int base = T - 1 - (i0 + 31) + j0;  // may be negative: those rows read zeros
#pragma unroll
    for (int it = 0; it < 4; ++it) t.k[it] = bload8(krs, (j0 + 8 * it) * row_bytes + lane_off);
#pragma unroll
    for (int it = 0; it < 8; ++it) t.p[it] = bload8(prs, (base + 8 * it) * row_bytes + lane_off);
  };
  auto load_v = [&](Tile& t, int n) {
#pragma unroll
    for (int it = 0; it < 4; ++it)
      t.v[it] = bload8(vrs, (32 * n + 8 * it) * row_bytes + lane_off);
  };
  // the wave's first tile is in flight while q is staged
  Tile t;
  if (wave < n_tiles) {
    load_kp(t, wave);
    load_v(t, wave);
  }

  // (q_i + u) and (q_i + v) of the workgroup's 32 queries, formed once with row-contiguous
  // loads (8 lanes per row), staged in LDS ([2][32][kStRow]), and read back as this lane's B
  // operand per 16-dim k-step.  (A lane per query row, in every wave, touched a cache line
  // per lane and load.)
  uint4 qu[4], qv[4];
  {
    uint16_t* qst = reinterpret_cast<uint16_t*>(lds);
    for (int it = tid; it < 32 * 8; it += 64 * kRpWaves) {
      const int c = it >> 3, d0 = 8 * (it & 7);
      // with no valid key (uniform) q + u and q + v are zero: every score is 0, the mask
      // below leaves the T keys, and the softmax averages V
      uint4 hu = make_uint4(0, 0, 0, 0), hv = hu;
      if (i0 + c < T && !a.uniform) {
        float x[8];
        load8_f(qp + (i0 + c) * rs + h * kRpDk + d0, x);
        const float* ub = a.u + h * kRpDk + d0;
        const float* vb = a.vb + h * kRpDk + d0;
        hu = make_uint4(pack_h2(x[0] + ub[0], x[1] + ub[1]), pack_h2(x[2] + ub[2], x[3] + ub[3]),
                        pack_h2(x[4] + ub[4], x[5] + ub[5]), pack_h2(x[6] + ub[6], x[7] + ub[7]));
        hv = make_uint4(pack_h2(x[0] + vb[0], x[1] + vb[1]), pack_h2(x[2] + vb[2], x[3] + vb[3]),
                        pack_h2(x[4] + vb[4], x[5] + vb[5]), pack_h2(x[6] + vb[6], x[7] + vb[7]));
      }
      *reinterpret_cast<uint4*>(qst + c * kStRow + d0) = hu;
      *reinterpret_cast<uint4*>(qst + (32 + c) * kStRow + d0) = hv;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      qu[ks] = *reinterpret_cast<const uint4*>(qst + col * kStRow + 16 * ks + 8 * h2);
      qv[ks] = *reinterpret_cast<const uint4*>(qst + (32 + col) * kStRow + 16 * ks + 8 * h2);
    }
    __syncthreads();  // the tiles below overwrite the staging area
  }

  f32x16_t o[2];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.0f;
  float m = -INFINITY, lsum = 0.0f;
  const int tg = lane >> 4, ts = lane & 15;
  const uint16_t* vsrc0 = vt + (4 * (tg >> 1) + (ts >> 2)) * kVRowH + 16 * (tg & 1) + 4 * (ts & 3);
  const float c = a.scale_log2e;
  // One register set per wave: the next tile's K and P rows are loaded as soon as this tile's
  // are in LDS, its V rows as soon as this tile's V is, so each load is in flight under the
  // rest of the tile's work.
  auto process = [&](Tile& cur, int n, int next) {
    const int j0 = 32 * n;
    wave_lds_sync();  // the previous tile's LDS reads precede this tile's writes
    // K rows and the P window -> wave-private LDS; MFMA A fragments (row j0 + col / base +
    // col / base + 32 + col, dims 16 ks + 8 h2) read back conflict-free
#pragma unroll
    for (int it = 0; it < 4; ++it)
      *reinterpret_cast<uint4*>(kst + (8 * it + rv) * kStRow + 8 * dcv) = cur.k[it];
#pragma unroll
    for (int it = 0; it < 8; ++it)
      *reinterpret_cast<uint4*>(pst + (8 * it + rv) * kStRow + 8 * dcv) = cur.p[it];
    if (next < n_tiles) load_kp(cur, next);
    wave_lds_sync();
    uint4 kf[4], pf0[4], pf1[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int d0 = 16 * ks + 8 * h2;
      kf[ks] = *reinterpret_cast<const uint4*>(kst + col * kStRow + d0);
      pf0[ks] = *reinterpret_cast<const uint4*>(pst + col * kStRow + d0);
      pf1[ks] = *reinterpret_cast<const uint4*>(pst + (32 + col) * kStRow + d0);
    }
    wave_lds_sync();  // the fragments are read before V and R^T overwrite the staging
    // V tile -> wave-private LDS, row-major; the PV operand V^T is read back transposed
#pragma unroll
    for (int it = 0; it < 4; ++it)
      *reinterpret_cast<uint4*>(vt + (8 * it + rv) * kVRowH + 8 * dcv) = cur.v[it];
    if (next < n_tiles) load_v(cur, next);
    // AC^T and R = P_window (q + v)^T
    // (inline asm: the first k-step takes the inline constant 0 as its accumulator, where the
    // compiler zeroed 48 registers with moves every tile; wait states by hand, see rp_mfma)
    f32x16_t s, r0, r1;
    rp_mfma0(s, kf[0], qu[0]);
    rp_mfma0(r0, pf0[0], qv[0]);
    rp_mfma0(r1, pf1[0], qv[0]);
#pragma unroll
    for (int ks = 1; ks < 4; ++ks) {
      rp_mfma(s, kf[ks], qu[ks]);
      rp_mfma(r0, pf0[ks], qv[ks]);
      rp_mfma(r1, pf1[ks], qv[ks]);
    }
    rp_mfma_result_guard();
    // R^T -> LDS; the lane's accumulator rows are 8i + 4*h2 + j (+32 for r1), column = col
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int rr = 8 * (e >> 2) + 4 * h2 + (e & 3);
      rt[col * kRtRow + rr] = r0[e];
      rt[col * kRtRow + 32 + rr] = r1[e];
    }
    wave_lds_sync();  // R^T and V written by all lanes before any lane reads them
    // scores (log2 units): (AC + BD) * scale; keys >= valid masked on the one tile that
    // holds them (padding query columns carry zero q rows: finite, never stored)
    float tmax = -INFINITY;
    {
      float bd[16];
#pragma unroll
      for (int e = 0; e < 16; ++e)
        bd[e] = rt[col * kRtRow + 8 * (e >> 2) + 4 * h2 + (e & 3) - col + 31];
#pragma unroll
      for (int e = 0; e < 16; ++e) s[e] = (s[e] + bd[e]) * c;
      if (j0 + 32 > a.valid) {  // uniform over the workgroup
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int jl = 8 * (e >> 2) + 4 * h2 + (e & 3);
          if (j0 + jl >= a.valid) s[e] = -INFINITY;
        }
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) tmax = fmaxf(tmax, s[e]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    // reference max moved (and O, l rescaled) only when a score exceeds it by more than 2^8:
    // weights stay <= 256 (exact in fp16's range), and most tiles skip the rescale
    if (__builtin_amdgcn_ballot_w64(tmax > m + 8.0f)) {
      const float mn = fmaxf(m, tmax);
      const float corr = m == -INFINITY ? 0.0f : fast_exp2(m - mn);
      m = mn;
      lsum *= corr;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] *= corr;
    }
    const float mref = m == -INFINITY ? 0.0f : m;
    uint4 pk[2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pv[e] = fast_exp2(s[8 * st + e] - mref);
        lsum += pv[e];
      }
      pk[st] = make_uint4(pack_h2(pv[0], pv[1]), pack_h2(pv[2], pv[3]), pack_h2(pv[4], pv[5]),
                          pack_h2(pv[6], pv[7]));
    }
    // A operand of O^T += V^T P^T: row = dim 32 dt + col, k = keys 16 st + 4 h2 + 8 (e / 4) +
    // e % 4, by ds_read_b64_tr_b16 of the row-major tile (16-lane group g covers dims
    // 16 (g & 1) .. of the 32-dim block and keys 4 (g >> 1) .., +8 for the second half)
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const uint16_t* vsrc = vsrc0 + 16 * st * kVRowH + 32 * dt;
        const uint2 v0 = lds_read_tr16(vsrc);
        const uint2 v1 = lds_read_tr16(vsrc + 8 * kVRowH);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_f16x8(make_uint4(v0.x, v0.y, v1.x, v1.y)),
                                                       as_f16x8(pk[st]), o[dt], 0, 0, 0);
      }
  };
  for (int n = wave; n < n_tiles; n += kRpWaves) process(t, n, n + kRpWaves);

  // ---- merge the waves' partial softmax states ----
  lsum += __shfl_xor(lsum, 32);
  if (h2 == 0) {
    mo_lds[wave][0][col] = m;
    mo_lds[wave][1][col] = lsum;
  }
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e)
      o_lds(wave, 32 * dt + 8 * (e >> 2) + 4 * h2 + (e & 3), col) = o[dt][e];
  __syncthreads();
  // thread -> query column qc, dims d0 .. d0 + 3: the column's wave weights once, one float4
  static_assert(32 * kRpDk == 4 * 64 * kRpWaves, "one float4 of the output per thread");
  const int qc = tid >> 4, d0 = 4 * (tid & 15);
  float mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < kRpWaves; ++w) mx = fmaxf(mx, mo_lds[w][0][qc]);
  const float mr = mx == -INFINITY ? 0.0f : mx;
  float lv = 0.0f, ov[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int w = 0; w < kRpWaves; ++w) {
    const float wt = fast_exp2(mo_lds[w][0][qc] - mr);
    lv = fmaf(wt, mo_lds[w][1][qc], lv);
#pragma unroll
    for (int e = 0; e < 4; ++e) ov[e] = fmaf(wt, o_lds(w, d0 + e, qc), ov[e]);
  }
  if (i0 + qc < T) {
    const float inv = lv > 0.0f ? 1.0f / lv : 0.0f;
    *reinterpret_cast<float4*>(a.out + (static_cast<long>(i0 + qc) * H + h) * kRpDk + d0) =
        make_float4(ov[0] * inv, ov[1] * inv, ov[2] * inv, ov[3] * inv);
  }
}

}  // namespace
}  // namespace orator_hip

extern "C" {

int orator_relpos_attention_fast(const void* q, const void* k, const void* v, const void* p,
                                 const float* pos_bias_u, const float* pos_bias_v, float* out,
                                 int T, int H, int Dk, int valid_len, float scale, int in_f16,
                                 void* stream) {
  using namespace orator_hip;
  if (T <= 0 || H <= 0 || Dk <= 0) return ORATOR_OK;
  if (!q || !k || !v || !p || !pos_bias_u || !pos_bias_v || !out)
    return fail(ORATOR_ERR_INVALID, "relpos_attention_fast: null pointer");
  if (Dk != kRpDk) return fail(ORATOR_ERR_UNSUPPORTED, "relpos_attention_fast: Dk must be 64");
  if (in_f16 < 0 || in_f16 > 2)
    return fail(ORATOR_ERR_INVALID, "relpos_attention_fast: in_f16 must be 0, 1 or 2");
  // rows are addressed with 32-bit byte offsets (buffer loads): the P tensor [2T-1][H][64]
  if (static_cast<long>(2 * T) * H * kRpDk * 4 >= (1L << 31))
    return fail(ORATOR_ERR_UNSUPPORTED, "relpos_attention_fast: (2T-1) * H * 64 * 4 >= 2^31");
  // The reference masks keys >= valid_len with a finite -1e30 (conformer_layer.cu:140-143):
  // with no valid key every score is the same and the softmax averages V over all T keys.
  const bool none_valid = valid_len <= 0;
  RelPosArgs args{q, k, v, p, pos_bias_u, pos_bias_v, out, T, H,
                  none_valid ? T : (valid_len > T ? T : valid_len), scale * 1.4426950408889634f,
                  none_valid ? 1 : 0};
  const dim3 grid(((T + 31) / 32) * H);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (in_f16 == 1)
    hipLaunchKernelGGL((relpos_fused_kernel<_Float16, _Float16>), grid, dim3(64 * kRpWaves), 0, s,
                       args);
  else if (in_f16 == 2)
    hipLaunchKernelGGL((relpos_fused_kernel<float, _Float16>), grid, dim3(64 * kRpWaves), 0, s,
                       args);
  else
    hipLaunchKernelGGL((relpos_fused_kernel<float, float>), grid, dim3(64 * kRpWaves), 0, s, args);
  return check_launch("relpos_fused_kernel");
}

}  // extern "C"
