// Small operators of the asr_ops / asr_gemm family and the decoder's KV write, gfx950.
//
// These are memory- or launch-bound; the point of each design is one pass over HBM with
// wide loads and no idle lanes:
//  * RmsNorm: one wave64 per row (the reference's 256-thread block left half its
//    threads idle on the 128-wide QK-norm rows), float4 loads, DPP reduction.
//  * RoPE: one lane per rotation pair; inv_freq, sin and cos are evaluated in fp64 from
//    the fp32 exponent and fp32 angle the reference forms, and rounded once.
//  * ArgmaxBanned keeps the reference's 256-slot strided scan + halving tree, because
//    its tie rule is part of the observable result.
#include "common.hpp"
#include "internal.hpp"

namespace orator_hip {
namespace {

constexpr int kBlock = 256;

inline int blocks_for(long n, int per_block = kBlock) {
  return static_cast<int>((n + per_block - 1) / per_block);
}

// ------------------------------------------------------------------ RmsNorm ----
// OUT = float: the reference's RmsNorm; OUT = uint16_t: RmsNorm then F32ToBf16 (RNE) of the
// same fp32 values, in one pass.  One wave per row; with VEC lane l takes float4 l, l + 64, ...
// and sums their squares in that order.  PER > 0 (VEC, dim <= 256 PER): the row and the
// weights are loaded once, all together, into registers; same arithmetic, same bits.
template <bool VEC, typename OUT = float, int PER = 0>
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ w,
                                                       OUT* out, int rows, int dim,
                                                       float eps) {
#pragma clang fp contract(off)
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* xr = x + static_cast<long>(row) * dim;
  OUT* yr = out + static_cast<long>(row) * dim;
  float local = 0.0f;
  if constexpr (PER > 0) {
    float4 v[PER], g[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int d = min(lane * 4 + 256 * i, dim - 4);
      v[i] = *reinterpret_cast<const float4*>(xr + d);
      g[i] = *reinterpret_cast<const float4*>(w + d);
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (lane * 4 + 256 * i < dim) {
        local += v[i].x * v[i].x;
        local += v[i].y * v[i].y;
        local += v[i].z * v[i].z;
        local += v[i].w * v[i].w;
      }
    }
    const float sum = wave_sum(local);
    const float ms = sum / static_cast<float>(dim) + eps;
    const float inv = rsqrt_via_f64(ms);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int d = lane * 4 + 256 * i;
      if (d >= dim) continue;
      const float4 y = make_float4(v[i].x * inv * g[i].x, v[i].y * inv * g[i].y,
                                   v[i].z * inv * g[i].z, v[i].w * inv * g[i].w);
      if constexpr (sizeof(OUT) == 4)
        *reinterpret_cast<float4*>(yr + d) = y;
      else
        *reinterpret_cast<uint2*>(yr + d) = make_uint2(pack_bf16x2(y.x, y.y), pack_bf16x2(y.z, y.w));
    }
    return;
  }
  if (VEC) {
    for (int d = lane * 4; d < dim; d += 256) {
      const float4 v = *reinterpret_cast<const float4*>(xr + d);
      local += v.x * v.x;
      local += v.y * v.y;
      local += v.z * v.z;
      local += v.w * v.w;
    }
  } else {
    for (int d = lane; d < dim; d += 64) local += xr[d] * xr[d];
  }
  const float sum = wave_sum(local);
  const float ms = sum / static_cast<float>(dim) + eps;
  const float inv = rsqrt_via_f64(ms);
  if (VEC) {
    for (int d = lane * 4; d < dim; d += 256) {
      const float4 v = *reinterpret_cast<const float4*>(xr + d);
      const float4 g = *reinterpret_cast<const float4*>(w + d);
      const float4 y =
          make_float4(v.x * inv * g.x, v.y * inv * g.y, v.z * inv * g.z, v.w * inv * g.w);
      if constexpr (sizeof(OUT) == 4)
        *reinterpret_cast<float4*>(yr + d) = y;
      else
        *reinterpret_cast<uint2*>(yr + d) = make_uint2(pack_bf16x2(y.x, y.y), pack_bf16x2(y.z, y.w));
    }
  } else {
    for (int d = lane; d < dim; d += 64) {
      const float y = xr[d] * inv * w[d];
      if constexpr (sizeof(OUT) == 4)
        yr[d] = y;
      else
        yr[d] = f32_to_bf16(y);
    }
  }
}

// --------------------------------------------------------------------- RoPE ----
__device__ __forceinline__ void rope_cs(float p, float base, int j, int head_dim, float* c,
                                        float* s) {
  const float e = -2.0f * static_cast<float>(j) / static_cast<float>(head_dim);
  const float inv_freq = static_cast<float>(pow(static_cast<double>(base), static_cast<double>(e)));
  const float angle = p * inv_freq;
  double sd, cd;
  sincos(static_cast<double>(angle), &sd, &cd);
  *c = static_cast<float>(cd);
  *s = static_cast<float>(sd);
}

template <bool HALF>
__global__ __launch_bounds__(256) void rope_kernel(float* __restrict__ x,
                                                   const int* __restrict__ pos, int T, int H,
                                                   int Dh, float base) {
#pragma clang fp contract(off)
  const int half = Dh / 2;
  const long idx = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  const long total = static_cast<long>(T) * H * half;
  if (idx >= total) return;
  const int j = static_cast<int>(idx % half);
  const long th = idx / half;
  const int t = static_cast<int>(th / H);
  float* xr = x + th * Dh;
  float c, s;
  rope_cs(static_cast<float>(pos[t]), base, j, Dh, &c, &s);
  if (HALF) {
    const float a = xr[j];
    const float b = xr[j + half];
    xr[j] = a * c - b * s;
    xr[j + half] = b * c + a * s;
  } else {
    const float a = xr[2 * j];
    const float b = xr[2 * j + 1];
    xr[2 * j] = a * c - b * s;
    xr[2 * j + 1] = a * s + b * c;
  }
}

// (cos, sin) of RoPE pair j (head_dim 128) at position p: out[(p * 64 + j) * 2 + {0, 1}].
__global__ __launch_bounds__(256) void rope_table_kernel(float* __restrict__ out, int n_pos,
                                                         float theta) {
  const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<long>(n_pos) * 64) return;
  float c, s;
  rope_cs(static_cast<float>(i / 64), theta, static_cast<int>(i % 64), 128, &c, &s);
  out[2 * i] = c;
  out[2 * i + 1] = s;
}

// ------------------------------------------------------------------- SwiGLU ----
__global__ __launch_bounds__(256) void swiglu_kernel(const float* g, const float* u, float* o,
                                                     int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float gv = g[i];
  o[i] = (gv / (1.0f + expf(-gv))) * u[i];
}

// SwiGLU of a fused gate|up row block gu [T][2I] (gate = columns [0, I), up = [I, 2I)) with
// the bf16 cast of the down projection's input folded in: out[t][i] = bf16(silu(g) * u), the
// same fp32 value as swiglu_kernel's.  4 columns per thread (I % 4 == 0).
__global__ __launch_bounds__(256) void swiglu_bf16_kernel(const float* __restrict__ gu,
                                                          uint16_t* __restrict__ out, int T,
                                                          int I) {
  const long i4 = 4 * (static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x);
  if (i4 >= static_cast<long>(T) * I) return;
  const long t = i4 / I;
  const int i = static_cast<int>(i4 - t * I);
  const float4 g = *reinterpret_cast<const float4*>(gu + t * 2 * I + i);
  const float4 u = *reinterpret_cast<const float4*>(gu + t * 2 * I + I + i);
  const float y0 = (g.x / (1.0f + expf(-g.x))) * u.x, y1 = (g.y / (1.0f + expf(-g.y))) * u.y;
  const float y2 = (g.z / (1.0f + expf(-g.z))) * u.z, y3 = (g.w / (1.0f + expf(-g.w))) * u.w;
  *reinterpret_cast<uint2*>(out + i4) = make_uint2(pack_bf16x2(y0, y1), pack_bf16x2(y2, y3));
}

// -------------------------------------------------------------------- casts ----
// VEC: 16-byte fp32 side and 8-byte bf16 side (4 elements per access); otherwise element
// accesses (operands at their natural alignment only).
template <bool VEC>
__global__ __launch_bounds__(256) void f32_to_bf16_kernel(const float* __restrict__ in,
                                                          uint16_t* __restrict__ out, long n) {
  const long i = (static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (VEC && i + 3 < n) {
    const float4 v = *reinterpret_cast<const float4*>(in + i);
    *reinterpret_cast<uint2*>(out + i) = make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
  } else {
    for (long k = i; k < n && k < i + 4; ++k) out[k] = f32_to_bf16(in[k]);
  }
}

template <bool VEC>
__global__ __launch_bounds__(256) void bf16_to_f32_kernel(const uint16_t* __restrict__ in,
                                                          float* __restrict__ out, long n) {
  const long i = (static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (VEC && i + 3 < n) {
    const uint2 v = *reinterpret_cast<const uint2*>(in + i);
    *reinterpret_cast<float4*>(out + i) =
        make_float4(bf16_lo(v.x), bf16_hi(v.x), bf16_lo(v.y), bf16_hi(v.y));
  } else {
    for (long k = i; k < n && k < i + 4; ++k) out[k] = bf16_to_f32(in[k]);
  }
}

// ----------------------------------------------------------- ArgmaxBanned ----
__global__ __launch_bounds__(256) void argmax_banned_kernel(const float* __restrict__ x, int n,
                                                            int ban0, int ban1,
                                                            int* __restrict__ out_idx) {
  __shared__ float sval[256];
  __shared__ int sidx[256];
  float best = -1e30f;
  int bi = 0;
  for (int i = threadIdx.x; i < n; i += 256) {
    if (i == ban0 || i == ban1) continue;
    const float v = x[i];
    if (v > best) {
      best = v;
      bi = i;
    }
  }
  sval[threadIdx.x] = best;
  sidx[threadIdx.x] = bi;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s && sval[threadIdx.x + s] > sval[threadIdx.x]) {
      sval[threadIdx.x] = sval[threadIdx.x + s];
      sidx[threadIdx.x] = sidx[threadIdx.x + s];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) *out_idx = sidx[0];
}

// Two-stage form for long rows (the vocabulary).  The single-block kernel above fixes the
// tie rule: thread t keeps the first maximum of its strided subsequence i = t (mod 256),
// then the tree above picks among the 256 thread candidates.  Stage 1 splits every thread's
// subsequence into row ranges (row r = elements [256 r, 256 r + 256)), one range per
// workgroup, and keeps each range's first maximum per thread; stage 2 folds the ranges in
// order per thread (strict >, so the first maximum survives) and runs the same tree.  The
// result is the single-block kernel's on every input.
constexpr int kArgmaxRows = 8;  // rows of 256 elements per stage-1 workgroup

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ x, int n,
                                                             int ban0, int ban1,
                                                             float* __restrict__ pval,
                                                             int* __restrict__ pidx) {
  const int t = threadIdx.x;
  float best = -1e30f;
  int bi = 0;
  const int r0 = blockIdx.x * kArgmaxRows;
#pragma unroll
  for (int r = 0; r < kArgmaxRows; ++r) {
    const int i = (r0 + r) * 256 + t;
    if (i < n && i != ban0 && i != ban1) {
      const float v = x[i];
      if (v > best) {
        best = v;
        bi = i;
      }
    }
  }
  pval[blockIdx.x * 256 + t] = best;
  pidx[blockIdx.x * 256 + t] = bi;
}

__global__ __launch_bounds__(256) void argmax_finish_kernel(const float* __restrict__ pval,
                                                            const int* __restrict__ pidx,
                                                            int parts, int* __restrict__ out_idx) {
  __shared__ float sval[256];
  __shared__ int sidx[256];
  float best = -1e30f;
  int bi = 0;
  // 16 ranges' candidates are loaded together, then folded in range order
  for (int g0 = 0; g0 < parts; g0 += 16) {
    float v[16];
    int ix[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int g = min(g0 + u, parts - 1);
      v[u] = pval[g * 256 + threadIdx.x];
      ix[u] = pidx[g * 256 + threadIdx.x];
    }
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (g0 + u < parts && v[u] > best) {
        best = v[u];
        bi = ix[u];
      }
  }
  sval[threadIdx.x] = best;
  sidx[threadIdx.x] = bi;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s && sval[threadIdx.x + s] > sval[threadIdx.x]) {
      sval[threadIdx.x] = sval[threadIdx.x + s];
      sidx[threadIdx.x] = sidx[threadIdx.x + s];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) *out_idx = sidx[0];
}

// ----------------------------------------------------------------- KV write ----
// One lane per 4 elements of one (t, h) row; both K and V rows are converted in the
// same lane.  Rows at or past the capacity (or with an out-of-range page) are dropped.
__global__ __launch_bounds__(256) void kv_write_kernel(const float* __restrict__ k,
                                                       const float* __restrict__ v,
                                                       uint16_t* __restrict__ kc,
                                                       uint16_t* __restrict__ vc, int Tq,
                                                       int Hkv, int Dh,
                                                       const int* __restrict__ pos0p,
                                                       int capacity, const int* page_table,
                                                       int max_pages, int page_shift, int n_pages,
                                                       int B) {
  const int q4 = Dh / 4;
  const long idx = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  const long total = static_cast<long>(B) * Tq * Hkv * q4;
  if (idx >= total) return;
  const int d = static_cast<int>(idx % q4) * 4;
  const long row = idx / q4;  // ((b*Tq + t)*Hkv + h)
  const int h = static_cast<int>(row % Hkv);
  const long bt = row / Hkv;
  const int t = static_cast<int>(bt % Tq);
  const int b = static_cast<int>(bt / Tq);
  const int p = pos0p[b] + t;
  long dst_row;
  if (page_table) {
    const int pi = p >> page_shift;
    if (p < 0 || pi >= max_pages) return;
    const int page = page_table[static_cast<long>(b) * max_pages + pi];
    if (page < 0 || page >= n_pages) return;
    dst_row = (static_cast<long>(page) << page_shift) | (p & ((1 << page_shift) - 1));
  } else {
    if (p < 0 || p >= capacity) return;
    dst_row = p;
  }
  const long src = row * Dh + d;
  const long dst = (dst_row * Hkv + h) * Dh + d;
  const float4 kv = *reinterpret_cast<const float4*>(k + src);
  const float4 vv = *reinterpret_cast<const float4*>(v + src);
  *reinterpret_cast<uint2*>(kc + dst) = make_uint2(pack_bf16x2(kv.x, kv.y), pack_bf16x2(kv.z, kv.w));
  *reinterpret_cast<uint2*>(vc + dst) = make_uint2(pack_bf16x2(vv.x, vv.y), pack_bf16x2(vv.z, vv.w));
}

// -------------------------------------------- fused QK-norm + RoPE + KV write ----
// One wave64 per (token, head) row of Dh = 128: lane j owns the rotate-half pair
// (j, j + 64).  q rows: RMSNorm(q_norm) then RoPE, written back in place.  k rows:
// RMSNorm(k_norm), RoPE, written back in place and as bf16 into the cache row of the
// token's position, together with the bf16 of the matching v row.  Same arithmetic as
// RmsNorm + RopeHalf + WriteKvCache run back to back (src/model/asr_text_decoder.cu:408-413,
// 530-536); only the order of the sum of squares differs.
struct QkvArgs {
  float* q;
  float* k;
  const float* v;
  long q_stride;   // elements between consecutive tokens of q
  long kv_stride;  // ... of k and v
  const float* q_norm;
  const float* k_norm;
  float eps;
  const int* positions;  // [n_tokens]
  float theta;
  int n_tokens, tokens_per_stream, Hq, Hkv;
  uint16_t* kpool;
  uint16_t* vpool;
  const int* page_table;  // nullptr => contiguous cache of `capacity` rows
  int max_pages, page_shift, capacity;  // paged: capacity = number of pages in the pool
  const float* rope;  // optional (cos, sin) table of rope_table_kernel, instead of rope_cs
  int rope_rows;      // positions the table holds
};

// (cos, sin) of RoPE pair `lane` at position pos: the table row when it holds pos (the same
// values rope_cs forms), else formed here.
__device__ __forceinline__ void qkv_rope_cs(const QkvArgs& a, int pos, int lane, float* c,
                                            float* s) {
  if (a.rope && pos >= 0 && pos < a.rope_rows) {
    const float* cs = a.rope + (static_cast<long>(pos) * 64 + lane) * 2;
    *c = cs[0];
    *s = cs[1];
  } else {
    rope_cs(static_cast<float>(pos), a.theta, lane, 128, c, s);
  }
}

// Row hh of token t (q heads first, then k heads): RmsNorm of the loaded halves x0 = x[lane],
// x1 = x[lane + 64], RoPE with this lane's (c, s), store; a k row also writes its k and v
// rows into the cache row of the token's position.
__device__ __forceinline__ void qkv_row(const QkvArgs& a, int t, int hh, int lane, float c,
                                        float s, float x0, float x1) {
#pragma clang fp contract(off)
  constexpr int Dh = 128, half = 64;
  const bool is_q = hh < a.Hq;
  const int h = is_q ? hh : hh - a.Hq;
  float* x = is_q ? a.q + t * a.q_stride + static_cast<long>(h) * Dh
                  : a.k + t * a.kv_stride + static_cast<long>(h) * Dh;
  const float* w = is_q ? a.q_norm : a.k_norm;
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float inv = rsqrt_via_f64(ss / Dh + a.eps);
  const float n0 = x0 * inv * w[lane], n1 = x1 * inv * w[lane + half];
  const float r0 = n0 * c - n1 * s;
  const float r1 = n1 * c + n0 * s;
  x[lane] = r0;
  x[lane + half] = r1;
  if (is_q) return;
  // cache row of this token's position
  const int pos = a.positions[t];
  long crow;
  if (a.page_table) {
    const int b = t / a.tokens_per_stream;
    const int pi = pos >> a.page_shift;
    if (pos < 0 || pi >= a.max_pages) return;
    const int page = a.page_table[static_cast<long>(b) * a.max_pages + pi];
    if (page < 0 || page >= a.capacity) return;
    crow = (static_cast<long>(page) << a.page_shift) | (pos & ((1 << a.page_shift) - 1));
  } else {
    if (pos < 0 || pos >= a.capacity) return;
    crow = pos;
  }
  const long dst = (crow * a.Hkv + h) * Dh;
  const float* vr = a.v + t * a.kv_stride + static_cast<long>(h) * Dh;
  a.kpool[dst + lane] = f32_to_bf16(r0);
  a.kpool[dst + lane + half] = f32_to_bf16(r1);
  a.vpool[dst + lane] = f32_to_bf16(vr[lane]);
  a.vpool[dst + lane + half] = f32_to_bf16(vr[lane + half]);
}

__device__ __forceinline__ const float* qkv_row_ptr(const QkvArgs& a, int t, int hh) {
  return hh < a.Hq ? a.q + t * a.q_stride + static_cast<long>(hh) * 128
                   : a.k + t * a.kv_stride + static_cast<long>(hh - a.Hq) * 128;
}

// Decode-sized calls: one wave per (token, head) row, 4 rows per workgroup.
__global__ __launch_bounds__(256) void qk_norm_rope_kv_kernel(QkvArgs a) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int per_token = a.Hq + a.Hkv;
  if (row >= a.n_tokens * per_token) return;
  const int t = row / per_token;
  const int hh = row % per_token;
  const float* x = qkv_row_ptr(a, t, hh);
  const float x0 = x[lane], x1 = x[lane + 64];
  float c, s;
  qkv_rope_cs(a, a.positions[t], lane, &c, &s);
  qkv_row(a, t, hh, lane, c, s, x0, x1);
}

// Prompts: one workgroup per token; wave w takes rows w, w+4, ... of the token, forms this
// lane's RoPE (cos, sin) once for all of them (the fp64 pow/sincos depend only on the
// position and the lane) and loads kQkvBatch rows before processing them.  Same per-row
// arithmetic as qk_norm_rope_kv_kernel.
constexpr int kQkvBatch = 8;
__global__ __launch_bounds__(256) void qk_norm_rope_kv_token_kernel(QkvArgs a) {
  const int t = blockIdx.x;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int per_token = a.Hq + a.Hkv;
  float c, s;
  qkv_rope_cs(a, a.positions[t], lane, &c, &s);
  for (int hb = wave; hb < per_token; hb += 4 * kQkvBatch) {
    float x0[kQkvBatch], x1[kQkvBatch];
#pragma unroll
    for (int i = 0; i < kQkvBatch; ++i) {
      const int hh = hb + 4 * i;
      if (hh < per_token) {
        const float* x = qkv_row_ptr(a, t, hh);
        x0[i] = x[lane];
        x1[i] = x[lane + 64];
      }
    }
#pragma unroll
    for (int i = 0; i < kQkvBatch; ++i) {
      const int hh = hb + 4 * i;
      if (hh < per_token) qkv_row(a, t, hh, lane, c, s, x0[i], x1[i]);
    }
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace orator_hip

namespace orator_hip {

int launch_rms_norm_bf16(const float* x, const float* w, uint16_t* out, int rows, int dim,
                         float eps, hipStream_t s) {
  if (rows <= 0 || dim <= 0) return ORATOR_OK;
  const dim3 grid(blocks_for(rows, 4));
  const bool vec =
      dim % 4 == 0 && aligned16(x) && aligned16(w) && (reinterpret_cast<uintptr_t>(out) & 7u) == 0;
  if (vec && dim <= 512)
    hipLaunchKernelGGL((rms_norm_kernel<true, uint16_t, 2>), grid, dim3(256), 0, s, x, w, out,
                       rows, dim, eps);
  else if (vec && dim <= 1024)
    hipLaunchKernelGGL((rms_norm_kernel<true, uint16_t, 4>), grid, dim3(256), 0, s, x, w, out,
                       rows, dim, eps);
  else if (vec && dim <= 2048)
    hipLaunchKernelGGL((rms_norm_kernel<true, uint16_t, 8>), grid, dim3(256), 0, s, x, w, out,
                       rows, dim, eps);
  else if (vec)
    hipLaunchKernelGGL((rms_norm_kernel<true, uint16_t>), grid, dim3(256), 0, s, x, w, out, rows,
                       dim, eps);
  else
    hipLaunchKernelGGL((rms_norm_kernel<false, uint16_t>), grid, dim3(256), 0, s, x, w, out, rows,
                       dim, eps);
  return check_launch("rms_norm_bf16");
}

int launch_qk_norm_rope_kv(float* q, float* k, const float* v, long q_stride, long kv_stride,
                           const float* q_norm, const float* k_norm, float eps,
                           const int* positions, float theta, const float* rope,
                           int rope_rows, int n_tokens, int tokens_per_stream, int Hq, int Hkv,
                           int Dh, uint16_t* kpool, uint16_t* vpool, const int* page_table,
                           int max_pages, int page_size, int capacity, hipStream_t stream) {
  if (n_tokens <= 0 || Hq <= 0 || Hkv <= 0 || Dh <= 0) return ORATOR_OK;
  if (!q || !k || !v || !q_norm || !k_norm || !positions || !kpool || !vpool)
    return fail(ORATOR_ERR_INVALID, "qk_norm_rope_kv_write: null pointer");
  if (Dh != 128) return fail(ORATOR_ERR_UNSUPPORTED, "qk_norm_rope_kv_write: Dh must be 128");
  if (capacity <= 0) return fail(ORATOR_ERR_INVALID, "qk_norm_rope_kv_write: capacity must be > 0");
  QkvArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.q_stride = q_stride;
  a.kv_stride = kv_stride;
  a.q_norm = q_norm;
  a.k_norm = k_norm;
  a.eps = eps;
  a.positions = positions;
  a.theta = theta;
  a.n_tokens = n_tokens;
  a.tokens_per_stream = tokens_per_stream > 0 ? tokens_per_stream : n_tokens;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.kpool = kpool;
  a.vpool = vpool;
  a.page_table = page_table;
  a.capacity = capacity;
  a.rope = rope;
  a.rope_rows = rope ? rope_rows : 0;
  if (page_table) {
    a.page_shift = ilog2_exact(page_size);
    if (a.page_shift < 0 || max_pages <= 0)
      return fail(ORATOR_ERR_INVALID, "qk_norm_rope_kv_write: page_size must be a power of two");
    a.max_pages = max_pages;
  }
  // Prompts: a workgroup per token (RoPE angles formed once per token and wave); a few
  // tokens (decode): a wave per row, which spreads the rows over more of the chip.
  if (n_tokens >= 64) {
    hipLaunchKernelGGL(qk_norm_rope_kv_token_kernel, dim3(n_tokens), dim3(256), 0,
                       stream, a);
  } else {
    const long rows = static_cast<long>(n_tokens) * (Hq + Hkv);
    hipLaunchKernelGGL(qk_norm_rope_kv_kernel, dim3(blocks_for(rows, 4)), dim3(256), 0,
                       stream, a);
  }
  return check_launch("qk_norm_rope_kv_write");
}


int launch_rope_table(float* out, int n_pos, float theta, hipStream_t s) {
  if (n_pos <= 0) return ORATOR_OK;
  const long n = static_cast<long>(n_pos) * 64;
  hipLaunchKernelGGL(rope_table_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256),
                     0, s, out, n_pos, theta);
  return check_launch("rope_table");
}

int launch_swiglu_bf16(const float* gu, uint16_t* out, int T, int I, hipStream_t s) {
  if (T <= 0 || I <= 0) return ORATOR_OK;
  if (I % 4 || !aligned16(gu) || (reinterpret_cast<uintptr_t>(out) & 7u))
    return fail(ORATOR_ERR_UNSUPPORTED, "swiglu_bf16: I % 4 and 16/8-byte alignment");
  const long threads = static_cast<long>(T) * I / 4;
  hipLaunchKernelGGL(swiglu_bf16_kernel, dim3(static_cast<unsigned>((threads + 255) / 256)),
                     dim3(256), 0, s, gu, out, T, I);
  return check_launch("swiglu_bf16");
}

size_t argmax_scratch_bytes(int n) {
  const int rows = (n + 255) / 256;
  const int parts = (rows + kArgmaxRows - 1) / kArgmaxRows;
  return parts > 1 ? static_cast<size_t>(parts) * 256 * (sizeof(float) + sizeof(int)) : 0;
}

int launch_argmax_banned(const float* logits, int n, int ban0, int ban1, int* out_idx,
                         void* scratch, hipStream_t s) {
  const int rows = (n + 255) / 256;
  const int parts = (rows + kArgmaxRows - 1) / kArgmaxRows;
  if (parts <= 1) {
    hipLaunchKernelGGL(argmax_banned_kernel, dim3(1), dim3(256), 0, s, logits, n, ban0, ban1,
                       out_idx);
    return check_launch("argmax_banned");
  }
  if (!scratch) return fail(ORATOR_ERR_INVALID, "argmax_banned: scratch needed");
  float* pval = static_cast<float*>(scratch);
  int* pidx = reinterpret_cast<int*>(pval + static_cast<size_t>(parts) * 256);
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(parts), dim3(256), 0, s, logits, n, ban0, ban1,
                     pval, pidx);
  hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(256), 0, s, pval, pidx, parts, out_idx);
  return check_launch("argmax_banned");
}

}  // namespace orator_hip

using namespace orator_hip;

extern "C" {

int orator_rms_norm(const float* x, const float* weight, float* out, int rows, int dim, float eps,
                    void* stream) {
  if (rows <= 0 || dim <= 0) return ORATOR_OK;
  if (!x || !weight || !out) return fail(ORATOR_ERR_INVALID, "rms_norm: null pointer");
  const bool vec = (dim % 4 == 0) && aligned16(x) && aligned16(weight) && aligned16(out);
  const dim3 grid(blocks_for(rows, 4));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (vec && dim <= 512)
    hipLaunchKernelGGL((rms_norm_kernel<true, float, 2>), grid, dim3(256), 0, s, x, weight, out,
                       rows, dim, eps);
  else if (vec && dim <= 1024)
    hipLaunchKernelGGL((rms_norm_kernel<true, float, 4>), grid, dim3(256), 0, s, x, weight, out,
                       rows, dim, eps);
  else if (vec && dim <= 2048)
    hipLaunchKernelGGL((rms_norm_kernel<true, float, 8>), grid, dim3(256), 0, s, x, weight, out,
                       rows, dim, eps);
  else if (vec)
    hipLaunchKernelGGL(rms_norm_kernel<true>, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                       x, weight, out, rows, dim, eps);
  else
    hipLaunchKernelGGL(rms_norm_kernel<false>, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                       x, weight, out, rows, dim, eps);
  return check_launch("rms_norm");
}

int orator_rope_interleaved(float* x, const int* positions, int n_tokens, int n_heads, int head_dim,
                            float theta_base) {
  if (n_tokens <= 0 || n_heads <= 0 || head_dim <= 0) return ORATOR_OK;
  if (!x || !positions) return fail(ORATOR_ERR_INVALID, "rope_interleaved: null pointer");
  if (head_dim % 2) return fail(ORATOR_ERR_UNSUPPORTED, "rope_interleaved: head_dim must be even");
  const long total = static_cast<long>(n_tokens) * n_heads * (head_dim / 2);
  hipLaunchKernelGGL(rope_kernel<false>, dim3(blocks_for(total)), dim3(kBlock), 0, nullptr, x,
                     positions, n_tokens, n_heads, head_dim, theta_base);
  return check_launch("rope_interleaved");
}

int orator_rope_half(float* x, const int* positions, int n_tokens, int n_heads, int head_dim,
                     float theta_base, void* stream) {
  if (n_tokens <= 0 || n_heads <= 0 || head_dim <= 0) return ORATOR_OK;
  if (!x || !positions) return fail(ORATOR_ERR_INVALID, "rope_half: null pointer");
  if (head_dim % 2) return fail(ORATOR_ERR_UNSUPPORTED, "rope_half: head_dim must be even");
  const long total = static_cast<long>(n_tokens) * n_heads * (head_dim / 2);
  hipLaunchKernelGGL(rope_kernel<true>, dim3(blocks_for(total)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), x, positions, n_tokens, n_heads, head_dim,
                     theta_base);
  return check_launch("rope_half");
}

int orator_swiglu(const float* gate, const float* up, float* out, int n, void* stream) {
  if (n <= 0) return ORATOR_OK;
  if (!gate || !up || !out) return fail(ORATOR_ERR_INVALID, "swiglu: null pointer");
  hipLaunchKernelGGL(swiglu_kernel, dim3(blocks_for(n)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), gate, up, out, n);
  return check_launch("swiglu");
}

int orator_f32_to_bf16(const float* in, uint16_t* out, long n, void* stream) {
  if (n <= 0) return ORATOR_OK;
  if (!in || !out) return fail(ORATOR_ERR_INVALID, "f32_to_bf16: null pointer");
  if ((reinterpret_cast<uintptr_t>(in) & 3u) || (reinterpret_cast<uintptr_t>(out) & 1u))
    return fail(ORATOR_ERR_INVALID, "f32_to_bf16: in must be 4-byte and out 2-byte aligned");
  const bool vec = aligned16(in) && (reinterpret_cast<uintptr_t>(out) & 7u) == 0;
  if (vec)
    hipLaunchKernelGGL(f32_to_bf16_kernel<true>, dim3(blocks_for((n + 3) / 4)), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), in, out, n);
  else
    hipLaunchKernelGGL(f32_to_bf16_kernel<false>, dim3(blocks_for((n + 3) / 4)), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), in, out, n);
  return check_launch("f32_to_bf16");
}

int orator_bf16_to_f32(const uint16_t* in, float* out, long n, void* stream) {
  if (n <= 0) return ORATOR_OK;
  if (!in || !out) return fail(ORATOR_ERR_INVALID, "bf16_to_f32: null pointer");
  if ((reinterpret_cast<uintptr_t>(in) & 1u) || (reinterpret_cast<uintptr_t>(out) & 3u))
    return fail(ORATOR_ERR_INVALID, "bf16_to_f32: in must be 2-byte and out 4-byte aligned");
  const bool vec = (reinterpret_cast<uintptr_t>(in) & 7u) == 0 && aligned16(out);
  if (vec)
    hipLaunchKernelGGL(bf16_to_f32_kernel<true>, dim3(blocks_for((n + 3) / 4)), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), in, out, n);
  else
    hipLaunchKernelGGL(bf16_to_f32_kernel<false>, dim3(blocks_for((n + 3) / 4)), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), in, out, n);
  return check_launch("bf16_to_f32");
}

int orator_argmax_banned(const float* logits, int n, int ban0, int ban1, int* out_idx,
                         void* stream) {
  if (n <= 0) return ORATOR_OK;
  if (!logits || !out_idx) return fail(ORATOR_ERR_INVALID, "argmax_banned: null pointer");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  void* scratch = nullptr;
  if (argmax_scratch_bytes(n)) {
    scratch = workspace(s, argmax_scratch_bytes(n));
    if (!scratch) return ORATOR_ERR_HIP;
  }
  return launch_argmax_banned(logits, n, ban0, ban1, out_idx, scratch, s);
}

int orator_kv_write(const float* k, const float* v, uint16_t* kc, uint16_t* vc, int Tq, int Hkv,
                    int Dh, const int* d_pos0, int capacity, void* stream) {
  if (Tq <= 0 || Hkv <= 0 || Dh <= 0) return ORATOR_OK;
  if (!k || !v || !kc || !vc || !d_pos0) return fail(ORATOR_ERR_INVALID, "kv_write: null pointer");
  if (Dh % 4) return fail(ORATOR_ERR_UNSUPPORTED, "kv_write: Dh must be a multiple of 4");
  if (!aligned16(k) || !aligned16(v) || (reinterpret_cast<uintptr_t>(kc) & 7u) ||
      (reinterpret_cast<uintptr_t>(vc) & 7u))
    return fail(ORATOR_ERR_INVALID, "kv_write: k/v must be 16-byte and caches 8-byte aligned");
  const long total = static_cast<long>(Tq) * Hkv * (Dh / 4);
  hipLaunchKernelGGL(kv_write_kernel, dim3(blocks_for(total)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), k, v, kc, vc, Tq, Hkv, Dh, d_pos0, capacity,
                     nullptr, 0, 0, 0, 1);
  return check_launch("kv_write");
}

int orator_kv_write_paged(const float* k, const float* v, uint16_t* kpool, uint16_t* vpool,
                          const int* page_table, int max_pages, int page_size, int n_pages, int B,
                          int Tq, int Hkv, int Dh, const int* d_pos0, void* stream) {
  if (B <= 0 || Tq <= 0 || Hkv <= 0 || Dh <= 0) return ORATOR_OK;
  if (!k || !v || !kpool || !vpool || !page_table || !d_pos0)
    return fail(ORATOR_ERR_INVALID, "kv_write_paged: null pointer");
  if (Dh % 4) return fail(ORATOR_ERR_UNSUPPORTED, "kv_write_paged: Dh must be a multiple of 4");
  if (!aligned16(k) || !aligned16(v) || (reinterpret_cast<uintptr_t>(kpool) & 7u) ||
      (reinterpret_cast<uintptr_t>(vpool) & 7u))
    return fail(ORATOR_ERR_INVALID, "kv_write_paged: k/v must be 16-byte and pools 8-byte aligned");
  const int shift = ilog2_exact(page_size);
  if (shift < 0 || max_pages <= 0 || n_pages <= 0)
    return fail(ORATOR_ERR_INVALID, "kv_write_paged: page_size must be a power of two");
  const long total = static_cast<long>(B) * Tq * Hkv * (Dh / 4);
  hipLaunchKernelGGL(kv_write_kernel, dim3(blocks_for(total)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), k, v, kpool, vpool, Tq, Hkv, Dh, d_pos0, 0,
                     page_table, max_pages, shift, n_pages, B);
  return check_launch("kv_write_paged");
}

int orator_rope_table(float* out, int n_pos, float theta, void* stream) {
  if (n_pos > 0 && !out) return orator_hip::fail(ORATOR_ERR_INVALID, "rope_table: null pointer");
  return orator_hip::launch_rope_table(out, n_pos, theta, static_cast<hipStream_t>(stream));
}

int orator_qk_norm_rope_kv_write_table(float* q, float* k, const float* v, long q_stride,
                                       long kv_stride, const float* q_norm, const float* k_norm,
                                       float eps, const int* positions, float theta,
                                       const float* rope, int rope_rows, int n_tokens,
                                       int tokens_per_stream, int Hq, int Hkv, int Dh,
                                       uint16_t* kpool, uint16_t* vpool, const int* page_table,
                                       int max_pages, int page_size, int capacity, void* stream) {
  if (n_tokens > 0 && (!rope || rope_rows <= 0))
    return orator_hip::fail(ORATOR_ERR_INVALID, "qk_norm_rope_kv_write_table: no RoPE table");
  return orator_hip::launch_qk_norm_rope_kv(q, k, v, q_stride, kv_stride, q_norm, k_norm, eps,
                                            positions, theta, rope, rope_rows, n_tokens,
                                            tokens_per_stream, Hq, Hkv, Dh, kpool, vpool,
                                            page_table, max_pages, page_size, capacity,
                                            static_cast<hipStream_t>(stream));
}

int orator_qk_norm_rope_kv_write(float* q, float* k, const float* v, long q_stride, long kv_stride,
                                 const float* q_norm, const float* k_norm, float eps,
                                 const int* positions, float theta, int n_tokens,
                                 int tokens_per_stream, int Hq, int Hkv, int Dh, uint16_t* kpool,
                                 uint16_t* vpool, const int* page_table, int max_pages,
                                 int page_size, int capacity, void* stream) {
  return orator_hip::launch_qk_norm_rope_kv(q, k, v, q_stride, kv_stride, q_norm, k_norm, eps,
                                            positions, theta, nullptr, 0, n_tokens,
                                            tokens_per_stream, Hq, Hkv, Dh, kpool, vpool,
                                            page_table, max_pages, page_size, capacity,
                                            static_cast<hipStream_t>(stream));
}

}  // extern "C"
