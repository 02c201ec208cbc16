// Split-K (flash-decoding) GQA decode attention over a bf16 KV cache, gfx950.
//
// Replaces GqaDecodeAttnKernel (src/model/asr_text_decoder.cu:149-213): one fp32 query
// per q-head attends S = pos+1 cached keys.  Semantics kept: fp32 q, bf16 K/V widened
// exactly, fp32 accumulation, scores scaled after the dot, softmax normalised by
// multiplying with 1/sum.  The exponent is taken base 2 on scores pre-multiplied by
// log2(e) (same value up to fp32 rounding).
//
// Design (memory-bound, ~2 flop/byte):
//  * one workgroup = (split of SPLIT keys, kv head, stream); 4 wave64s, each owning a
//    contiguous quarter of the split.  Both (all G) q heads of the GQA group consume
//    every K/V row the workgroup loads, so K/V are read from HBM exactly once.
//  * QK phase, "quad" layout: 4 lanes per key, each lane 4 x 16-byte loads covering 32
//    of the 128 dims; a quad's 4 loads of one instruction are one contiguous 64-byte
//    segment of the row.  The 4-lane dot reduction is two DPP quad_perm adds.
//  * scores stay in registers; workgroup max and sum go through LDS; probabilities are
//    written to LDS for the PV phase.
//  * PV phase, "row" layout: Dh/8 lanes per key, one 16-byte load each, so every load
//    instruction reads whole contiguous K/V rows; per-lane accumulators hold 8 dims x G
//    heads, reduced across rows with lane shuffles and across waves through LDS.
//  * split combine: each workgroup stores (acc, max, sum); the last one to finish for
//    its (stream, kv head) -- found with a device-scope counter that it resets -- merges
//    the splits in the same launch.
#include "common.hpp"
#include "internal.hpp"

namespace orator_hip {
namespace {

struct DecodeArgs {
  const float* q;
  const uint16_t* kpool;
  const uint16_t* vpool;
  const int* page_table;
  const int* pos;
  float* out;
  float* part_o;       // [B*Hq][max_splits][DH]
  float* part_ml;      // [B*Hq][max_splits][2]
  unsigned* counters;  // [B*Hkv], zero between launches
  long stream_stride;
  int max_pages;
  int page_shift;
  int Hkv;
  int max_splits;
  int capacity;
  float scale_log2e;
};

template <int DH, int G, int SPLIT>
__global__ __launch_bounds__(256) void gqa_decode_kernel(DecodeArgs a) {
  constexpr int NW = 4;
  constexpr int TPW = SPLIT / NW;   // keys per wave
  constexpr int C = DH / 32;        // 32-dim chunks in the quad layout
  constexpr int NI = TPW / 16;      // QK iterations, 16 keys each
  constexpr int LPT = DH / 8;       // lanes per key in the row layout
  constexpr int TPI = kWave / LPT;  // keys per PV iteration
  constexpr int NI2 = TPW / TPI;
  static_assert(TPW % 16 == 0 && TPW % TPI == 0, "split must cover whole iterations");

  __shared__ float p_lds[G][SPLIT];
  __shared__ float red_o[NW][G][DH];
  __shared__ float red_ml[NW][G];
  __shared__ int s_last;

  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  int S = a.pos[b] + 1;
  if (S > a.capacity) S = a.capacity;
  if (S <= 0) {  // no keys: the reference's 1/sum guard yields zeros
    if (split == 0)
      for (int idx = threadIdx.x; idx < G * DH; idx += 256)
        a.out[(static_cast<long>(b) * a.Hkv * G + kvh * G) * DH + idx] = 0.0f;
    return;
  }
  const int t0 = split * SPLIT;
  if (t0 >= S) return;
  const int n_splits = (S + SPLIT - 1) / SPLIT;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int Hq = a.Hkv * G;
  const KvMap map{a.page_table ? a.page_table + static_cast<long>(b) * a.max_pages : nullptr,
                  a.page_shift, a.page_table ? 0 : static_cast<long>(b) * a.stream_stride};

  // ---- q of the G heads, quad layout: lane owns dims 32c + 8*k4 + e ----
  const int k4 = lane & 3;
  float qr[G][C][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float* qh = a.q + (static_cast<long>(b) * Hq + kvh * G + g) * DH + 8 * k4;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const float4 x0 = *reinterpret_cast<const float4*>(qh + 32 * c);
      const float4 x1 = *reinterpret_cast<const float4*>(qh + 32 * c + 4);
      qr[g][c][0] = x0.x; qr[g][c][1] = x0.y; qr[g][c][2] = x0.z; qr[g][c][3] = x0.w;
      qr[g][c][4] = x1.x; qr[g][c][5] = x1.y; qr[g][c][6] = x1.z; qr[g][c][7] = x1.w;
    }
  }

  // ---- phase 1: scores (base-2 scaled) ----
  const int wbase = wave * TPW;
  uint4 kreg[NI][C];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int j = t0 + wbase + 16 * i + (lane >> 2);
    if (j < S) {
      const uint16_t* row = a.kpool + map.row_offset(j, a.Hkv, kvh, DH) + 8 * k4;
#pragma unroll
      for (int c = 0; c < C; ++c) kreg[i][c] = *reinterpret_cast<const uint4*>(row + 32 * c);
    } else {
#pragma unroll
      for (int c = 0; c < C; ++c) kreg[i][c] = make_uint4(0, 0, 0, 0);
    }
  }
  float s[NI][G];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    float d[G];
#pragma unroll
    for (int g = 0; g < G; ++g) d[g] = 0.0f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const uint32_t w[4] = {kreg[i][c].x, kreg[i][c].y, kreg[i][c].z, kreg[i][c].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float klo = bf16_lo(w[e]);
        const float khi = bf16_hi(w[e]);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          d[g] = fmaf(qr[g][c][2 * e], klo, d[g]);
          d[g] = fmaf(qr[g][c][2 * e + 1], khi, d[g]);
        }
      }
    }
    const bool valid = t0 + wbase + 16 * i + (lane >> 2) < S;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float dot = quad_sum(d[g]);
      s[i][g] = valid ? dot * a.scale_log2e : -INFINITY;
    }
  }

  // ---- workgroup max ----
  float M[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float m = s[0][g];
#pragma unroll
    for (int i = 1; i < NI; ++i) m = fmaxf(m, s[i][g]);
    m = wave_max(m);
    if (lane == 0) red_ml[wave][g] = m;
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float m = red_ml[0][g];
#pragma unroll
    for (int w = 1; w < NW; ++w) m = fmaxf(m, red_ml[w][g]);
    M[g] = m;
  }
  __syncthreads();

  // ---- probabilities -> LDS, workgroup sum ----
  float lsum[G];
#pragma unroll
  for (int g = 0; g < G; ++g) lsum[g] = 0.0f;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float p = fast_exp2(s[i][g] - M[g]);
      if (k4 == 0) {
        p_lds[g][wbase + 16 * i + (lane >> 2)] = p;
        lsum[g] += p;
      }
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float l = wave_sum(lsum[g]);
    if (lane == 0) red_ml[wave][g] = l;
  }
  __syncthreads();
  float L[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float l = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) l += red_ml[w][g];
    L[g] = l;
  }

  // ---- phase 2: PV, row layout ----
  const int dg = lane % LPT;
  const int r = lane / LPT;
  uint4 vreg[NI2];
#pragma unroll
  for (int i = 0; i < NI2; ++i) {
    const int j = t0 + wbase + TPI * i + r;
    vreg[i] = j < S ? *reinterpret_cast<const uint4*>(a.vpool + map.row_offset(j, a.Hkv, kvh, DH) +
                                                     8 * dg)
                    : make_uint4(0, 0, 0, 0);
  }
  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.0f;
#pragma unroll
  for (int i = 0; i < NI2; ++i) {
    const int lt = wbase + TPI * i + r;
    const uint32_t w[4] = {vreg[i].x, vreg[i].y, vreg[i].z, vreg[i].w};
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float p = p_lds[g][lt];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[g][2 * e] = fmaf(p, bf16_lo(w[e]), acc[g][2 * e]);
        acc[g][2 * e + 1] = fmaf(p, bf16_hi(w[e]), acc[g][2 * e + 1]);
      }
    }
  }
#pragma unroll
  for (int off = LPT; off < kWave; off <<= 1)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] += __shfl_xor(acc[g][e], off);
  if (r == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float4* dst = reinterpret_cast<float4*>(&red_o[wave][g][8 * dg]);
      dst[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
      dst[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
    }
  }
  __syncthreads();

  for (int idx = tid; idx < G * DH; idx += 256) {
    const int g = idx / DH;
    const int d = idx % DH;
    float o = red_o[0][g][d];
#pragma unroll
    for (int w = 1; w < NW; ++w) o += red_o[w][g][d];
    const long bh = static_cast<long>(b) * Hq + kvh * G + g;
    if (n_splits == 1) {
      a.out[bh * DH + d] = o * (1.0f / L[g]);
    } else {
      const long ps = bh * a.max_splits + split;
      a.part_o[ps * DH + d] = o;
      if (d == 0) {
        a.part_ml[ps * 2] = M[g];
        a.part_ml[ps * 2 + 1] = L[g];
      }
    }
  }
  if (n_splits == 1) return;

  // ---- split combine by the last workgroup of this (stream, kv head) ----
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned old = atomicAdd(&a.counters[b * a.Hkv + kvh], 1u);
    s_last = (old == static_cast<unsigned>(n_splits - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  for (int idx = tid; idx < G * DH; idx += 256) {
    const int g = idx / DH;
    const int d = idx % DH;
    const long bh = static_cast<long>(b) * Hq + kvh * G + g;
    const long base = bh * a.max_splits;
    float mx = -INFINITY;
    for (int sp = 0; sp < n_splits; ++sp) mx = fmaxf(mx, a.part_ml[(base + sp) * 2]);
    float num = 0.0f, den = 0.0f;
    for (int sp = 0; sp < n_splits; ++sp) {
      const float w = fast_exp2(a.part_ml[(base + sp) * 2] - mx);
      num = fmaf(w, a.part_o[(base + sp) * DH + d], num);
      den = fmaf(w, a.part_ml[(base + sp) * 2 + 1], den);
    }
    a.out[bh * DH + d] = num * (1.0f / den);
  }
  if (tid == 0) a.counters[b * a.Hkv + kvh] = 0u;
}

template <int DH, int G, int SPLIT>
int launch_split(const DecodeArgs& args, int B, hipStream_t stream) {
  dim3 grid(args.max_splits, args.Hkv, B);
  hipLaunchKernelGGL((gqa_decode_kernel<DH, G, SPLIT>), grid, dim3(256), 0, stream, args);
  return check_launch("gqa_decode_kernel");
}

template <int DH, int G>
int launch_dh_g(const DecodeArgs& args, int B, int split, hipStream_t stream) {
  switch (split) {
    case 64: return launch_split<DH, G, 64>(args, B, stream);
    case 128: return launch_split<DH, G, 128>(args, B, stream);
    default: return launch_split<DH, G, 256>(args, B, stream);
  }
}

}  // namespace

int launch_gqa_decode(const DecodeProblem& p, hipStream_t stream) {
  if (p.B <= 0 || p.Hq <= 0 || p.Hkv <= 0 || p.Dh <= 0) return ORATOR_OK;  // reference no-op
  if (!p.q || !p.kpool || !p.vpool || !p.pos || !p.out)
    return fail(ORATOR_ERR_INVALID, "gqa_decode: null pointer");
  if (p.Hq % p.Hkv) return fail(ORATOR_ERR_INVALID, "gqa_decode: Hq must be a multiple of Hkv");
  const int G = p.Hq / p.Hkv;
  if (!(p.Dh == 64 || p.Dh == 128) || !(G == 1 || G == 2 || G == 4))
    return fail(ORATOR_ERR_UNSUPPORTED, "gqa_decode: supported Dh {64,128}, Hq/Hkv {1,2,4}");
  if (p.capacity <= 0) return fail(ORATOR_ERR_INVALID, "gqa_decode: capacity must be > 0");
  int page_shift = 0;
  if (p.page_table) {
    page_shift = ilog2_exact(p.page_size);
    if (page_shift < 4 || p.max_pages <= 0)
      return fail(ORATOR_ERR_INVALID, "gqa_decode: page_size must be a power of two >= 16");
    if (static_cast<long>(p.max_pages) * p.page_size < p.capacity)
      return fail(ORATOR_ERR_CAPACITY, "gqa_decode: capacity exceeds max_pages*page_size");
  }
  // Largest split that still puts >= 1024 workgroups (4 per CU) on the device.
  int split = 64;
  for (int cand : {256, 128}) {
    const long wgs = static_cast<long>(p.B) * p.Hkv * ((p.capacity + cand - 1) / cand);
    if (wgs >= 1024) {
      split = cand;
      break;
    }
  }
  const int max_splits = (p.capacity + split - 1) / split;
  const long counters = static_cast<long>(p.B) * p.Hkv;
  if (counters * 4 > static_cast<long>(kCounterBytes))
    return fail(ORATOR_ERR_UNSUPPORTED, "gqa_decode: B*Hkv exceeds the combine counter pool");
  const size_t part_o = static_cast<size_t>(p.B) * p.Hq * max_splits * p.Dh * sizeof(float);
  const size_t part_ml = static_cast<size_t>(p.B) * p.Hq * max_splits * 2 * sizeof(float);
  char* ws = static_cast<char*>(workspace(stream, kCounterBytes + part_o + part_ml, kCounterBytes));
  if (!ws) return ORATOR_ERR_HIP;

  DecodeArgs args;
  args.q = p.q;
  args.kpool = p.kpool;
  args.vpool = p.vpool;
  args.page_table = p.page_table;
  args.pos = p.pos;
  args.out = p.out;
  args.counters = reinterpret_cast<unsigned*>(ws);
  args.part_o = reinterpret_cast<float*>(ws + kCounterBytes);
  args.part_ml = reinterpret_cast<float*>(ws + kCounterBytes + part_o);
  args.stream_stride = p.stream_stride;
  args.max_pages = p.max_pages;
  args.page_shift = page_shift;
  args.Hkv = p.Hkv;
  args.max_splits = max_splits;
  args.capacity = p.capacity;
  args.scale_log2e = p.scale * 1.4426950408889634f;

  if (p.Dh == 128) {
    if (G == 1) return launch_dh_g<128, 1>(args, p.B, split, stream);
    if (G == 2) return launch_dh_g<128, 2>(args, p.B, split, stream);
    return launch_dh_g<128, 4>(args, p.B, split, stream);
  }
  if (G == 1) return launch_dh_g<64, 1>(args, p.B, split, stream);
  if (G == 2) return launch_dh_g<64, 2>(args, p.B, split, stream);
  return launch_dh_g<64, 4>(args, p.B, split, stream);
}

}  // namespace orator_hip

using namespace orator_hip;

extern "C" {

int orator_gqa_decode(const float* q, const uint16_t* kc, const uint16_t* vc, float* out, int Hq,
                      int Hkv, int Dh, const int* d_pos, int capacity, float scale, void* stream) {
  DecodeProblem p{};
  p.q = q;
  p.kpool = kc;
  p.vpool = vc;
  p.page_table = nullptr;
  p.stream_stride = 0;
  p.pos = d_pos;
  p.out = out;
  p.B = 1;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.Dh = Dh;
  p.capacity = capacity;
  p.scale = scale;
  return launch_gqa_decode(p, static_cast<hipStream_t>(stream));
}

int orator_gqa_decode_paged(const float* q, const uint16_t* kpool, const uint16_t* vpool,
                            const int* page_table, int max_pages, int page_size, const int* d_pos,
                            float* out, int B, int Hq, int Hkv, int Dh, float scale,
                            void* stream) {
  if (!page_table && B > 0) return fail(ORATOR_ERR_INVALID, "gqa_decode_paged: null page table");
  DecodeProblem p{};
  p.q = q;
  p.kpool = kpool;
  p.vpool = vpool;
  p.page_table = page_table;
  p.max_pages = max_pages;
  p.page_size = page_size;
  p.pos = d_pos;
  p.out = out;
  p.B = B;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.Dh = Dh;
  p.capacity = max_pages * page_size;
  p.scale = scale;
  return launch_gqa_decode(p, static_cast<hipStream_t>(stream));
}

}  // extern "C"
