// Causal GQA prefill attention over a bf16 KV cache on MFMA (gfx950).
//
// Replaces GqaCacheAttnKernel (src/model/asr_text_decoder.cu:88-142): query row t (absolute
// position pos0 + t) attends keys [0, pos0 + t] of the cache; online softmax; out = acc/l,
// or 0 when l == 0.  K/V are bf16 in the cache, accumulation is fp32.
//
// Two precisions share the kernel:
//  * bf16 mode: q (and the softmax weights fed to the PV product) rounded to bf16 -- one
//    v_mfma_f32_32x32x16_bf16 per product;
//  * fp32 mode: q carried as three bf16 terms (hi + mid + lo, exact to fp32 rounding) and
//    the softmax weights as two (hi + lo, ~2^-17 relative); K/V are exact in bf16, so QK is
//    fp32-exact and PV within ~1e-6 of the fp32 reference, at 2.5x the MFMA work.
//
// Tiling (one workgroup = 4 wave64s = 128 query rows = 64 tokens x 2 heads of one GQA
// group; K/V tiles of 64 keys shared by both heads through LDS):
//  * S^T = K Q^T: K tile rows are the MFMA A operand (ds_read_b128 from a padded,
//    conflict-free LDS layout), the wave's 32 query columns stay in registers as B.  In the
//    32x32 accumulator layout every lane owns ONE query column and 16 keys, so the row
//    max / sum of the online softmax are in-lane plus one lane exchange (xor 32).
//  * O^T += V^T P^T: P^T comes straight from the S^T accumulators (no LDS round trip);
//    V^T is read from an LDS copy of the tile that is transposed while it is stored.
//  * K/V tiles are re-read by every token block of the head, so they use plain (L2-
//    cached) loads; the next tile is loaded from HBM into registers while the current one is
//    multiplied, then stored to the other LDS buffer (double buffering, one barrier/tile).
//  * workgroups are ordered heaviest (latest tokens, most keys) first, and the kv head is
//    the fastest-varying index, so each kv head's workgroups share an XCD (blockIdx % 8).
#include "common.hpp"
#include "internal.hpp"

namespace orator_hip {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kDh = 128;
constexpr int kBN = 64;              // keys per tile
constexpr int kKRow = kDh + 8;       // padded K row (bf16 elements): 272 bytes
constexpr int kVRow = kBN + 8;       // padded V^T row: 144 bytes
constexpr int kMaxRowGroups = 1024;  // page-row table: up to 16384 keys

struct PrefillArgs {
  const float* q;         // [Tq, Hq, Dh] fp32, or
  const uint16_t* q_bf16; // [Tq, Hq, Dh] bf16 (then q == nullptr)
  const uint16_t* kpool;
  const uint16_t* vpool;
  const int* page_table;  // nullptr => contiguous cache
  int page_shift;
  const int* pos0p;
  float* out;
  int Tq, Hq, Hkv;
  int capacity;
  int n_tblocks;
  float scale_log2e;
};

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8_t, u); }

__device__ __forceinline__ f32x16_t mfma32(bf16x8_t a, bf16x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Splits 8 fp32 into bf16 hi (RNE) and the bf16 of the remainder (x - hi is exact in fp32).
__device__ __forceinline__ void split8(float (&x)[8], uint4& hi, uint4& lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint16_t h0 = f32_to_bf16(x[2 * e]), h1 = f32_to_bf16(x[2 * e + 1]);
    h[e] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16);
    x[2 * e] -= bf16_to_f32(h0);
    x[2 * e + 1] -= bf16_to_f32(h1);
    l[e] = pack_bf16x2(x[2 * e], x[2 * e + 1]);
  }
  hi = make_uint4(h[0], h[1], h[2], h[3]);
  lo = make_uint4(l[0], l[1], l[2], l[3]);
}

template <int G, bool PRECISE>
__global__ __launch_bounds__(256) void gqa_prefill_kernel(PrefillArgs a) {
  constexpr int TW = 32 / G;   // tokens per wave (32 query columns = TW tokens x G heads)
  constexpr int BT = 4 * TW;   // tokens per workgroup
  __shared__ uint16_t k_lds[2][kBN][kKRow];
  __shared__ uint16_t vt_lds[2][kDh][kVRow];
  __shared__ int row_lds[kMaxRowGroups];

  const int kvh = blockIdx.x % a.Hkv;
  const int tblock = a.n_tblocks - 1 - static_cast<int>(blockIdx.x / a.Hkv);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int h2 = lane >> 5;     // which half of the 32x32 accumulator rows this lane holds
  const int col = lane & 31;    // this lane's query column
  const int pos0 = *a.pos0p;

  const int t_blk = tblock * BT;
  const int t_end = min(t_blk + BT, a.Tq);
  const int n_keys = min(pos0 + t_end, a.capacity);  // keys [0, n_keys) are needed
  const int n_tiles = (n_keys + kBN - 1) / kBN;

  // ---- page rows of the needed keys (16-key groups) ----
  const int n_groups = (n_keys + 15) >> 4;
  for (int gi = tid; gi < n_groups; gi += 256) {
    int row = gi << 4;
    if (a.page_table) {
      const int j0 = gi << 4;
      const int page = a.page_table[j0 >> a.page_shift];
      row = (page << a.page_shift) | (j0 & ((1 << a.page_shift) - 1));
    }
    row_lds[gi] = row;
  }

  // ---- this wave's query columns: token tq, head hq ----
  const int tq = t_blk + wave * TW + (col % TW);
  const int hq = kvh * G + col / TW;
  const bool q_valid = tq < a.Tq;
  const int q_lim = pos0 + tq;  // last key this column may attend
  // B operand per 16-dim k-step (dims 16ks + 8*h2 + e).  fp32 mode carries q as three bf16
  // terms hi + mid + lo (exact to fp32 rounding); bf16 mode uses hi only.
  uint4 qhi[8], qmid[8], qlo[8];
  {
    const long qoff = (static_cast<long>(tq) * a.Hq + hq) * kDh + 8 * h2;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      qmid[ks] = qlo[ks] = make_uint4(0, 0, 0, 0);
      if (!q_valid) {
        qhi[ks] = make_uint4(0, 0, 0, 0);
      } else if (a.q) {
        const float4 x0 = *reinterpret_cast<const float4*>(a.q + qoff + 16 * ks);
        const float4 x1 = *reinterpret_cast<const float4*>(a.q + qoff + 16 * ks + 4);
        float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        split8(xs, qhi[ks], qmid[ks]);
        if (PRECISE) split8(xs, qmid[ks], qlo[ks]);
      } else {
        qhi[ks] = *reinterpret_cast<const uint4*>(a.q_bf16 + qoff + 16 * ks);
      }
    }
  }
  __syncthreads();  // row_lds ready

  // ---- tile loader: K rows as 16-byte chunks, V as key pairs for the transposed store ----
  const long rs = static_cast<long>(a.Hkv) * kDh;
  const uint16_t* kbase = a.kpool + static_cast<long>(kvh) * kDh;
  const uint16_t* vbase = a.vpool + static_cast<long>(kvh) * kDh;
  uint4 kreg[4], vreg[2][2];
  auto load_tile = [&](int n) {
    const int k0 = n * kBN;
#pragma unroll
    for (int p = 0; p < 4; ++p) {  // 16 keys per pass, 16 lanes per 256-byte row
      const int key = k0 + 16 * p + (tid >> 4);
      kreg[p] = key < n_keys ? *reinterpret_cast<const uint4*>(
                                   kbase + (row_lds[key >> 4] + (key & 15)) * rs + 8 * (tid & 15))
                             : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {  // key pair kp, 8 dims at 8*dc
      const int kp = 16 * u + (tid >> 4);
      const int key = k0 + 2 * kp;
      const int dc = tid & 15;
#pragma unroll
      for (int t = 0; t < 2; ++t)
        vreg[u][t] = key + t < n_keys
                         ? *reinterpret_cast<const uint4*>(
                               vbase + (row_lds[(key + t) >> 4] + ((key + t) & 15)) * rs + 8 * dc)
                         : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int p = 0; p < 4; ++p)
      *reinterpret_cast<uint4*>(&k_lds[buf][16 * p + (tid >> 4)][8 * (tid & 15)]) = kreg[p];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int kp = 16 * u + (tid >> 4);
      const int dc = tid & 15;
      const uint32_t w0[4] = {vreg[u][0].x, vreg[u][0].y, vreg[u][0].z, vreg[u][0].w};
      const uint32_t w1[4] = {vreg[u][1].x, vreg[u][1].y, vreg[u][1].z, vreg[u][1].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // dims 8dc+2e (low halves) and 8dc+2e+1 (high halves) of keys 2kp, 2kp+1
        const uint32_t lo = (w0[e] & 0xffffu) | (w1[e] << 16);
        const uint32_t hi = (w0[e] >> 16) | (w1[e] & 0xffff0000u);
        *reinterpret_cast<uint32_t*>(&vt_lds[buf][8 * dc + 2 * e][2 * kp]) = lo;
        *reinterpret_cast<uint32_t*>(&vt_lds[buf][8 * dc + 2 * e + 1][2 * kp]) = hi;
      }
    }
  };

  f32x16_t o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.0f;
  float m = -INFINITY, lsum = 0.0f;

  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int n = 0; n < n_tiles; ++n) {
    const int buf = n & 1;
    if (n + 1 < n_tiles) load_tile(n + 1);

    // S^T for keys [64n, 64n+64): two 32-key accumulators
    f32x16_t s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int e = 0; e < 16; ++e) s[kt][e] = 0.0f;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const bf16x8_t ka = as_bf16x8(
            *reinterpret_cast<const uint4*>(&k_lds[buf][32 * kt + col][16 * ks + 8 * h2]));
        if (PRECISE) {  // small terms first
          s[kt] = mfma32(ka, as_bf16x8(qlo[ks]), s[kt]);
          s[kt] = mfma32(ka, as_bf16x8(qmid[ks]), s[kt]);
        }
        s[kt] = mfma32(ka, as_bf16x8(qhi[ks]), s[kt]);
      }
    }
    // scale, causal mask, online softmax (this lane: one query column, 32 keys of the tile)
    const int kbase_n = kBN * n + 4 * h2;
    float tmax = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = kbase_n + 32 * kt + 8 * (e >> 2) + (e & 3);
        const float v = (q_valid && key <= q_lim) ? s[kt][e] * a.scale_log2e : -INFINITY;
        s[kt][e] = v;
        tmax = fmaxf(tmax, v);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float mn = fmaxf(m, tmax);
    const float mref = mn == -INFINITY ? 0.0f : mn;  // fully masked column (padding token)
    const float corr = fast_exp2(m - mref);
    m = mn;
    float psum = 0.0f;
    uint4 phi[4], plo[4];  // B operand per 16-key k-step a: keys 16a + 8(e/4) + 4*h2 + e%4
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pv[e] = fast_exp2(s[st >> 1][8 * (st & 1) + e] - mref);
        psum += pv[e];
      }
      if (PRECISE) {
        split8(pv, phi[st], plo[st]);
      } else {
        phi[st] = make_uint4(pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3]),
                             pack_bf16x2(pv[4], pv[5]), pack_bf16x2(pv[6], pv[7]));
      }
    }
    lsum = lsum * corr + psum;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[dt][e] *= corr;
    // O^T[dims, queries] += V^T[dims, keys] P^T[keys, queries]
#pragma unroll
    for (int st = 0; st < 4; ++st) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const uint16_t* vr = &vt_lds[buf][32 * dt + col][16 * st + 4 * h2];
        const uint2 v0 = *reinterpret_cast<const uint2*>(vr);
        const uint2 v1 = *reinterpret_cast<const uint2*>(vr + 8);
        const bf16x8_t va = as_bf16x8(make_uint4(v0.x, v0.y, v1.x, v1.y));
        o[dt] = mfma32(va, as_bf16x8(phi[st]), o[dt]);
        if (PRECISE) o[dt] = mfma32(va, as_bf16x8(plo[st]), o[dt]);
      }
    }
    if (n + 1 < n_tiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- normalise and store: lane owns query column `col`, dims 32dt + 8i + 4*h2 + j ----
  lsum += __shfl_xor(lsum, 32);
  if (!q_valid) return;
  const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
  float* orow = a.out + (static_cast<long>(tq) * a.Hq + hq) * kDh + 4 * h2;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<float4*>(orow + 32 * dt + 8 * i) =
          make_float4(o[dt][4 * i] * inv, o[dt][4 * i + 1] * inv, o[dt][4 * i + 2] * inv,
                      o[dt][4 * i + 3] * inv);
}

template <int G>
int launch_g(const PrefillArgs& args, bool precise, hipStream_t stream) {
  const dim3 grid(args.n_tblocks * args.Hkv);
  if (precise)
    hipLaunchKernelGGL((gqa_prefill_kernel<G, true>), grid, dim3(256), 0, stream, args);
  else
    hipLaunchKernelGGL((gqa_prefill_kernel<G, false>), grid, dim3(256), 0, stream, args);
  return check_launch("gqa_prefill_kernel");
}

int launch_prefill(const float* q, const uint16_t* q_bf16, const uint16_t* kpool,
                   const uint16_t* vpool, const int* page_table, int max_pages, int page_size,
                   float* out, int Tq, int Hq, int Hkv, int Dh, const int* d_pos0, int capacity,
                   float scale, int mode, hipStream_t stream) {
  if (Tq <= 0 || Hq <= 0 || Hkv <= 0 || Dh <= 0) return ORATOR_OK;  // reference no-op
  if ((!q && !q_bf16) || !kpool || !vpool || !out || !d_pos0)
    return fail(ORATOR_ERR_INVALID, "gqa_prefill: null pointer");
  if (Hq % Hkv) return fail(ORATOR_ERR_INVALID, "gqa_prefill: Hq must be a multiple of Hkv");
  const int G = Hq / Hkv;
  if (Dh != kDh || !(G == 1 || G == 2 || G == 4))
    return fail(ORATOR_ERR_UNSUPPORTED, "gqa_prefill: supported Dh 128, Hq/Hkv {1,2,4}");
  if (mode != ORATOR_PREFILL_FP32 && mode != ORATOR_PREFILL_BF16)
    return fail(ORATOR_ERR_INVALID, "gqa_prefill: unknown precision mode");
  if (capacity <= 0) return fail(ORATOR_ERR_INVALID, "gqa_prefill: capacity must be > 0");
  if (capacity > 16 * kMaxRowGroups)
    return fail(ORATOR_ERR_UNSUPPORTED, "gqa_prefill: more than 16384 cached keys");
  PrefillArgs args{};
  args.page_shift = 0;
  if (page_table) {
    args.page_shift = ilog2_exact(page_size);
    if (args.page_shift < 4 || max_pages <= 0)
      return fail(ORATOR_ERR_INVALID, "gqa_prefill: page_size must be a power of two >= 16");
    if (static_cast<long>(max_pages) * page_size < capacity)
      return fail(ORATOR_ERR_CAPACITY, "gqa_prefill: capacity exceeds max_pages*page_size");
  }
  args.q = q;
  args.q_bf16 = q ? nullptr : q_bf16;
  args.kpool = kpool;
  args.vpool = vpool;
  args.page_table = page_table;
  args.pos0p = d_pos0;
  args.out = out;
  args.Tq = Tq;
  args.Hq = Hq;
  args.Hkv = Hkv;
  args.capacity = capacity;
  args.scale_log2e = scale * 1.4426950408889634f;
  const int BT = 4 * (32 / G);
  args.n_tblocks = (Tq + BT - 1) / BT;
  const bool precise = mode == ORATOR_PREFILL_FP32;
  if (G == 1) return launch_g<1>(args, precise, stream);
  if (G == 2) return launch_g<2>(args, precise, stream);
  return launch_g<4>(args, precise, stream);
}

}  // namespace
}  // namespace orator_hip

using namespace orator_hip;

extern "C" {

int orator_gqa_prefill(const float* q, const uint16_t* kc, const uint16_t* vc, float* out, int Tq,
                       int Hq, int Hkv, int Dh, const int* d_pos0, int capacity, float scale,
                       void* stream) {
  return launch_prefill(q, nullptr, kc, vc, nullptr, 0, 0, out, Tq, Hq, Hkv, Dh, d_pos0, capacity,
                        scale, ORATOR_PREFILL_FP32, static_cast<hipStream_t>(stream));
}

int orator_gqa_prefill_ex(const float* q, const uint16_t* q_bf16, const uint16_t* kpool,
                          const uint16_t* vpool, const int* page_table, int max_pages,
                          int page_size, float* out, int Tq, int Hq, int Hkv, int Dh,
                          const int* d_pos0, int capacity, float scale, int mode, void* stream) {
  return launch_prefill(q, q_bf16, kpool, vpool, page_table, max_pages, page_size, out, Tq, Hq,
                        Hkv, Dh, d_pos0, capacity, scale, mode, static_cast<hipStream_t>(stream));
}

}  // extern "C"
