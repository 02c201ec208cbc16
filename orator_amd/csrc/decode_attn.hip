// Split-K (flash-decoding) GQA decode attention over a bf16 KV cache, gfx950.
//
// Replaces GqaDecodeAttnKernel (src/model/asr_text_decoder.cu:149-213): one fp32 query
// per q-head attends S = pos+1 cached keys.  Semantics kept: fp32 q, bf16 K/V widened
// exactly, fp32 accumulation, scores scaled after the dot, softmax normalised by
// multiplying with 1/sum.  Exponents are taken base 2 on scores pre-multiplied by
// log2(e) (same value up to fp32 rounding).
//
// Design (HBM-bound, ~2 flop/byte):
//  * one workgroup = (split of SPLIT keys, kv head, stream), 4 wave64s; each wave streams
//    a contiguous quarter of the split in 32-key chunks.  All G q heads of the GQA group
//    consume every K/V row the wave loads, so K/V leave HBM exactly once.  At the default
//    128-key splits every wave issues its whole chunk (16 KB of K and V) at once.
//  * longer splits: software pipeline, the K and V loads of chunk c+1 are issued before
//    chunk c is computed (two chunk buffers).
//  * QK, "octet" layout: 8 lanes per key, each lane 2 x 16-byte loads (one contiguous
//    128-byte half row per instruction and octet); dot reduced with 3 DPP steps.
//  * online softmax per wave (running max / sum, accumulator rescale once per chunk);
//    probabilities move to the PV layout with one lane shuffle per key row.
//  * PV, "row" layout: Dh/8 lanes per key, one 16-byte load each (whole contiguous rows
//    per instruction); per-lane accumulators hold 8 dims x G heads.
//  * waves merge in LDS at the end.  Splits are merged either by a second small kernel (one
//    memory round trip for up to 34 splits: loads issued together, online max), or, for
//    small grids, inside the split launch by the last workgroup of each (stream, kv head)
//    to finish: partials written and read as agent-scope atomics (coherent across the XCDs'
//    L2s without the L2 write-back a device-scope release fence costs, which measured 7-10x
//    slower) and an arrival counter.  One launch instead of two is what a single stream
//    gains most from.
//  * paged KV: each wave reads the two page-table entries of its chunk with uniform loads
//    at entry, together with the stream's position; no workgroup-wide table and no barrier
//    stand between the entry and the K/V loads.  Keys past the range load the last valid
//    row (branch-free; their weights are 0).
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>

#include "common.hpp"
#include "internal.hpp"

namespace orator_hip {
namespace {

struct DecodeArgs {
  const float* q;
  const void* kpool;  // bf16 bits or fp32, per the kernel's KV type
  const void* vpool;
  const int* page_table;
  const int* pos;      // [B]: stream b attends pos[b]+1 keys (pos_mode 0)
  int pos_mode;        // 0: pos[b]+1 keys; 1: b+1 keys (causal self-attn); 2: capacity keys;
                       // 3: keys [seg_start[b], seg_end[b]) (windowed self-attention)
  const int* seg_start;
  const int* seg_end;
  float* out;
  float* part_o;       // [B*Hq][max_splits][DH]
  float* part_ml;      // [B*Hq][max_splits][2]
  // [B*Hkv] arrival counters, zero between launches: when set, the split kernel's last
  // workgroup of each (stream, kv head) merges the splits (no second launch)
  unsigned* arrive;
  long stream_stride;
  int max_pages;
  int page_shift;
  int Hkv;
  int max_splits;
  int capacity;
  float scale_log2e;
  // Append (pos_mode 0, bf16 caches): the new token's K/V rows [B][Hkv][DH] fp32 are written
  // at position pos[b] and attended as the last key; nullptr when there is nothing to append.
  const float* k_new;
  const float* v_new;
  long pool_rows;  // rows the pools hold (paged writes past it are dropped)
  // QK-norm + RoPE folded in (the QKN kernels): see DecodeProblem
  const float* q_norm;
  const float* k_norm;
  const float* rope;
  float eps;
};

// RmsNorm (weights w, eps) + rotate-half RoPE (cos, sin of pairs j = EPV * o + e at cs) of one
// 128-dim head held in the octet layout: lane o of each 8-lane group owns dims 8o + e and
// 64 + 8o + e (x[e], x[8 + e]), so every RoPE pair is lane-local; the sum of squares is
// reduced over the octet.  Same operations as the fused QK-norm/RoPE kernel (no contraction).
// The operands are loaded by load_norm_rope (this lane's 16 weights and 8 (cos, sin) pairs,
// 16-byte loads) so that a caller can have them in flight with other loads before it waits.
struct NormRope {
  float w[16];   // w[8o + e], w[64 + 8o + e]
  float cs[16];  // cos, sin of pairs 8o .. 8o + 7
};
__device__ __forceinline__ void load_norm_rope(NormRope& nr, const float* w, const float* cs,
                                               int o) {
  const float4* w0 = reinterpret_cast<const float4*>(w + 8 * o);
  const float4* w1 = reinterpret_cast<const float4*>(w + 64 + 8 * o);
  const float4* c4 = reinterpret_cast<const float4*>(cs + 16 * o);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float4 a = w0[i], b = w1[i];
    nr.w[4 * i] = a.x; nr.w[4 * i + 1] = a.y; nr.w[4 * i + 2] = a.z; nr.w[4 * i + 3] = a.w;
    nr.w[8 + 4 * i] = b.x; nr.w[9 + 4 * i] = b.y; nr.w[10 + 4 * i] = b.z; nr.w[11 + 4 * i] = b.w;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 c = c4[i];
    nr.cs[4 * i] = c.x; nr.cs[4 * i + 1] = c.y; nr.cs[4 * i + 2] = c.z; nr.cs[4 * i + 3] = c.w;
  }
}
__device__ __forceinline__ void norm_rope_apply(float (&x)[16], const NormRope& nr, float eps) {
#pragma clang fp contract(off)
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) ss += x[i] * x[i];
  ss += dpp<0xB1>(ss);
  ss += dpp<0x4E>(ss);
  ss += dpp<0x141>(ss);
  const float inv = rsqrt_via_f64(ss / 128.0f + eps);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float n0 = x[e] * inv * nr.w[e], n1 = x[8 + e] * inv * nr.w[8 + e];
    const float c = nr.cs[2 * e], s = nr.cs[2 * e + 1];
    x[e] = n0 * c - n1 * s;
    x[8 + e] = n1 * c + n0 * s;
  }
}
__device__ __forceinline__ void qk_norm_rope_octet(float (&x)[16], const float* w, float eps,
                                                   const float* cs, int o) {
  NormRope nr;
  load_norm_rope(nr, w, cs, o);
  norm_rope_apply(x, nr, eps);
}

// Number of keys stream b attends, clamped to the capacity; pos_b = pos[b] (pos_mode 0).
__device__ __forceinline__ int stream_keys(const DecodeArgs& a, int b, int pos_b) {
  if (a.pos_mode == 3) {  // window [seg_start, seg_end) clamped into [0, capacity)
    const int j0 = min(max(a.seg_start[b], 0), a.capacity);
    return min(max(a.seg_end[b], j0), a.capacity) - j0;
  }
  const int S = a.pos_mode == 0 ? pos_b + 1 : (a.pos_mode == 1 ? b + 1 : a.capacity);
  return S > a.capacity ? a.capacity : S;
}

// First key row of stream b's range (non-zero only for windows).
__device__ __forceinline__ int stream_key0(const DecodeArgs& a, int b) {
  return a.pos_mode == 3 ? min(max(a.seg_start[b], 0), a.capacity) : 0;
}

// Pool rows of keys c and c + 16 (c a multiple of 16) of stream b, whose range starts at pool
// key key0 (windows; 0 otherwise): through the page table for paged caches (pages hold >= 16
// aligned keys), else the key offset by key0.  Both table indices are clamped into the table
// (capacity - 1 at most) and depend on nothing loaded, so the two reads go out together at
// entry; a row past the stream's keys is never dereferenced (the chunk loads clamp to the
// last valid key).  Called with wave-uniform arguments: no workgroup-wide table, no barrier.
// A readable zero word: the address the entry load of a lane uses when its value is not needed.
__device__ int g_decode_zero[1] = {0};  // never written

__device__ __forceinline__ void chunk_rows(const DecodeArgs& a, int b, int key0, int c, long& r0,
                                           long& r1) {
  const int lim = a.capacity - 1;
  const int j0 = min(c, lim) & ~15, j1 = min(c + 16, lim) & ~15;
  if (a.page_table) {
    const int* pt = a.page_table + static_cast<long>(b) * a.max_pages;
    const int p0 = pt[j0 >> a.page_shift], p1 = pt[j1 >> a.page_shift];
    const int msk = (1 << a.page_shift) - 1;
    // long arithmetic: an unmapped page (< 0) yields a negative row, never a wrapped one
    r0 = static_cast<long>(p0) * (1L << a.page_shift) + (j0 & msk);
    r1 = static_cast<long>(p1) * (1L << a.page_shift) + (j1 & msk);
  } else {
    r0 = j0 + key0;
    r1 = j1 + key0;
  }
}

// Element helpers: K/V rows are bf16 (cache) or fp32 (self-attention over fp32 K/V).
template <typename KV>
struct KvElem {
  static constexpr int EPV = 16 / sizeof(KV);  // elements per 16-byte load
  // element e of a 16-byte load, widened to fp32
  static __device__ __forceinline__ float get(const uint4& u, int e) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
    if constexpr (sizeof(KV) == 2)
      return (e & 1) ? bf16_hi(w[e >> 1]) : bf16_lo(w[e >> 1]);
    else
      return __uint_as_float(w[e]);
  }
};

template <int DH, typename KV>
struct Chunk {
  static constexpr int EPV = KvElem<KV>::EPV;
  static constexpr int CH = sizeof(KV) == 2 ? 32 : 16;  // keys per chunk (same bytes)
  static constexpr int NCQ = DH / (8 * EPV);    // 16-byte loads per lane per key (octet layout)
  static constexpr int QPL = NCQ * EPV;         // dims per lane in the octet layout
  static constexpr int NIQ = CH / 8;            // octet iterations per chunk
  static constexpr int LPT = DH / 8;            // lanes per key, row layout (8 dims per lane)
  static constexpr int NV = 8 / EPV;            // 16-byte loads per lane per key, row layout
  static constexpr int TPI = kWave / LPT;       // keys per row-layout instruction
  static constexpr int NIV = CH / TPI;          // row-layout instructions per chunk
  uint4 k[NIQ][NCQ];
  uint4 v[NIV][NV];
};

// Loads one 32-key chunk starting at absolute key c; rb0 / rb1 are the pool rows of keys c and
// c + 16.
// Octet layout: lane o of a key's 8 lanes reads bytes 128*cc + 16*o of the row.  Keys at or
// past `end` load the row of key end-1 instead (branch-free, always in bounds): their scores
// are masked to -inf, so their weights are exactly 0 and the finite row adds nothing.
template <int DH, typename KV>
__device__ __forceinline__ void load_chunk(Chunk<DH, KV>& ch, const KV* kbase, const KV* vbase,
                                           long rb0, long rb1, long rs, int c, int end,
                                           int lane) {
  using CK = Chunk<DH, KV>;
  constexpr int EPV = CK::EPV;
  const int o = lane & 7;
  const int last = end - 1 - c;  // last valid key within the chunk (>= 0)
#pragma unroll
  for (int i = 0; i < CK::NIQ; ++i) {
    const int kk = min(8 * i + (lane >> 3), last);  // key within the chunk
    const long row = (kk < 16 ? rb0 : rb1) + (kk & 15);
    const KV* src = kbase + row * rs + EPV * o;
#pragma unroll
    for (int cc = 0; cc < CK::NCQ; ++cc) ch.k[i][cc] = load_nt(src + 8 * EPV * cc);
  }
  const int dg = lane % CK::LPT;
  const int r = lane / CK::LPT;
#pragma unroll
  for (int i = 0; i < CK::NIV; ++i) {
    const int kk = min(CK::TPI * i + r, last);
    const long row = (kk < 16 ? rb0 : rb1) + (kk & 15);
    const KV* src = vbase + row * rs + 8 * dg;
#pragma unroll
    for (int u = 0; u < CK::NV; ++u) ch.v[i][u] = load_nt(src + EPV * u);
  }
}

// Scores, online-softmax update and PV accumulation for one resident chunk at key c.
template <int DH, int G, typename KV>
__device__ __forceinline__ void process_chunk(const Chunk<DH, KV>& cur,
                                              const float (&qr)[G][Chunk<DH, KV>::QPL],
                                              float (&m)[G], float (&lpart)[G],
                                              float (&acc)[G][8], int c, int end, int lane,
                                              float scale_log2e) {
  using CK = Chunk<DH, KV>;
  using E = KvElem<KV>;
  // scores, octet layout
  float s[CK::NIQ][G];
#pragma unroll
  for (int i = 0; i < CK::NIQ; ++i) {
    float d[G];
#pragma unroll
    for (int g = 0; g < G; ++g) d[g] = 0.0f;
#pragma unroll
    for (int cc = 0; cc < CK::NCQ; ++cc) {
#pragma unroll
      for (int e = 0; e < CK::EPV; ++e) {
        const float kv = E::get(cur.k[i][cc], e);
#pragma unroll
        for (int g = 0; g < G; ++g) d[g] = fmaf(qr[g][cc * CK::EPV + e], kv, d[g]);
      }
    }
    const bool valid = c + 8 * i + (lane >> 3) < end;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float dot = d[g];
      dot += dpp<0xB1>(dot);
      dot += dpp<0x4E>(dot);
      dot += dpp<0x141>(dot);
      s[i][g] = valid ? dot * scale_log2e : -INFINITY;
    }
  }
  // online softmax update (one rescale per chunk)
  float pk[CK::NIQ][G];
  const int o = lane & 7;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float cm = s[0][g];
#pragma unroll
    for (int i = 1; i < CK::NIQ; ++i) cm = fmaxf(cm, s[i][g]);
    cm = fmaxf(cm, __shfl_xor(cm, 8));
    cm = fmaxf(cm, __shfl_xor(cm, 16));
    cm = fmaxf(cm, __shfl_xor(cm, 32));
    const float mn = fmaxf(m[g], cm);
    const float corr = fast_exp2(m[g] - mn);
    m[g] = mn;
    float ps = 0.0f;
#pragma unroll
    for (int i = 0; i < CK::NIQ; ++i) {
      pk[i][g] = fast_exp2(s[i][g] - mn);
      ps += pk[i][g];
    }
    lpart[g] = lpart[g] * corr + (o == 0 ? ps : 0.0f);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] *= corr;
  }
  // PV, row layout: the probability of key row r comes from its octet by a lane shuffle
  const int r = lane / CK::LPT;
#pragma unroll
  for (int i = 0; i < CK::NIV; ++i) {
    const int src = 8 * ((CK::TPI * i + r) & 7);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float p = __shfl(pk[(CK::TPI * i) >> 3][g], src);
#pragma unroll
      for (int u = 0; u < CK::NV; ++u)
#pragma unroll
        for (int e = 0; e < CK::EPV; ++e)
          acc[g][u * CK::EPV + e] = fmaf(p, E::get(cur.v[i][u], e), acc[g][u * CK::EPV + e]);
    }
  }
}

// The appended key (bf16-rounded from the fp32 input, exactly what the cache will hold)
// folded into a wave's running softmax state: the score in every octet (octet layout, all
// 64 lanes hold it after the reduction), one lane adds its weight to the row sum, the r == 0
// lanes its weighted V row.  Returns this lane's bf16 K (octet layout) and V (row layout)
// pieces for the cache write.
template <int DH, int G, bool QKN>
__device__ __forceinline__ void append_key(const float* kn, const float* vn,
                                           const float (&qr)[G][Chunk<DH, uint16_t>::QPL],
                                           float (&m)[G], float (&lpart)[G], float (&acc)[G][8],
                                           int lane, float scale_log2e,
                                           uint4 (&kw)[Chunk<DH, uint16_t>::NCQ], uint4& vw,
                                           const float* k_norm, float eps, const float* cs) {
  using CK = Chunk<DH, uint16_t>;
  const int o = lane & 7;
  float kf[CK::QPL];
  float kx[CK::QPL];
#pragma unroll
  for (int cc = 0; cc < CK::NCQ; ++cc) {
    const float4 x0 = *reinterpret_cast<const float4*>(kn + 8 * CK::EPV * cc + CK::EPV * o);
    const float4 x1 = *reinterpret_cast<const float4*>(kn + 8 * CK::EPV * cc + CK::EPV * o + 4);
    kx[cc * 8 + 0] = x0.x; kx[cc * 8 + 1] = x0.y; kx[cc * 8 + 2] = x0.z; kx[cc * 8 + 3] = x0.w;
    kx[cc * 8 + 4] = x1.x; kx[cc * 8 + 5] = x1.y; kx[cc * 8 + 6] = x1.z; kx[cc * 8 + 7] = x1.w;
  }
  if constexpr (QKN) qk_norm_rope_octet(kx, k_norm, eps, cs, o);
#pragma unroll
  for (int cc = 0; cc < CK::NCQ; ++cc) {
    kw[cc] = make_uint4(pack_bf16x2(kx[cc * 8 + 0], kx[cc * 8 + 1]),
                        pack_bf16x2(kx[cc * 8 + 2], kx[cc * 8 + 3]),
                        pack_bf16x2(kx[cc * 8 + 4], kx[cc * 8 + 5]),
                        pack_bf16x2(kx[cc * 8 + 6], kx[cc * 8 + 7]));
    const uint32_t w[4] = {kw[cc].x, kw[cc].y, kw[cc].z, kw[cc].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) kf[cc * 8 + e] = (e & 1) ? bf16_hi(w[e >> 1]) : bf16_lo(w[e >> 1]);
  }
  const int dg = lane % CK::LPT;
  const float4 y0 = *reinterpret_cast<const float4*>(vn + 8 * dg);
  const float4 y1 = *reinterpret_cast<const float4*>(vn + 8 * dg + 4);
  vw = make_uint4(pack_bf16x2(y0.x, y0.y), pack_bf16x2(y0.z, y0.w), pack_bf16x2(y1.x, y1.y),
                  pack_bf16x2(y1.z, y1.w));
  const uint32_t vwd[4] = {vw.x, vw.y, vw.z, vw.w};
  const bool row0 = lane < CK::LPT;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float d = 0.0f;
#pragma unroll
    for (int i = 0; i < CK::QPL; ++i) d = fmaf(qr[g][i], kf[i], d);
    d += dpp<0xB1>(d);
    d += dpp<0x4E>(d);
    d += dpp<0x141>(d);
    const float sc = d * scale_log2e;
    const float mn = fmaxf(m[g], sc);
    const float corr = fast_exp2(m[g] - mn);
    const float p = fast_exp2(sc - mn);
    m[g] = mn;
    lpart[g] = lpart[g] * corr + (lane == 0 ? p : 0.0f);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float vv = (e & 1) ? bf16_hi(vwd[e >> 1]) : bf16_lo(vwd[e >> 1]);
      acc[g][e] = acc[g][e] * corr + (row0 ? p * vv : 0.0f);
    }
  }
}

// ---- split merge: the combine kernel, or the split kernel's last workgroup ----
// Splits' maxima, sums and partial rows are loaded kSplitBatch at a time and folded in with an
// online max; the next batch is in flight while the current one is folded, so up to 34
// splits (4352 keys at 128-key splits) cost one memory round trip.
constexpr int kSplitBatch = 17;
struct SplitBatch {
  float m[kSplitBatch], l[kSplitBatch], o[kSplitBatch];
};

// Device-coherent (agent-scope) float store and load.  The XCDs' L2 caches are not coherent
// with each other; agent-scope atomic accesses are (the store is complete at the coherent
// level once the wave's store counter has drained, the load reads that level), without the
// L2 write-back an agent-scope release fence costs.
__device__ __forceinline__ void store_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Splits s0 .. s0 + kSplitBatch - 1 of partial row `base` (= (stream * Hq + q head) *
// max_splits), dim d.  Slots past the launch's splits are clamped to its last (an in-range
// address); slots past the stream's splits hold stale data and are excluded by the fold's
// selects.  DEV: device-coherent loads (partials written by other workgroups of this launch).
template <int DH, bool DEV>
__device__ __forceinline__ void load_splits(SplitBatch& x, const DecodeArgs& a, long base, int s0,
                                            int d) {
#pragma unroll
  for (int i = 0; i < kSplitBatch; ++i) {
    const long ps = base + min(s0 + i, a.max_splits - 1);
    if constexpr (DEV) {
      x.m[i] = load_dev(a.part_ml + ps * 2);
      x.l[i] = load_dev(a.part_ml + ps * 2 + 1);
      x.o[i] = load_dev(a.part_o + ps * DH + d);
    } else {
      x.m[i] = a.part_ml[ps * 2];
      x.l[i] = a.part_ml[ps * 2 + 1];
      x.o[i] = a.part_o[ps * DH + d];
    }
  }
}

__device__ __forceinline__ void fold_splits(const SplitBatch& x, int s0, int n_splits, float& M,
                                            float& L, float& acc) {
  float mx = M;
#pragma unroll
  for (int i = 0; i < kSplitBatch; ++i)
    if (s0 + i < n_splits) mx = fmaxf(mx, x.m[i]);
  const float c_old = M == mx ? 1.0f : fast_exp2(M - mx);
  acc *= c_old;
  L *= c_old;
#pragma unroll
  for (int i = 0; i < kSplitBatch; ++i) {
    if (s0 + i < n_splits) {
      const float w = fast_exp2(x.m[i] - mx);
      acc = fmaf(w, x.o[i], acc);
      L = fmaf(w, x.l[i], L);
    }
  }
  M = mx;
}

// The merged output of dim d over n_splits (>= 2) splits; A holds splits 0 .. kSplitBatch - 1
// (loaded by the caller, so its loads can go out before n_splits is known).
template <int DH, bool DEV>
__device__ __forceinline__ float merge_splits(const DecodeArgs& a, long base, int d, int n_splits,
                                              SplitBatch& A) {
  SplitBatch Bb;
  float M = -INFINITY, L = 0.0f, acc = 0.0f;
  // ping-pong: the next batch's loads are issued before the current one is folded
  for (int s0 = 0;;) {
    if (s0 + kSplitBatch < n_splits) load_splits<DH, DEV>(Bb, a, base, s0 + kSplitBatch, d);
    fold_splits(A, s0, n_splits, M, L, acc);
    s0 += kSplitBatch;
    if (s0 >= n_splits) break;
    if (s0 + kSplitBatch < n_splits) load_splits<DH, DEV>(A, a, base, s0 + kSplitBatch, d);
    fold_splits(Bb, s0, n_splits, M, L, acc);
    s0 += kSplitBatch;
    if (s0 >= n_splits) break;
  }
  return acc * (1.0f / L);
}

// The merged output of dim d over n_splits (2 .. 64) splits of partial row `base`, for a
// wave whose lanes all merge the same row (dims d): lane s loads split s's maximum and sum
// (one load each for the wave, where every lane loading every split's took 2 per split), the
// weights are formed once per split and broadcast by lane, and the partial rows are loaded
// kWaveMergeBatch at a time, the next batch in flight while one is folded.
constexpr int kWaveMergeBatch = 24;
template <int DH>
__device__ __forceinline__ float merge_splits_wave(const DecodeArgs& a, long base, int d,
                                                   int n_splits, int lane) {
  float o_a[kWaveMergeBatch], o_b[kWaveMergeBatch];
  auto load_o = [&](float (&o)[kWaveMergeBatch], int s0) {
#pragma unroll
    for (int i = 0; i < kWaveMergeBatch; ++i)
      o[i] = load_dev(a.part_o + (base + min(s0 + i, n_splits - 1)) * DH + d);
  };
  float ms = -INFINITY, ls = 0.0f;
  if (lane < n_splits) {
    ms = load_dev(a.part_ml + (base + lane) * 2);
    ls = load_dev(a.part_ml + (base + lane) * 2 + 1);
  }
  load_o(o_a, 0);
  if (kWaveMergeBatch < n_splits) load_o(o_b, kWaveMergeBatch);
  const float mx = wave_max(ms);
  const float w = lane < n_splits ? fast_exp2(ms - mx) : 0.0f;  // a split's -inf: weight 0
  const float L = wave_sum(w * ls);
  float acc = 0.0f;
  auto fold = [&](const float (&o)[kWaveMergeBatch], int s0) {
#pragma unroll
    for (int i = 0; i < kWaveMergeBatch; ++i)
      if (s0 + i < n_splits)  // uniform
        acc = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), s0 + i)), o[i], acc);
  };
  for (int s0 = 0;;) {
    fold(o_a, s0);
    s0 += kWaveMergeBatch;
    if (s0 >= n_splits) break;
    if (s0 + kWaveMergeBatch < n_splits) load_o(o_a, s0 + kWaveMergeBatch);
    fold(o_b, s0);
    s0 += kWaveMergeBatch;
    if (s0 >= n_splits) break;
    if (s0 + kWaveMergeBatch < n_splits) load_o(o_b, s0 + kWaveMergeBatch);
  }
  return acc * (1.0f / L);
}

// Waves per split workgroup: bf16 splits of 256 / 512 keys give every wave one 32-key
// chunk (8 / 16 waves); otherwise 4 waves.
template <int SPLIT, typename KV, int G>
constexpr int decode_waves() {
  return (sizeof(KV) == 2 && G <= 2 && SPLIT >= 256 && SPLIT <= 512) ? SPLIT / 32 : 4;
}

// FUSE: the splits are merged by the last workgroup of each (stream, kv head) to finish
// (a.arrive set), else by the combine kernel.
template <int DH, int G, int SPLIT, typename KV, bool QKN, bool FUSE>
__global__ __launch_bounds__((64 * decode_waves<SPLIT, KV, G>())) __attribute__((
    amdgpu_waves_per_eu(2))) void gqa_decode_kernel(DecodeArgs a) {
  static_assert(!QKN || (DH == 128 && sizeof(KV) == 2), "QK-norm folding: Dh 128, bf16 caches");
  using CK = Chunk<DH, KV>;
  constexpr int NW = decode_waves<SPLIT, KV, G>();
  constexpr int NT = 64 * NW;
  constexpr int TPW = SPLIT / NW;  // keys per wave
  static_assert(TPW % CK::CH == 0, "a wave covers whole chunks");

  __shared__ float red_o[NW][G][DH];
  __shared__ float red_ml[NW][G][2];

  // split index slowest: the short last splits of the streams are dispatched last, where
  // they fill the drain of the final round instead of lengthening it
  const int kvh = blockIdx.x;
  const int b = blockIdx.y;
  const int split = blockIdx.z;
  const int t0 = split * SPLIT;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: wave-level branches
  // The stream's position (lane 0) and the page-table entries of the wave's first chunk (keys
  // w0, w0 + 16; lanes 1, 2) in one vector load, one wait: as separate uniform loads behind
  // the branches for absent arrays, each got a wait of its own before the next was issued.
  // Table indices are clamped into the table (capacity - 1 at most).
  const int lim = a.capacity - 1;
  const int wj0 = min(t0 + wave * TPW, lim) & ~15, wj1 = min(t0 + wave * TPW + 16, lim) & ~15;
  const bool paged = a.page_table != nullptr;
  const int* ptb = a.page_table + static_cast<long>(b) * a.max_pages;
  const int* esrc = g_decode_zero;
  if (lane == 0 && a.pos_mode == 0) esrc = a.pos + b;
  if (lane == 1 && paged) esrc = ptb + (wj0 >> a.page_shift);
  if (lane == 2 && paged) esrc = ptb + (wj1 >> a.page_shift);
  const int eld = *esrc;
  // ---- q of the G heads, octet layout: lane owns dims 8*EPV*cc + EPV*o + e; loaded while
  // the position is in flight (q does not depend on it) ----
  const int o = lane & 7;
  float qr[G][CK::QPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float* qh = a.q + (static_cast<long>(b) * a.Hkv * G + kvh * G + g) * DH + CK::EPV * o;
#pragma unroll
    for (int cc = 0; cc < CK::NCQ; ++cc)
#pragma unroll
      for (int e4 = 0; e4 < CK::EPV; e4 += 4) {
        const float4 x = *reinterpret_cast<const float4*>(qh + 8 * CK::EPV * cc + e4);
        qr[g][cc * CK::EPV + e4] = x.x;
        qr[g][cc * CK::EPV + e4 + 1] = x.y;
        qr[g][cc * CK::EPV + e4 + 2] = x.z;
        qr[g][cc * CK::EPV + e4 + 3] = x.w;
      }
  }
  const int pos_b = a.pos_mode == 0 ? __builtin_amdgcn_readlane(eld, 0) : 0;
  const int key0 = stream_key0(a, b);
  long wr0, wr1;
  if (paged) {
    const int msk = (1 << a.page_shift) - 1;
    // long arithmetic: an unmapped page (< 0) yields a negative row, never a wrapped one
    wr0 = static_cast<long>(__builtin_amdgcn_readlane(eld, 1)) * (1L << a.page_shift) + (wj0 & msk);
    wr1 = static_cast<long>(__builtin_amdgcn_readlane(eld, 2)) * (1L << a.page_shift) + (wj1 & msk);
  } else {
    wr0 = wj0 + key0;
    wr1 = wj1 + key0;
  }
  int S = stream_keys(a, b, pos_b);
  if (S <= 0) {  // no keys: the reference's 1/sum guard yields zeros
    if (split == 0)
      for (int idx = threadIdx.x; idx < G * DH; idx += NT)
        a.out[(static_cast<long>(b) * a.Hkv * G + kvh * G) * DH + idx] = 0.0f;
    return;
  }
  if (t0 >= S) return;
  const int n_splits = (S + SPLIT - 1) / SPLIT;
  const int Hq = a.Hkv * G;

  // QK-norm folding: the q-norm weights and the position's RoPE pairs are loaded here, ahead
  // of the wave's K/V chunk, and applied after the chunk's loads are issued: loads return in
  // issue order, so the q-norm then runs while the chunk streams in (applied before the
  // chunk's loads went out, it delayed them by the table read and the norm, ~1.1 us per
  // layer at B = 1).
  const float* rope_cs = nullptr;  // (cos, sin) pairs of this stream's position (QKN)
  NormRope qnr;
  if constexpr (QKN) {
    rope_cs = a.rope + static_cast<long>(min(max(pos_b, 0), a.capacity - 1)) * DH;
    load_norm_rope(qnr, a.q_norm, rope_cs, o);
  }

  const long kv_base = (a.page_table ? 0 : static_cast<long>(b) * a.stream_stride) +
                       static_cast<long>(kvh) * DH;
  const KV* kbase = static_cast<const KV*>(a.kpool) + kv_base;
  const KV* vbase = static_cast<const KV*>(a.vpool) + kv_base;
  const long rs = static_cast<long>(a.Hkv) * DH;  // elements per pool row
  // The appended key (the stream's last, S - 1) is not read from the cache: this launch
  // writes it.  The cache holds S_cache keys; the wave streams [w0, w_end) of them and the
  // wave whose range would hold the new key folds it in afterwards.
  int new_key = -1;
  if constexpr (sizeof(KV) == 2)
    if (a.k_new && S == pos_b + 1) new_key = S - 1;
  const int S_cache = new_key >= 0 ? S - 1 : S;
  const int w0 = t0 + wave * TPW;
  const int w_end = min(w0 + TPW, S_cache);
  const bool owns_new = new_key >= w0 && new_key < w0 + TPW;
  const float* kn = nullptr;
  const float* vn = nullptr;
  if (owns_new) {
    kn = a.k_new + (static_cast<long>(b) * a.Hkv + kvh) * DH;
    vn = a.v_new + (static_cast<long>(b) * a.Hkv + kvh) * DH;
  }

  float m[G], lpart[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    lpart[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.0f;
  }
  const int r = lane / CK::LPT;

  auto apply_qnorm = [&]() {
    if constexpr (QKN) {
#pragma unroll
      for (int g = 0; g < G; ++g) norm_rope_apply(qr[g], qnr, a.eps);
    }
  };
  if constexpr (TPW == CK::CH) {
    // one chunk per wave (128-key splits): no second buffer
    if (w0 < w_end) {
      CK A;
      load_chunk<DH, KV>(A, kbase, vbase, wr0, wr1, rs, w0, w_end, lane);
      apply_qnorm();
      process_chunk<DH, G, KV>(A, qr, m, lpart, acc, w0, w_end, lane, a.scale_log2e);
    } else {
      apply_qnorm();  // the appended key's score needs the normed q
    }
  } else if (w0 < w_end) {
    // Ping-pong buffers: the loads of one chunk are in flight while the other is computed.
    CK A, Bb;
    load_chunk<DH, KV>(A, kbase, vbase, wr0, wr1, rs, w0, w_end, lane);
    apply_qnorm();
    int c = w0;
    while (true) {
      if (c + CK::CH < w_end) {
        long r0, r1;
        chunk_rows(a, b, key0, c + CK::CH, r0, r1);
        load_chunk<DH, KV>(Bb, kbase, vbase, r0, r1, rs, c + CK::CH, w_end, lane);
      }
      process_chunk<DH, G, KV>(A, qr, m, lpart, acc, c, w_end, lane, a.scale_log2e);
      c += CK::CH;
      if (c >= w_end) break;
      if (c + CK::CH < w_end) {
        long r0, r1;
        chunk_rows(a, b, key0, c + CK::CH, r0, r1);
        load_chunk<DH, KV>(A, kbase, vbase, r0, r1, rs, c + CK::CH, w_end, lane);
      }
      process_chunk<DH, G, KV>(Bb, qr, m, lpart, acc, c, w_end, lane, a.scale_log2e);
      c += CK::CH;
      if (c >= w_end) break;
    }
  } else {
    apply_qnorm();  // no cached keys in this wave's range: the appended key may still be its
  }
  if constexpr (sizeof(KV) == 2) {
    if (owns_new) {  // uniform over the wave
      uint4 kw[CK::NCQ], vw;
      append_key<DH, G, QKN>(kn, vn, qr, m, lpart, acc, lane, a.scale_log2e, kw, vw, a.k_norm,
                             a.eps, rope_cs);
      // write the new row into the cache; a row outside the pool (an unmapped page, < 0, or
      // a page past the pool) is dropped, as the KV write does
      long row, row_unused;
      chunk_rows(a, b, key0, new_key & ~15, row, row_unused);
      row += new_key & 15;
      if (row >= 0 && row < a.pool_rows) {
        uint16_t* kdst = const_cast<uint16_t*>(reinterpret_cast<const uint16_t*>(kbase)) + row * rs;
        uint16_t* vdst = const_cast<uint16_t*>(reinterpret_cast<const uint16_t*>(vbase)) + row * rs;
        if (lane < 8)
#pragma unroll
          for (int cc = 0; cc < CK::NCQ; ++cc)
            *reinterpret_cast<uint4*>(kdst + 8 * CK::EPV * cc + CK::EPV * (lane & 7)) = kw[cc];
        if (lane < CK::LPT) *reinterpret_cast<uint4*>(vdst + 8 * (lane % CK::LPT)) = vw;
      }
    }
  }

  // ---- wave partials -> LDS ----
#pragma unroll
  for (int off = CK::LPT; off < kWave; off <<= 1)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] += __shfl_xor(acc[g][e], off);
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float l = wave_sum(lpart[g]);
    if (lane == 0) {
      red_ml[wave][g][0] = m[g];
      red_ml[wave][g][1] = l;
    }
  }
  if (r == 0) {
    const int dg = lane % CK::LPT;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float4* dst = reinterpret_cast<float4*>(&red_o[wave][g][8 * dg]);
      dst[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
      dst[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
    }
  }
  __syncthreads();

  // ---- merge the waves; write the split partial (or the output if it is the only split) ----
  for (int idx = tid; idx < G * DH; idx += NT) {
    const int g = idx / DH;
    const int d = idx % DH;
    float mx = red_ml[0][g][0];
#pragma unroll
    for (int w = 1; w < NW; ++w) mx = fmaxf(mx, red_ml[w][g][0]);
    float ov = 0.0f, lv = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = fast_exp2(red_ml[w][g][0] - mx);  // idle waves: 2^-inf = 0
      ov = fmaf(wt, red_o[w][g][d], ov);
      lv = fmaf(wt, red_ml[w][g][1], lv);
    }
    const long bh = static_cast<long>(b) * Hq + kvh * G + g;
    if (n_splits == 1) {
      a.out[bh * DH + d] = ov * (1.0f / lv);
    } else {
      const long ps = bh * a.max_splits + split;
      if constexpr (FUSE) {
        store_dev(a.part_o + ps * DH + d, ov);
        if (d == 0) {
          store_dev(a.part_ml + ps * 2, mx);
          store_dev(a.part_ml + ps * 2 + 1, lv);
        }
      } else {
        a.part_o[ps * DH + d] = ov;
        if (d == 0) {
          a.part_ml[ps * 2] = mx;
          a.part_ml[ps * 2 + 1] = lv;
        }
      }
    }
  }
  if constexpr (FUSE) {
    if (n_splits == 1) return;
    // ---- in-launch split merge: the last workgroup of (stream, kv head) to arrive ----
    // Every thread's partial stores have completed at the coherent level (vmcnt 0) before
    // the barrier; then one thread counts the workgroup in.  The workgroup whose add brings
    // the count to n_splits reads the partials (issued after the add returned) and returns
    // the counter to zero for the next launch.
    __shared__ int s_last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      unsigned* ctr = a.arrive + (static_cast<long>(b) * a.Hkv + kvh) * kCounterStride;
      const unsigned prev =
          __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = prev + 1 == static_cast<unsigned>(n_splits);
      if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = last;
    }
    __syncthreads();
    if (!s_last) return;
    for (int idx = tid; idx < G * DH; idx += NT) {
      const int g = idx / DH;
      const int d = idx % DH;
      const long bh = static_cast<long>(b) * Hq + kvh * G + g;
      const long base = bh * a.max_splits;
      if (n_splits <= kWave && DH % kWave == 0) {  // a wave's lanes share g: wave-wide merge
        a.out[bh * DH + d] = merge_splits_wave<DH>(a, base, d, n_splits, lane);
      } else {
        SplitBatch A;
        load_splits<DH, true>(A, a, base, 0, d);
        a.out[bh * DH + d] = merge_splits<DH, true>(a, base, d, n_splits, A);
      }
    }
  }
}

// Wide split kernel for many streams (B * Hkv pairs >= half the CUs): each (stream, kv head)
// is cut into `parts` ranges of `split_len` keys (a multiple of 256, fixed by the capacity so
// the page-table entries of every chunk are known before the position is; the last range runs
// to the capacity), one workgroup of kWideWaves waves per range.  Wave w takes the range's 32-key chunks w, w + 8, ... in a
// ping-pong loop (the next chunk's K/V loads are in flight while the current one is
// computed), so a workgroup keeps ~128 KB of K/V in flight for its whole life instead of
// paying a dispatch, an entry round trip and a barrier per 64 KB.  The entry load reads the
// position and the page-table entries of every chunk of the wave at once (lane 2k, 2k + 1:
// chunk k; lane 63: the position).  Partials go to the split merge (range index = split).
constexpr int kWideWaves = 8;
constexpr int kWideMaxChunks = 31;  // chunks per wave: 2 table entries each in lanes 0..61

// FUSE: the ranges are merged by the last workgroup of each (stream, kv head) to finish
// (a.arrive set), else by the combine kernel.
template <int DH, int G, bool FUSE>
__global__ __launch_bounds__(64 * kWideWaves) __attribute__((amdgpu_waves_per_eu(2)))
void gqa_decode_wide_kernel(DecodeArgs a, int split_len) {
  using KV = uint16_t;
  using CK = Chunk<DH, KV>;
  constexpr int NW = kWideWaves;
  constexpr int NT = 64 * NW;
  __shared__ float red_o[NW][G][DH];
  __shared__ float red_ml[NW][G][2];

  const int kvh = blockIdx.x;
  const int b = blockIdx.y;
  const int part = blockIdx.z;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int p0 = part * split_len;  // first key of this range
  const int lim = a.capacity - 1;
  const bool paged = a.page_table != nullptr;
  // entry load: lanes 2k, 2k + 1 the page-table entries of keys c_k, c_k + 16 of the wave's
  // chunk k (c_k = p0 + 32 (wave + NW k)), lane 63 the stream's position
  const int* esrc = g_decode_zero;
  {
    const int k = lane >> 1;
    const int key = min(p0 + 32 * (wave + NW * k) + 16 * (lane & 1), lim) & ~15;
    if (paged && lane < 2 * kWideMaxChunks)
      esrc = a.page_table + static_cast<long>(b) * a.max_pages + (key >> a.page_shift);
    if (lane == 63 && a.pos_mode == 0) esrc = a.pos + b;
  }
  const int eld = *esrc;
  const int pos_b = a.pos_mode == 0 ? __builtin_amdgcn_readlane(eld, 63) : 0;
  const int S = stream_keys(a, b, pos_b);
  if (S <= 0) {
    if (part == 0)
      for (int idx = tid; idx < G * DH; idx += NT)
        a.out[(static_cast<long>(b) * a.Hkv * G + kvh * G) * DH + idx] = 0.0f;
    return;
  }
  if (p0 >= S) return;
  // ranges of split_len keys, the last one (range max_splits - 1) running to the capacity
  const int n_parts = min((S + split_len - 1) / split_len, a.max_splits);
  const int p_end = part == a.max_splits - 1 ? a.capacity : p0 + split_len;
  const int Hq = a.Hkv * G;
  const int o = lane & 7;
  float qr[G][CK::QPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float* qh = a.q + (static_cast<long>(b) * Hq + kvh * G + g) * DH + CK::EPV * o;
#pragma unroll
    for (int cc = 0; cc < CK::NCQ; ++cc)
#pragma unroll
      for (int e4 = 0; e4 < CK::EPV; e4 += 4) {
        const float4 x = *reinterpret_cast<const float4*>(qh + 8 * CK::EPV * cc + e4);
        qr[g][cc * CK::EPV + e4] = x.x;
        qr[g][cc * CK::EPV + e4 + 1] = x.y;
        qr[g][cc * CK::EPV + e4 + 2] = x.z;
        qr[g][cc * CK::EPV + e4 + 3] = x.w;
      }
  }
  const long kv_base = (paged ? 0 : static_cast<long>(b) * a.stream_stride) +
                       static_cast<long>(kvh) * DH;
  const KV* kbase = static_cast<const KV*>(a.kpool) + kv_base;
  const KV* vbase = static_cast<const KV*>(a.vpool) + kv_base;
  const long rs = static_cast<long>(a.Hkv) * DH;
  int new_key = -1;
  if (a.k_new && S == pos_b + 1) new_key = S - 1;
  const int S_cache = new_key >= 0 ? S - 1 : S;
  const int r_end = min(p_end, S_cache);  // this range's cached keys: [p0, r_end)
  // rows of keys c_k, c_k + 16 of chunk k (wave-uniform)
  auto rows = [&](int k, long& r0, long& r1) {
    const int c = p0 + 32 * (wave + NW * k);
    const int j0 = min(c, lim) & ~15, j1 = min(c + 16, lim) & ~15;
    if (paged) {
      const int msk = (1 << a.page_shift) - 1;
      r0 = static_cast<long>(__builtin_amdgcn_readlane(eld, 2 * k)) * (1L << a.page_shift) + (j0 & msk);
      r1 = static_cast<long>(__builtin_amdgcn_readlane(eld, 2 * k + 1)) * (1L << a.page_shift) + (j1 & msk);
    } else {
      r0 = j0;
      r1 = j1;
    }
  };
  // chunks of this wave holding cached keys: c_k < r_end
  const int first = p0 + 32 * wave;
  const int n_ch = first < r_end ? (r_end - first + 32 * NW - 1) / (32 * NW) : 0;

  float m[G], lpart[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    lpart[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.0f;
  }
  if (n_ch > 0) {
    CK A, Bb;
    long r0, r1;
    rows(0, r0, r1);
    load_chunk<DH, KV>(A, kbase, vbase, r0, r1, rs, first, r_end, lane);
    for (int k = 0;;) {
      const int c = first + 32 * NW * k;
      if (k + 1 < n_ch) {
        rows(k + 1, r0, r1);
        load_chunk<DH, KV>(Bb, kbase, vbase, r0, r1, rs, c + 32 * NW, r_end, lane);
      }
      process_chunk<DH, G, KV>(A, qr, m, lpart, acc, c, r_end, lane, a.scale_log2e);
      if (++k >= n_ch) break;
      const int c2 = first + 32 * NW * k;
      if (k + 1 < n_ch) {
        rows(k + 1, r0, r1);
        load_chunk<DH, KV>(A, kbase, vbase, r0, r1, rs, c2 + 32 * NW, r_end, lane);
      }
      process_chunk<DH, G, KV>(Bb, qr, m, lpart, acc, c2, r_end, lane, a.scale_log2e);
      if (++k >= n_ch) break;
    }
  }
  // the appended key: folded in by the wave whose chunk slot holds it, then written
  if (new_key >= p0 && new_key < p_end && ((new_key - p0) >> 5) % NW == wave) {
    const float* kn = a.k_new + (static_cast<long>(b) * a.Hkv + kvh) * DH;
    const float* vn = a.v_new + (static_cast<long>(b) * a.Hkv + kvh) * DH;
    uint4 kw[CK::NCQ], vw;
    append_key<DH, G, false>(kn, vn, qr, m, lpart, acc, lane, a.scale_log2e, kw, vw, nullptr,
                             0.0f, nullptr);
    long row, row_unused;
    chunk_rows(a, b, 0, new_key & ~15, row, row_unused);
    row += new_key & 15;
    if (row >= 0 && row < a.pool_rows) {
      uint16_t* kdst = const_cast<uint16_t*>(kbase) + row * rs;
      uint16_t* vdst = const_cast<uint16_t*>(vbase) + row * rs;
      if (lane < 8)
#pragma unroll
        for (int cc = 0; cc < CK::NCQ; ++cc)
          *reinterpret_cast<uint4*>(kdst + 8 * CK::EPV * cc + CK::EPV * (lane & 7)) = kw[cc];
      if (lane < CK::LPT) *reinterpret_cast<uint4*>(vdst + 8 * (lane % CK::LPT)) = vw;
    }
  }

  // ---- wave partials -> LDS -> the range's partial (or the output) ----
  const int r = lane / CK::LPT;
#pragma unroll
  for (int off = CK::LPT; off < kWave; off <<= 1)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] += __shfl_xor(acc[g][e], off);
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float l = wave_sum(lpart[g]);
    if (lane == 0) {
      red_ml[wave][g][0] = m[g];
      red_ml[wave][g][1] = l;
    }
  }
  if (r == 0) {
    const int dg = lane % CK::LPT;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float4* dst = reinterpret_cast<float4*>(&red_o[wave][g][8 * dg]);
      dst[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
      dst[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
    }
  }
  __syncthreads();
  for (int idx = tid; idx < G * DH; idx += NT) {
    const int g = idx / DH;
    const int d = idx % DH;
    float mx = red_ml[0][g][0];
#pragma unroll
    for (int w = 1; w < NW; ++w) mx = fmaxf(mx, red_ml[w][g][0]);
    float ov = 0.0f, lv = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = fast_exp2(red_ml[w][g][0] - mx);
      ov = fmaf(wt, red_o[w][g][d], ov);
      lv = fmaf(wt, red_ml[w][g][1], lv);
    }
    const long bh = static_cast<long>(b) * Hq + kvh * G + g;
    if (n_parts == 1) {
      a.out[bh * DH + d] = ov * (1.0f / lv);
    } else {
      const long ps = bh * a.max_splits + part;
      if constexpr (FUSE) {
        store_dev(a.part_o + ps * DH + d, ov);
        if (d == 0) {
          store_dev(a.part_ml + ps * 2, mx);
          store_dev(a.part_ml + ps * 2 + 1, lv);
        }
      } else {
        a.part_o[ps * DH + d] = ov;
        if (d == 0) {
          a.part_ml[ps * 2] = mx;
          a.part_ml[ps * 2 + 1] = lv;
        }
      }
    }
  }
  if constexpr (FUSE) {
    if (n_parts == 1) return;
    // ---- in-launch range merge: the last workgroup of (stream, kv head) to arrive, as in
    // the split kernel; its own range's partial is read back like the others, four ranges'
    // loads in flight at a time ----
    __shared__ int s_last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      unsigned* ctr = a.arrive + (static_cast<long>(b) * a.Hkv + kvh) * kCounterStride;
      const unsigned prev =
          __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = prev + 1 == static_cast<unsigned>(n_parts);
      if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = last;
    }
    __syncthreads();
    if (!s_last) return;
    for (int idx = tid; idx < G * DH; idx += NT) {
      const int g = idx / DH;
      const int d = idx % DH;
      const long bh = static_cast<long>(b) * Hq + kvh * G + g;
      const long base = bh * a.max_splits;
      float M = -INFINITY, L = 0.0f, acc = 0.0f;
      for (int s0 = 0; s0 < n_parts; s0 += 4) {
        float pm[4], pl[4], po[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const long ps = base + min(s0 + i, n_parts - 1);
          pm[i] = load_dev(a.part_ml + ps * 2);
          pl[i] = load_dev(a.part_ml + ps * 2 + 1);
          po[i] = load_dev(a.part_o + ps * DH + d);
        }
        float mx = M;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (s0 + i < n_parts) mx = fmaxf(mx, pm[i]);
        const float c_old = M == mx ? 1.0f : fast_exp2(M - mx);
        acc *= c_old;
        L *= c_old;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (s0 + i < n_parts) {
            const float w = fast_exp2(pm[i] - mx);
            acc = fmaf(w, po[i], acc);
            L = fmaf(w, pl[i], L);
          }
        }
        M = mx;
      }
      a.out[bh * DH + d] = acc * (1.0f / L);
    }
  }
}

// Measurement: the decode operation's K/V bytes read with nothing else (no arithmetic, no
// partials, no merge): grid (kv head, stream, 128-key split), 4 waves, each wave one 32-key
// chunk of K and of V through the page table with the non-temporal loads the decode kernels
// use.  Its time is the streaming ceiling of this access pattern on the device.
__global__ __launch_bounds__(256) void decode_read_probe_kernel(const uint16_t* __restrict__ kp,
                                                                const uint16_t* __restrict__ vp,
                                                                const int* __restrict__ table,
                                                                int max_pages, int page_shift,
                                                                int S, int Hkv,
                                                                unsigned* __restrict__ sink) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kvh = blockIdx.x, b = blockIdx.y;
  const int c0 = (blockIdx.z * 4 + wave) * 32;  // first key of the wave's chunk
  if (c0 >= S) return;
  const int last = S - 1;
  const int* pt = table + static_cast<long>(b) * max_pages;
  const long rs = static_cast<long>(Hkv) * 128;
  const int sub = lane >> 4, ch = lane & 15;  // 4 keys x 16 pieces of 16 bytes per load
  unsigned acc = 0;
  uint4 kv[8], vv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int key = min(c0 + 4 * i + sub, last);
    const long row = static_cast<long>(pt[key >> page_shift]) * (1L << page_shift) +
                     (key & ((1 << page_shift) - 1));
    const long off = row * rs + kvh * 128 + 8 * ch;
    kv[i] = load_nt(kp + off);
    vv[i] = load_nt(vp + off);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) acc ^= kv[i].x ^ kv[i].w ^ vv[i].y ^ vv[i].z;
  if (acc == 0x9e3779b9u && lane == 0) sink[0] = acc;  // keeps the loads; practically never
}

__global__ __launch_bounds__(256) void zero_u32_kernel(unsigned* p) {
  p[blockIdx.x * 256 + threadIdx.x] = 0u;
}

// Split merge: one workgroup per (stream, q head), after the split kernel; thread d owns
// output dim d (the split fold above, plain loads).
template <int DH>
__global__ __launch_bounds__(DH) void gqa_decode_combine_kernel(DecodeArgs a, int split_len,
                                                                int Hq) {
  // x = kv head + Hkv * (q head within the group): the kv head is the fastest grid index, as
  // in the split kernel, so with 8 kv heads a head's merge runs on the XCD (workgroup index %
  // 8) that ran its splits.  Measured 0.9 us per op faster than q-head order (B = 16, L = 4096,
  // same box), though the partials are still fetched from memory either way.
  const int G = Hq / a.Hkv;
  const int h = (blockIdx.x % a.Hkv) * G + blockIdx.x / a.Hkv;
  const int b = blockIdx.y;
  const long bh = static_cast<long>(b) * Hq + h;
  const long base = bh * a.max_splits;
  const int d = threadIdx.x;
  // Addresses use the launch's split count, not the stream's, so the first batch goes out
  // together with the read of the stream's position instead of after it.
  SplitBatch A;
  load_splits<DH, false>(A, a, base, 0, d);
  // the stream's position, read by lane 0 of each wave in a vector load that every thread
  // issues (the others read a zero word): as a uniform load behind the branch for an absent
  // position array, it and the pointer it needs cost two round trips before the batch's row
  // loads
  const int* psrc = ((d & 63) == 0 && a.pos_mode == 0) ? a.pos + b : g_decode_zero;
  const int pos_ld = *psrc;
  asm volatile("" ::: "memory");  // keeps the batch's loads here, ahead of the early return
  const int S = stream_keys(a, b, a.pos_mode == 0 ? __builtin_amdgcn_readlane(pos_ld, 0) : 0);
  // (the wide kernel's last range runs to the capacity: at most max_splits ranges)
  const int n_splits = min((S + split_len - 1) / split_len, a.max_splits);
  if (n_splits <= 1) return;  // written directly by the split kernel
  a.out[bh * DH + d] = merge_splits<DH, false>(a, base, d, n_splits, A);
}

template <int DH, int G, int SPLIT, typename KV, bool QKN>
void launch_split_kernel(const DecodeArgs& args, dim3 grid, hipStream_t stream) {
  constexpr int NT = 64 * decode_waves<SPLIT, KV, G>();
  if constexpr (sizeof(KV) == 2) {
    if (args.arrive) {
      hipLaunchKernelGGL((gqa_decode_kernel<DH, G, SPLIT, KV, QKN, true>), grid, dim3(NT), 0,
                         stream, args);
      return;
    }
  }
  hipLaunchKernelGGL((gqa_decode_kernel<DH, G, SPLIT, KV, QKN, false>), grid, dim3(NT), 0, stream,
                     args);
}

template <int DH, int G, int SPLIT, typename KV>
int launch_split(const DecodeArgs& args, int B, hipStream_t stream) {
  dim3 grid(args.Hkv, B, args.max_splits);
  hipEvent_t ev0, ev_split, ev1;
  take_timing_events(&ev0, &ev_split, &ev1);
  if (ev0) (void)hipEventRecord(ev0, stream);
  bool launched = false;
  if constexpr (DH == 128 && sizeof(KV) == 2) {
    if (args.q_norm) {
      launch_split_kernel<DH, G, SPLIT, KV, true>(args, grid, stream);
      launched = true;
    }
  }
  if (!launched) launch_split_kernel<DH, G, SPLIT, KV, false>(args, grid, stream);
  int rc = check_launch("gqa_decode_kernel");
  if (ev_split) (void)hipEventRecord(ev_split, stream);
  if (!rc && args.max_splits > 1 && !args.arrive) {
    hipLaunchKernelGGL((gqa_decode_combine_kernel<DH>), dim3(args.Hkv * G, B), dim3(DH), 0,
                       stream, args, SPLIT, args.Hkv * G);
    rc = check_launch("gqa_decode_combine_kernel");
  }
  if (ev1) (void)hipEventRecord(ev1, stream);
  return rc;
}

template <int DH, int G, typename KV>
int launch_dh_g(const DecodeArgs& args, int B, int split, hipStream_t stream) {
  // G = 4 keeps 4 q heads of state per lane: only 256-key splits fit 2 waves/SIMD unspilled.
  if constexpr (G == 4) {
    return launch_split<DH, G, 256, KV>(args, B, stream);
  } else {
    if (split == 128) return launch_split<DH, G, 128, KV>(args, B, stream);
    return launch_split<DH, G, 256, KV>(args, B, stream);
  }
}

template <typename KV>
int launch_kv(const DecodeArgs& args, int B, int Dh, int G, int split, hipStream_t stream) {
  if (Dh == 128) {
    if (G == 1) return launch_dh_g<128, 1, KV>(args, B, split, stream);
    if (G == 2) return launch_dh_g<128, 2, KV>(args, B, split, stream);
    return launch_dh_g<128, 4, KV>(args, B, split, stream);
  }
  if (G == 1) return launch_dh_g<64, 1, KV>(args, B, split, stream);
  if (G == 2) return launch_dh_g<64, 2, KV>(args, B, split, stream);
  return launch_dh_g<64, 4, KV>(args, B, split, stream);
}

template <int DH, int G>
int launch_wide(const DecodeArgs& args, int B, int split_len, hipStream_t stream) {
  const dim3 grid(args.Hkv, B, args.max_splits);
  hipEvent_t ev0, ev_split, ev1;
  take_timing_events(&ev0, &ev_split, &ev1);
  if (ev0) (void)hipEventRecord(ev0, stream);
  if (args.arrive)
    hipLaunchKernelGGL((gqa_decode_wide_kernel<DH, G, true>), grid, dim3(64 * kWideWaves), 0,
                       stream, args, split_len);
  else
    hipLaunchKernelGGL((gqa_decode_wide_kernel<DH, G, false>), grid, dim3(64 * kWideWaves), 0,
                       stream, args, split_len);
  int rc = check_launch("gqa_decode_wide_kernel");
  if (ev_split) (void)hipEventRecord(ev_split, stream);
  if (!rc && args.max_splits > 1 && !args.arrive) {
    hipLaunchKernelGGL((gqa_decode_combine_kernel<DH>), dim3(args.Hkv * G, B), dim3(DH), 0,
                       stream, args, split_len, args.Hkv * G);
    rc = check_launch("gqa_decode_combine_kernel");
  }
  if (ev1) (void)hipEventRecord(ev1, stream);
  return rc;
}

}  // namespace

// In-launch split merge: at most this many split workgroups (larger grids run the combine
// kernel, which measured faster there), and the counters a launch may use (B * Hkv).
constexpr long kFuseMaxWorkgroups = 2048;
static_assert(kFuseMaxWorkgroups <= kArriveCounters, "a fused launch has B * Hkv <= its splits");

// Split length: 128 keys (one 32-key chunk per wave, 117 VGPRs, 4 waves/SIMD), measured
// ahead of 256 (2 waves/SIMD) on every configs[2] case: B = 16 at 1K/2K/4K keys by 4-5%, a
// single stream by 6-23%.  G = 4 keeps 4 heads of state per lane and runs 256-key splits.
int choose_split(int /*B*/, int /*Hkv*/, int G, int /*capacity*/) {
  if (G == 4) return 256;  // the only G = 4 instantiation (launch_dh_g)
  return 128;
}

size_t decode_workspace_bytes(int B, int Hq, int Dh, int capacity) {
  const int split = 128;  // the shortest split choose_split() returns
  const size_t max_splits = (static_cast<size_t>(capacity) + split - 1) / split;
  return static_cast<size_t>(B) * Hq * max_splits * (Dh + 2) * sizeof(float);
}

int zeroed_counters(hipStream_t stream, int slot, unsigned** out) {
  bool fresh = false;
  *out = static_cast<unsigned*>(
      workspace(stream, static_cast<size_t>(kArriveCounters) * kCounterStride * sizeof(unsigned),
                slot, &fresh));
  if (!*out) return ORATOR_ERR_HIP;
  if (fresh) {
    hipLaunchKernelGGL(zero_u32_kernel, dim3(kArriveCounters * kCounterStride / 256), dim3(256), 0,
                       stream, *out);
    return check_launch("zero_u32_kernel");
  }
  return ORATOR_OK;
}

// The stream's arrival counters (kArriveCounters, a fixed-size block of its own so it never
// grows); each fused launch's last workgroups return the counters they used to zero.
static int arrival_counters(hipStream_t stream, unsigned** out) {
  return zeroed_counters(stream, kWsArrive, out);
}

int decode_workspace_reserve(int B, int Hq, int Dh, int capacity, hipStream_t stream) {
  if (!workspace(stream, decode_workspace_bytes(B, Hq, Dh, capacity))) return ORATOR_ERR_HIP;
  unsigned* unused = nullptr;
  return arrival_counters(stream, &unused);
}

int launch_gqa_decode(const DecodeProblem& p, hipStream_t stream) {
  if (p.B <= 0 || p.Hq <= 0 || p.Hkv <= 0 || p.Dh <= 0) return ORATOR_OK;  // reference no-op
  if (!p.q || !p.kpool || !p.vpool || (!p.pos && p.pos_mode == 0) || !p.out ||
      (p.pos_mode == 3 && (!p.seg_start || !p.seg_end)))
    return fail(ORATOR_ERR_INVALID, "gqa_decode: null pointer");
  if (p.Hq % p.Hkv) return fail(ORATOR_ERR_INVALID, "gqa_decode: Hq must be a multiple of Hkv");
  if (p.B > 65535) return fail(ORATOR_ERR_UNSUPPORTED, "gqa_decode: at most 65535 streams / rows");
  const int G = p.Hq / p.Hkv;
  // head sizes and groups the split-K kernels are not built for run on the generic kernel
  const bool generic = !(p.Dh == 64 || p.Dh == 128) || !(G == 1 || G == 2 || G == 4);
  if (generic && p.Dh > 1024)
    return fail(ORATOR_ERR_UNSUPPORTED, "gqa_decode: head size above 1024");
  if (p.capacity <= 0) return fail(ORATOR_ERR_INVALID, "gqa_decode: capacity must be > 0");
  if (p.k_new) {
    if (!p.v_new || p.kv_f32 || p.pos_mode != 0)
      return fail(ORATOR_ERR_INVALID, "gqa_decode: append needs k and v rows, bf16 caches");
    if ((reinterpret_cast<uintptr_t>(p.k_new) | reinterpret_cast<uintptr_t>(p.v_new)) & 15u)
      return fail(ORATOR_ERR_INVALID, "gqa_decode: appended k/v rows must be 16-byte aligned");
  }
  if (p.q_norm && (!p.k_norm || !p.rope || !p.k_new || p.Dh != 128 || p.kv_f32))
    return fail(ORATOR_ERR_INVALID,
                "gqa_decode: QK-norm folding needs k_norm, the RoPE table, an appended row, Dh 128");
  if (p.q_norm && generic)
    return fail(ORATOR_ERR_UNSUPPORTED, "gqa_decode: QK-norm folding needs Hq/Hkv in {1,2,4}");
  int page_shift = 0;
  if (p.page_table) {
    page_shift = ilog2_exact(p.page_size);
    if (page_shift < 4 || p.max_pages <= 0)
      return fail(ORATOR_ERR_INVALID, "gqa_decode: page_size must be a power of two >= 16");
    if (static_cast<long>(p.max_pages) * p.page_size < p.capacity)
      return fail(ORATOR_ERR_CAPACITY, "gqa_decode: capacity exceeds max_pages*page_size");
  }
  if (generic) return launch_decode_generic(p, page_shift, stream);
  // Many streams: the wide kernel (a few long ranges per (stream, kv head), one workgroup
  // each, enough ranges to give every CU a workgroup); otherwise 128-key splits.
  const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
  const long pairs = static_cast<long>(p.B) * p.Hkv;
  const int wide_parts = static_cast<int>(std::max<long>(
      (cus + pairs - 1) / pairs, (p.capacity + kWideMaxChunks * 256 - 1) / (kWideMaxChunks * 256)));
  // Ranges of a multiple of 256 keys (8 chunks: the same count for every wave), the last
  // range taking the remainder up to the capacity.  B = 16, S = 4097..4105, capacity 4160:
  // 2048 + 2112 keys, every wave 8 full chunks plus at most the short tail chunk, where
  // 2080-key ranges gave one wave of each first range a ninth full chunk.
  const int wide_len = p.capacity / wide_parts / 256 * 256;
  const int wide_last = p.capacity - (wide_parts - 1) * wide_len;
  // Ranges of >= 1536 keys (>= 6 chunks per wave): at B = 16 the wide kernel measured 50.5-51.6
  // us per op against 52.9 at 4096 keys, but 19.7 / 29.7 against 18.3 / 29.2 us at 1024 / 2048
  // (2 / 4 chunks per wave: its ramp and tail are not amortised).
  const bool wide = !p.kv_f32 && p.pos_mode == 0 && !p.q_norm && G <= 2 && wide_len >= 1536 &&
                    wide_last <= kWideMaxChunks * 256;
  const int split = wide ? wide_len : choose_split(p.B, p.Hkv, G, p.capacity);
  const int max_splits = wide ? wide_parts : (p.capacity + split - 1) / split;
  if (max_splits > 1024) return fail(ORATOR_ERR_CAPACITY, "gqa_decode: more than 1024 splits");
  const size_t part_o = static_cast<size_t>(p.B) * p.Hq * max_splits * p.Dh * sizeof(float);
  const size_t part_ml = static_cast<size_t>(p.B) * p.Hq * max_splits * 2 * sizeof(float);
  // Small split grids and the wide kernel merge their partials inside the launch (the last
  // workgroup of each (stream, kv head) to finish): one launch instead of two, which is most
  // of a single stream's time and 1.8 us of the wide op's 50.7 (B = 16, L = 4096, same box).
  const long split_wgs = pairs * max_splits;
  const bool fuse = !p.kv_f32 && max_splits > 1 &&
                    (wide ? pairs <= kArriveCounters : split_wgs <= kFuseMaxWorkgroups);
  unsigned* arrive = nullptr;
  if (fuse) {
    if (p.scratch) {
      arrive = p.arrive;  // the caller's counters (kArriveCounters, zero between launches)
    } else {
      // a fixed-size block, zeroed when it is allocated; each launch's last workgroups
      // return the counters they used to zero
      if (int rc = arrival_counters(stream, &arrive)) return rc;
    }
  }
  char* ws = nullptr;
  if (p.scratch) {
    if (part_o + part_ml > p.scratch_bytes)
      return fail(ORATOR_ERR_CAPACITY,
                  "gqa_decode: split partials (" + std::to_string(part_o + part_ml) +
                      " bytes) exceed the static scratch (" + std::to_string(p.scratch_bytes) +
                      " bytes)");
    ws = static_cast<char*>(p.scratch);
  } else {
    ws = static_cast<char*>(workspace(stream, part_o + part_ml));
    if (!ws) return ORATOR_ERR_HIP;
  }

  DecodeArgs args;
  args.pos_mode = p.pos_mode;
  args.seg_start = p.seg_start;
  args.seg_end = p.seg_end;
  args.q = p.q;
  args.kpool = p.kpool;
  args.vpool = p.vpool;
  args.page_table = p.page_table;
  args.pos = p.pos;
  args.out = p.out;
  args.part_o = reinterpret_cast<float*>(ws);
  args.part_ml = reinterpret_cast<float*>(ws + part_o);
  args.arrive = arrive;
  args.stream_stride = p.stream_stride;
  args.max_pages = p.max_pages;
  args.page_shift = page_shift;
  args.Hkv = p.Hkv;
  args.max_splits = max_splits;
  args.capacity = p.capacity;
  args.scale_log2e = p.scale * 1.4426950408889634f;
  args.k_new = p.k_new;
  args.v_new = p.v_new;
  args.pool_rows = p.pool_rows;
  args.q_norm = p.q_norm;
  args.k_norm = p.k_norm;
  args.rope = p.rope;
  args.eps = p.eps;

  if (wide) {
    if (p.Dh == 128)
      return G == 1 ? launch_wide<128, 1>(args, p.B, split, stream)
                    : launch_wide<128, 2>(args, p.B, split, stream);
    return G == 1 ? launch_wide<64, 1>(args, p.B, split, stream)
                  : launch_wide<64, 2>(args, p.B, split, stream);
  }
  if (p.kv_f32) return launch_kv<float>(args, p.B, p.Dh, G, split, stream);
  return launch_kv<uint16_t>(args, p.B, p.Dh, G, split, stream);
}

// ---- allocation-free decode: split partials in a static device array ----
// Each GPU holds its own copy of `scratch` from load until the process ends.  Host code
// never passes the array's name to a kernel (on the host it is only a stand-in for the
// symbol): the device address comes from hipGetSymbolAddress, once per device, with that
// device current.
// Layout: split partials, then kArriveCounters arrival counters of the in-launch split merge.
// The counters start at zero (static storage is zero-initialized) and every launch that uses
// them leaves them at zero.
constexpr size_t kStaticScratchBytes = size_t{16} << 20;
constexpr size_t kStaticPartialBytes =
    kStaticScratchBytes - size_t{kArriveCounters} * kCounterStride * sizeof(unsigned);
static __device__ __align__(256) float scratch[kStaticScratchBytes / sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// This device's address of `scratch` (looked up on the first call on the device).
int static_scratch(void** out) {
  *out = nullptr;
  int dev = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev < 0 || dev >= kMaxDevices)
    return fail(ORATOR_ERR_UNSUPPORTED, "static scratch: device index past 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (int rc = check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)),
                           "hipGetSymbolAddress(scratch)"))
      return rc;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return ORATOR_OK;
}
}  // namespace

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

// WriteKvCacheKernel + GqaDecodeAttnKernel of one decode step (asr_text_decoder.cu:412-418)
// in one launch: the new token's K/V rows are written at pos and attended as the last key.
int orator_gqa_decode_append(const float* q, const float* k_new, const float* v_new,
                             uint16_t* kc, uint16_t* vc, float* out, int Hq, int Hkv, int Dh,
                             const int* d_pos, int capacity, float scale, void* stream) {
  if (Hq > 0 && (!k_new || !v_new)) return fail(ORATOR_ERR_INVALID, "gqa_decode_append: null k/v");
  DecodeProblem p{};
  p.q = q;
  p.kpool = kc;
  p.vpool = vc;
  p.pos = d_pos;
  p.out = out;
  p.B = 1;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.Dh = Dh;
  p.capacity = capacity;
  p.scale = scale;
  p.k_new = k_new;
  p.v_new = v_new;
  p.pool_rows = capacity;
  return launch_gqa_decode(p, static_cast<hipStream_t>(stream));
}

int orator_gqa_decode_append_paged(const float* q, const float* k_new, const float* v_new,
                                   uint16_t* kpool, uint16_t* vpool, const int* page_table,
                                   int max_pages, int page_size, int n_pages, const int* d_pos,
                                   float* out, int B, int Hq, int Hkv, int Dh, float scale,
                                   void* stream) {
  if (B > 0 && (!page_table || !k_new || !v_new))
    return fail(ORATOR_ERR_INVALID, "gqa_decode_append_paged: null page table or k/v");
  if (B > 0 && n_pages <= 0)
    return fail(ORATOR_ERR_INVALID, "gqa_decode_append_paged: n_pages must be > 0");
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
  p.k_new = k_new;
  p.v_new = v_new;
  p.pool_rows = static_cast<long>(n_pages) * page_size;
  return launch_gqa_decode(p, static_cast<hipStream_t>(stream));
}

// The whole attention half of a decode step (asr_text_decoder.cu:408-418: RmsNorm q and k,
// RopeHalf q and k, WriteKvCacheKernel, GqaDecodeAttnKernel) in one launch: q and k_new are
// the raw projections; the per-head RMSNorm and the RoPE of position pos[b] (a table of
// orator_rope_table holding `rope_rows` >= capacity positions) are applied before attending.
static int decode_append_qknorm(const float* q, const float* k_new, const float* v_new,
                                uint16_t* kpool, uint16_t* vpool, const int* page_table,
                                int max_pages, int page_size, long pool_rows, int capacity,
                                const int* d_pos, float* out, int B, int Hq, int Hkv, int Dh,
                                float scale, const float* q_norm, const float* k_norm, float eps,
                                const float* rope, int rope_rows, hipStream_t stream) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Dh <= 0) return ORATOR_OK;
  if (!k_new || !v_new || !q_norm || !k_norm || !rope)
    return fail(ORATOR_ERR_INVALID, "gqa_decode_append_qknorm: null k/v, norm or RoPE table");
  if (Dh != 128) return fail(ORATOR_ERR_UNSUPPORTED, "gqa_decode_append_qknorm: Dh must be 128");
  if (rope_rows < capacity)
    return fail(ORATOR_ERR_INVALID, "gqa_decode_append_qknorm: RoPE table shorter than capacity");
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
  p.capacity = capacity;
  p.scale = scale;
  p.k_new = k_new;
  p.v_new = v_new;
  p.pool_rows = pool_rows;
  p.q_norm = q_norm;
  p.k_norm = k_norm;
  p.rope = rope;
  p.eps = eps;
  return launch_gqa_decode(p, stream);
}

int orator_gqa_decode_append_qknorm(const float* q, const float* k_new, const float* v_new,
                                    uint16_t* kc, uint16_t* vc, float* out, int Hq, int Hkv,
                                    int Dh, const int* d_pos, int capacity, float scale,
                                    const float* q_norm, const float* k_norm, float eps,
                                    const float* rope, int rope_rows, void* stream) {
  return decode_append_qknorm(q, k_new, v_new, kc, vc, nullptr, 0, 0, capacity, capacity, d_pos,
                              out, 1, Hq, Hkv, Dh, scale, q_norm, k_norm, eps, rope, rope_rows,
                              static_cast<hipStream_t>(stream));
}

int orator_gqa_decode_append_qknorm_paged(const float* q, const float* k_new, const float* v_new,
                                          uint16_t* kpool, uint16_t* vpool, const int* page_table,
                                          int max_pages, int page_size, int n_pages,
                                          const int* d_pos, float* out, int B, int Hq, int Hkv,
                                          int Dh, float scale, const float* q_norm,
                                          const float* k_norm, float eps, const float* rope,
                                          int rope_rows, void* stream) {
  if (B > 0 && (!page_table || n_pages <= 0))
    return fail(ORATOR_ERR_INVALID, "gqa_decode_append_qknorm_paged: page table / n_pages");
  return decode_append_qknorm(q, k_new, v_new, kpool, vpool, page_table, max_pages, page_size,
                              static_cast<long>(n_pages) * page_size, max_pages * page_size,
                              d_pos, out, B, Hq, Hkv, Dh, scale, q_norm, k_norm, eps, rope,
                              rope_rows, static_cast<hipStream_t>(stream));
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

// orator_gqa_decode_paged with the split partials in this file's static device scratch
// (16 MiB per GPU): no allocation of any kind, so callers that cannot allocate (graph
// capture, serving loops that forbid hipMalloc) can use it.  Calls that overlap on one GPU
// share the scratch and race.  Nothing in it needs clearing: every partial is written before
// it is read.
int orator_gqa_decode_paged_noalloc(const float* q, const uint16_t* kpool, const uint16_t* vpool,
                                    const int* page_table, int max_pages, int page_size,
                                    const int* d_pos, float* out, int B, int Hq, int Hkv, int Dh,
                                    float scale, void* stream) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Dh <= 0) return ORATOR_OK;  // reference no-op
  if (!page_table) return fail(ORATOR_ERR_INVALID, "gqa_decode_paged_noalloc: null page table");
  // reject sizes past the scratch before touching the device
  const size_t need = decode_workspace_bytes(B, Hq, Dh, max_pages * page_size);
  if (max_pages > 0 && page_size > 0 && need > kStaticPartialBytes)
    return fail(ORATOR_ERR_CAPACITY,
                "gqa_decode_paged_noalloc: B * Hq * splits * (Dh + 2) * 4 = " +
                    std::to_string(need) + " bytes exceeds the " +
                    std::to_string(kStaticPartialBytes) +
                    " bytes of the 16 MiB static scratch held for split partials");
  void* ptr = nullptr;
  if (int rc = static_scratch(&ptr)) return rc;
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
  p.scratch = ptr;
  p.scratch_bytes = kStaticPartialBytes;
  p.arrive = reinterpret_cast<unsigned*>(static_cast<char*>(ptr) + kStaticPartialBytes);
  return launch_gqa_decode(p, static_cast<hipStream_t>(stream));
}

// asr_ops::GqaAttention (include/model/asr_ops.cuh:50-56; src/model/asr_ops.cu:252-295):
// fp32 self-attention = decode of T query rows over one shared fp32 K/V, row i attending
// keys [0, i] (causal) or [0, T).  Default stream, as the reference.
int orator_gqa_attention(const float* q, const float* k, const float* v, float* out, int T, int Hq,
                         int Hkv, int Dh, float scale, int causal) {
  if (T <= 0 || Hq <= 0 || Hkv <= 0 || Dh <= 0) return ORATOR_OK;  // reference no-op
  if (!q || !k || !v || !out) return fail(ORATOR_ERR_INVALID, "gqa_attention: null pointer");
  if (Hq % Hkv) return fail(ORATOR_ERR_INVALID, "gqa_attention: Hq must be a multiple of Hkv");
  if (Dh > 1024 || (Dh & (Dh - 1)))
    return fail(ORATOR_ERR_UNSUPPORTED, "gqa_attention: Dh must be a power of two <= 1024");
  const int G = Hq / Hkv;
  if (!((Dh == 64 || Dh == 128) && (G == 1 || G == 2 || G == 4) && T <= 65535))
    return launch_gqa_attention_generic(q, k, v, out, T, Hq, Hkv, Dh, scale, causal != 0,
                                        nullptr);
  DecodeProblem p{};
  p.q = q;
  p.kpool = k;
  p.vpool = v;
  p.kv_f32 = true;
  p.pos_mode = causal ? 1 : 2;
  p.out = out;
  p.B = T;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.Dh = Dh;
  p.capacity = T;
  p.scale = scale;
  return launch_gqa_decode(p, nullptr);
}

// Measurement hook (no reference counterpart): the streaming-read ceiling of the paged decode
// access pattern, S keys per stream (head_dim 128, bf16, every page of the first ceil(S /
// page_size) table entries mapped).  `sink` is a 4-byte device word the kernel may write.
int orator_decode_read_probe(const uint16_t* kpool, const uint16_t* vpool, const int* page_table,
                             int max_pages, int page_size, int S, int B, int Hkv,
                             unsigned* sink, void* stream) {
  if (S <= 0 || B <= 0 || Hkv <= 0) return ORATOR_OK;
  if (!kpool || !vpool || !page_table || !sink)
    return fail(ORATOR_ERR_INVALID, "decode_read_probe: null pointer");
  const int shift = ilog2_exact(page_size);
  if (shift < 4) return fail(ORATOR_ERR_INVALID, "decode_read_probe: page_size must be 2^k >= 16");
  if (static_cast<long>(max_pages) * page_size < S)
    return fail(ORATOR_ERR_CAPACITY, "decode_read_probe: S exceeds max_pages * page_size");
  if (B > 65535) return fail(ORATOR_ERR_UNSUPPORTED, "decode_read_probe: at most 65535 streams");
  const dim3 grid(Hkv, B, (S + 127) / 128);
  hipLaunchKernelGGL(decode_read_probe_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     kpool, vpool, page_table, max_pages, shift, S, Hkv, sink);
  return check_launch("decode_read_probe_kernel");
}

// WindowAttnKernel (src/model/asr_audio_tower.cu:204-258): audio-tower self-attention, q/k/v
// fp32 [N, H, Dh], query i attends keys [seg_start[i], seg_end[i]) (device arrays), online
// softmax, 0 for an empty window.  Ranges are clamped into [0, N).
int orator_window_attention(const float* q, const float* k, const float* v, float* out,
                            const int* d_seg_start, const int* d_seg_end, int N, int H, int Dh,
                            float scale, void* stream) {
  // 64-wide heads (the audio tower's): a workgroup per 32-query block and head over the
  // union of the block's windows, on fp32 MFMA (range_attn.hip); 128-wide heads: every query
  // as a stream of the split decode kernel below
  if (Dh == 64 && N > 0 && H > 0) {
    if (!q || !k || !v || !out || !d_seg_start || !d_seg_end)
      return fail(ORATOR_ERR_INVALID, "window_attention: null pointer");
    return launch_range_attention(q, k, v, out, d_seg_start, d_seg_end, N, H, Dh, 0, scale,
                                  static_cast<hipStream_t>(stream));
  }
  DecodeProblem p{};
  p.q = q;
  p.kpool = k;
  p.vpool = v;
  p.kv_f32 = true;
  p.pos_mode = 3;
  p.seg_start = d_seg_start;
  p.seg_end = d_seg_end;
  p.out = out;
  p.B = N;
  p.Hq = H;
  p.Hkv = H;
  p.Dh = Dh;
  p.capacity = N;
  p.scale = scale;
  return launch_gqa_decode(p, static_cast<hipStream_t>(stream));
}

}  // extern "C"
