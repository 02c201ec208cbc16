// Causal GQA prefill attention over a bf16 KV cache on MFMA (gfx950).
//
// Replaces GqaCacheAttnKernel (src/model/asr_text_decoder.cu:88-142): query row t (absolute
// position pos0 + t) attends keys [0, pos0 + t] of the cache; online softmax; out = acc/l,
// or 0 when l == 0.  K/V are bf16 in the cache, accumulation is fp32.
//
// Two precisions share the kernel:
//  * bf16 mode: q (and the softmax weights fed to the PV product) rounded to bf16 -- one
//    v_mfma_f32_32x32x16_bf16 per product;
//  * fp32 mode: q and the softmax weights each carried as three bf16 terms (hi + mid + lo,
//    exact to fp32 rounding for q, ~2^-26 relative for the weights); K/V are exact in bf16,
//    so QK and PV are fp32-accurate, at 3x the MFMA work.  (Two weight terms, ~2^-17, put
//    near-zero outputs of long rows at the edge of a 1e-4 relative bound.)
//
// Work split.  A workgroup is 8 wave64s: RW query-row waves (32 query columns each) times
// KG = 8/RW key groups.  Key group g takes the 32-key tiles g, g+KG, g+2KG, ... of the
// block's causal key range with its own LDS tiles; the KG partial softmax states are merged
// through LDS at the end.  Two waves per SIMD (<= 256 VGPRs each) let one wave's softmax
// VALU run under the other's MFMAs.  The launcher picks
//  * RW = 4, KG = 2 (128 query rows share every K/V tile) when that still gives every CU
//    two workgroups: a CU then pulls 32 B/clk of K/V at full MFMA rate, half of what its
//    vector memory path sustains, and registers hold a prefetch two rounds ahead;
//  * RW = 2, KG = 4 (64 rows per tile, 64 B/clk at full rate) when RW = 4 would not;
//  * RW = 1, KG = 8 when even RW = 2 leaves CUs without a workgroup (T = 503 on 8 kv heads:
//    256 workgroups instead of 128, at most two tiles per wave).  Such prompts are a chain of
//    latencies, not a throughput problem: every wave is its own key group with a single
//    buffer (no barrier per round), the loads of its first two tiles go out before the pos0
//    read, and the workgroup's q is read once, row-contiguous, and staged in LDS (a lane per
//    query row re-read by all 8 groups touched 64 cache lines per load instruction).
//
// Per tile and wave:
//  * S^T = K Q^T: K tile rows are the MFMA A operand (ds_read_b128 from a padded,
//    conflict-free LDS layout), the wave's 32 query columns stay in registers as B.  In the
//    32x32 accumulator layout every lane owns ONE query column and 16 keys, so the row
//    max / sum of the online softmax are in-lane plus one exchange between lane halves.
//  * S^T of the next tile is issued interleaved with the softmax of the current one, so the
//    MFMAs of one overlap the VALU of the other inside a wave too.
//  * the running max is a stale reference: it is only moved (and O, l rescaled) when a new
//    score exceeds it by more than 2^8, so weights stay <= 256 and most tiles skip the
//    64-register rescale.  Softmax is invariant to the reference, so this is exact.
//  * O^T += V^T P^T: P^T comes straight from the S^T accumulators (no LDS round trip);
//    V stays row-major in LDS and the V^T operand is read with ds_read_b64_tr_b16 (a
//    transposing LDS read), so no VALU work transposes V; 288-byte rows keep both the
//    16-byte stores and the transposing reads conflict-free.
//  * K/V tiles travel HBM/L2 -> registers -> LDS; the register copy is loaded one or two
//    rounds before its LDS store, and barriers wait for LDS traffic only, never for these
//    loads.
//  * workgroups are ordered heaviest (latest tokens, most keys) first, and the kv head is
//    the fastest-varying index, so each kv head's workgroups share an XCD (blockIdx % 8).
//    With at least two token blocks per CU, workgroup i runs block n-1-i and then block i
//    (equal key counts per workgroup, one workgroup per CU).
//  * a contiguous cache's tile rows are plain arithmetic: the loads of a round never wait
//    on an LDS page-row lookup (which would also drain that round's LDS stores).  Paged
//    caches look the rows up in LDS.
//
// Measured alternative, not kept: feeding the tiles by LDS DMA (global_load_lds_dwordx4
// into swizzled 3-stage rings, no staging registers) was 7-20% slower at 503-4096 tokens.
#include <cstdlib>

#include "common.hpp"
#include "internal.hpp"
#include "mfma_tile.hpp"

namespace orator_hip {
namespace {

constexpr int kDh = 128;
constexpr int kBN = 32;                              // keys per tile
constexpr int kThreads = 512;                        // 8 wave64s per workgroup
constexpr int kKRow = kDh + 8;                       // padded K row (bf16 elements): 272 B
constexpr int kVRow = kDh + 16;                      // padded V row (bf16 elements): 288 B
constexpr int kMaxRowGroups = 1024;                  // page-row table: up to 16384 keys
constexpr int kSkMinTokens = 2048;                   // stream-K kernel from this prompt length
constexpr float kStaleMax = 8.0f;                    // log2 slack of the reference max

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
  int paired;             // 1: workgroup i runs token blocks n_tblocks-1-i, then i
  float scale_log2e;      // > 0
};

// One key group's LDS: NB buffers of K and V rows (double-buffered for groups of several
// waves, single for the one-wave groups of the short-prompt form).
template <int NB>
struct GroupTiles {
  uint16_t k[NB][kBN][kKRow];
  uint16_t v[NB][kBN][kVRow];
};

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


template <int G, bool PRECISE, int RW>
__global__ __launch_bounds__(kThreads) void gqa_prefill_kernel(PrefillArgs a) {
  constexpr int KG = 8 / RW;                   // key groups
  constexpr int TW = 32 / G;                   // tokens per wave (32 columns = TW tokens x G heads)
  constexpr int BT = RW * TW;                  // tokens per workgroup
  constexpr int GT = 64 * RW;                  // threads per key group
  constexpr int NP = kBN * 16 / GT;            // 16-byte chunks per thread per K (or V) tile
  constexpr int RPP = GT / 16;                 // tile rows covered by one pass of the group
  constexpr int DIST = (!PRECISE && RW == 4) ? 2 : 1;  // register prefetch distance (rounds)
  constexpr int NB = RW == 1 ? 1 : 2;          // tile buffers per key group
  constexpr int CS = 64 / KG;                  // accumulator values per lane each wave finalizes
  using Tiles = GroupTiles<NB>;
  // q staged once per workgroup through LDS (measured: a gain for the one-wave key groups and
  // fp32 mode's three terms at RW = 2, a small loss for bf16 at RW = 2)
  constexpr bool kStageQ = RW == 1 || (RW == 2 && PRECISE);
  static_assert(!kStageQ || (PRECISE ? 3 : 1) * RW * 32 * kKRow * 2 <= KG * (int)sizeof(Tiles),
                "q staging area fits in the tile buffers");
  static_assert(KG * RW == 8 && NP * RPP == kBN, "tile split");
  static_assert(8 * (KG - 1) * CS * 64 * 4 + 8 * 2 * 64 * 4 <= KG * (int)sizeof(Tiles),
                "merge area reuses the tile buffers");
  __shared__ __align__(16) unsigned char smem[KG * sizeof(Tiles)];
  __shared__ int row_lds[kMaxRowGroups];

  const int kvh = blockIdx.x % a.Hkv;
  const int wi = static_cast<int>(blockIdx.x / a.Hkv);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = __builtin_amdgcn_readfirstlane(wave / RW);  // key group (wave-uniform)
  const int rw = wave % RW;                                   // query-row wave of the group
  const int gt = tid % GT;                                    // thread index within the group
  const int h2 = lane >> 5;   // which half of the 32x32 accumulator rows this lane holds
  const int col = lane & 31;  // this lane's query column
  Tiles& tl = reinterpret_cast<Tiles*>(smem)[grp];
  const bool contiguous = a.page_table == nullptr;  // row of key k is k

  // ---- tile loader (group-local tile j = key tile grp + KG*j) ----
  // K and V rows ld_row + RPP*p (p < NP), one 16-byte chunk (dims 8*ld_chunk..) per thread;
  // with the padded rows the LDS stores are conflict-free.
  const long rs = static_cast<long>(a.Hkv) * kDh;  // elements between consecutive rows
  const uint16_t* kbase = a.kpool + static_cast<long>(kvh) * kDh;
  const uint16_t* vbase = a.vpool + static_cast<long>(kvh) * kDh;
  const int ld_row = gt >> 4, ld_chunk = gt & 15;
  const uint32_t lane_off = static_cast<uint32_t>((ld_row * rs + 8 * ld_chunk) * 2);  // bytes
  const long rs2 = rs * 2;

  // One-wave key groups over a contiguous cache issue the loads of their first two tiles
  // before the pos0 read, for the tiles a block needs whatever pos0 is (keys below
  // min(t_end, capacity)); rows are clamped to the capacity, and keys past the range a block
  // needs are masked (scores) or zeroed (V) as always.  fp32 mode leaves V(1) for later
  // (register budget).
  u32x4_t kr[NP], vr[NP], kn[NP], vn[NP];
  bool early0 = false, early1 = false;
  if constexpr (RW == 1) {
    if (contiguous) {
      const int tb = a.n_tblocks - 1 - wi;  // RW = 1 grids are never paired
      const int lb = min(min((tb + 1) * BT, a.Tq), a.capacity);
      auto early_rows = [&](const uint16_t* base, int k0, u32x4_t (&r)[NP]) {
#pragma unroll
        for (int p = 0; p < NP; ++p)
          r[p] = *reinterpret_cast<const u32x4_t*>(
              base + static_cast<long>(min(k0 + RPP * p + ld_row, a.capacity - 1)) * rs +
              8 * ld_chunk);
      };
      early0 = kBN * grp < lb;
      early1 = kBN * (grp + KG) < lb;
      if (early0) {
        early_rows(kbase, kBN * grp, kr);
        early_rows(vbase, kBN * grp, vr);
      }
      if (early1) {
        early_rows(kbase, kBN * (grp + KG), kn);
        if (!PRECISE) early_rows(vbase, kBN * (grp + KG), vn);
      }
    }
  }
  asm volatile("" ::: "memory");  // the loads above are issued before the pos0 read
  const int pos0 = *a.pos0p;

  // One token block: keys, tiles, softmax state, output.  Returns after its output is
  // stored; every thread runs every barrier of it.
  auto run_block = [&](int tblock) {
  const int t_blk = tblock * BT;
  const int t_end = min(t_blk + BT, a.Tq);
  const int n_keys = min(pos0 + t_end, a.capacity);  // keys [0, n_keys) are needed
  const int n_tiles = (n_keys + kBN - 1) / kBN;
  const int n_rounds = (n_tiles + KG - 1) / KG;
  const int my_tiles = n_tiles > grp ? (n_tiles - grp + KG - 1) / KG : 0;
  // tiles with a key beyond this need the causal / capacity mask
  const int mask_from = min(pos0 + t_blk, n_keys - 1);

  // ---- page rows of the needed keys (16-key groups; paged caches only) ----
  const int n_rowgroups = contiguous ? 0 : (n_keys + 15) >> 4;
  for (int gi = tid; gi < n_rowgroups; gi += kThreads) {
    int row = gi << 4;
    if (a.page_table) {
      const int j0 = gi << 4;
      const int page = a.page_table[j0 >> a.page_shift];
      row = (page << a.page_shift) | (j0 & ((1 << a.page_shift) - 1));
    }
    row_lds[gi] = row;
  }

  // ---- this wave's query columns: token tq, head hq ----
  const int tq = t_blk + rw * TW + (col % TW);
  const int hq = kvh * G + col / TW;
  const bool q_valid = tq < a.Tq;
  const int q_lim = min(pos0 + tq, n_keys - 1);  // last key this column may attend
  // B operand per 16-dim k-step (dims 16ks + 8*h2 + e).  fp32 mode carries q as three bf16
  // terms hi + mid + lo (exact to fp32 rounding); bf16 mode uses hi only.
  uint4 qhi[8], qmid[8], qlo[8];
  // Splits 8 fp32 q values into the bf16 terms (hi, mid, lo) this mode uses.
  auto q_terms = [&](const float* src, uint4& hi, uint4& mid, uint4& lo) {
    const float4 x0 = *reinterpret_cast<const float4*>(src);
    const float4 x1 = *reinterpret_cast<const float4*>(src + 4);
    float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    split8(xs, hi, mid);
    if (PRECISE) split8(xs, mid, lo);
  };
  if constexpr (kStageQ) {
    // The workgroup's RW*32 query columns are read once, with row-contiguous loads (a lane
    // per 8 dims), and staged in LDS as bf16 terms ([term][column][kKRow]; the K tiles'
    // padded rows, so the B-operand reads below are conflict-free), instead of every key
    // group's waves loading them a row per lane.
    uint16_t* qs = reinterpret_cast<uint16_t*>(smem);
    for (int it = tid; it < RW * 32 * 16; it += kThreads) {
      const int qc = it >> 4, qd = it & 15;  // column, 8-dim chunk
      const int t = t_blk + (qc >> 5) * TW + (qc & 31) % TW;
      const int h = kvh * G + (qc & 31) / TW;
      uint4 hi = make_uint4(0, 0, 0, 0), mid = hi, lo = hi;
      if (t < a.Tq) {
        const long off = (static_cast<long>(t) * a.Hq + h) * kDh + 8 * qd;
        if (a.q)
          q_terms(a.q + off, hi, mid, lo);
        else
          hi = *reinterpret_cast<const uint4*>(a.q_bf16 + off);
      }
      *reinterpret_cast<uint4*>(qs + qc * kKRow + 8 * qd) = hi;
      if (PRECISE) {
        *reinterpret_cast<uint4*>(qs + (RW * 32 + qc) * kKRow + 8 * qd) = mid;
        *reinterpret_cast<uint4*>(qs + (2 * RW * 32 + qc) * kKRow + 8 * qd) = lo;
      }
    }
    lds_barrier();  // staged q and row_lds ready
    const uint16_t* qrow = qs + (rw * 32 + col) * kKRow + 8 * h2;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      qhi[ks] = *reinterpret_cast<const uint4*>(qrow + 16 * ks);
      qmid[ks] = qlo[ks] = make_uint4(0, 0, 0, 0);
      if (PRECISE) {
        qmid[ks] = *reinterpret_cast<const uint4*>(qrow + RW * 32 * kKRow + 16 * ks);
        qlo[ks] = *reinterpret_cast<const uint4*>(qrow + 2 * RW * 32 * kKRow + 16 * ks);
      }
    }
    lds_barrier();  // every wave has its q before the tiles overwrite the staging area
  } else {
    const long qoff = (static_cast<long>(tq) * a.Hq + hq) * kDh + 8 * h2;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      qmid[ks] = qlo[ks] = make_uint4(0, 0, 0, 0);
      if (!q_valid)
        qhi[ks] = make_uint4(0, 0, 0, 0);
      else if (a.q)
        q_terms(a.q + qoff + 16 * ks, qhi[ks], qmid[ks], qlo[ks]);
      else
        qhi[ks] = *reinterpret_cast<const uint4*>(a.q_bf16 + qoff + 16 * ks);
    }
    lds_barrier();  // row_lds ready
  }

  // Row of `key` (clamped to the last needed key, so every load stays in bounds).
  auto row_clamped = [&](int key) -> long {
    key = min(key, n_keys - 1);
    return contiguous ? key : static_cast<long>(row_lds[key >> 4] + (key & 15));
  };
  auto load_rows = [&](const uint16_t* base, int j, u32x4_t (&r)[NP]) {
    const int k0 = (grp + KG * j) * kBN;  // uniform
    if (k0 + kBN <= n_keys) {
      // whole tile valid: two 16-row groups with uniform bases (no LDS lookup, and so no
      // wait on this round's LDS stores, for a contiguous cache)
      const long rg0 = contiguous ? k0 : __builtin_amdgcn_readfirstlane(row_lds[k0 >> 4]);
      const long rg1 =
          contiguous ? k0 + 16 : __builtin_amdgcn_readfirstlane(row_lds[(k0 >> 4) + 1]);
      const char* b0 = reinterpret_cast<const char*>(base + rg0 * rs) + lane_off;
      const char* b1 = reinterpret_cast<const char*>(base + rg1 * rs) + lane_off;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int roff = RPP * p;
        const char* bp = ((roff >> 4) ? b1 : b0) + (roff & 15) * rs2;
        r[p] = *reinterpret_cast<const u32x4_t*>(bp);
      }
    } else {
#pragma unroll
      for (int p = 0; p < NP; ++p)
        r[p] = *reinterpret_cast<const u32x4_t*>(
            base + row_clamped(k0 + RPP * p + ld_row) * rs + 8 * ld_chunk);
    }
  };
  auto load_k = [&](int j, u32x4_t (&r)[NP]) { load_rows(kbase, j, r); };
  auto load_v = [&](int j, u32x4_t (&r)[NP]) { load_rows(vbase, j, r); };
  auto store_k = [&](int buf, const u32x4_t (&r)[NP]) {
#pragma unroll
    for (int p = 0; p < NP; ++p)
      *reinterpret_cast<u32x4_t*>(&tl.k[buf][RPP * p + ld_row][8 * ld_chunk]) = r[p];
  };
  // Keys past the end are stored as zeros in V: their weights are 0, and 0 * inf must not
  // occur.  (Keys past the end in K need nothing: their scores are replaced by the mask.)
  auto store_v = [&](int buf, u32x4_t (&r)[NP], int j) {
    const int k0 = (grp + KG * j) * kBN;
    if (k0 + kBN > n_keys) {  // uniform over the group
#pragma unroll
      for (int p = 0; p < NP; ++p)
        if (k0 + RPP * p + ld_row >= n_keys) r[p] = u32x4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int p = 0; p < NP; ++p)
      *reinterpret_cast<u32x4_t*>(&tl.v[buf][RPP * p + ld_row][8 * ld_chunk]) = r[p];
  };

  // S^T (32 keys x this wave's 32 query columns) of the tile in K buffer `buf`.
  auto qk = [&](int buf) {
    f32x16_t s = {};
    uint4 kf[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      kf[ks] = *reinterpret_cast<const uint4*>(&tl.k[buf][col][16 * ks + 8 * h2]);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const bf16x8_t ka = as_bf16x8(kf[ks]);
      if (PRECISE) {  // small terms first
        s = mfma32(ka, as_bf16x8(qlo[ks]), s);
        s = mfma32(ka, as_bf16x8(qmid[ks]), s);
      }
      s = mfma32(ka, as_bf16x8(qhi[ks]), s);
    }
    return s;
  };

  f32x16_t o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.0f;
  float m = -INFINITY;  // reference max (log2 units), shared by the lane pair col, col+32
  float lsum = 0.0f;    // this lane's 16 keys of each tile
  const float c = a.scale_log2e;

  // Causal / capacity mask of tile j's scores, then the reference max: it is only moved
  // (and O, l rescaled) when some score exceeds it by more than 2^kStaleMax.  Returns the
  // reference to subtract (0 while nothing has been attended: all weights are then 0).
  auto mask_and_rescale = [&](f32x16_t& s, int j) {
    const int k0 = (grp + KG * j) * kBN;
    if (k0 + kBN - 1 > mask_from) {  // uniform over the workgroup
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = k0 + 8 * (e >> 2) + 4 * h2 + (e & 3);
        if (key > q_lim) s[e] = -INFINITY;
      }
    }
    float mx = s[0];
#pragma unroll
    for (int e = 1; e < 16; ++e) mx = fmaxf(mx, s[e]);
    mx = xor32_max(mx) * c;
    if (__builtin_amdgcn_ballot_w64(mx > m + kStaleMax)) {  // move the reference max
      const float mn = fmaxf(m, mx);
      const float corr = m == mn ? 1.0f : fast_exp2(m - mn);
      m = mn;
      lsum *= corr;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] *= corr;
    }
    return m == -INFINITY ? 0.0f : m;
  };

  // A operand of O^T += V^T P^T (V^T: row = dim 32dt + col, k = keys 16st + 4*h2 + 8*(e/4)
  // + e%4) by transposed reads of the row-major V tile: 16-lane group g covers dims
  // 16*(g & 1) .. of the 32-dim block and keys 4*(g >> 1) .. (+8 for the second half).
  const int tg = lane >> 4, ts = lane & 15;
  const int v_lane = (4 * (tg >> 1) + (ts >> 2)) * kVRow + 16 * (tg & 1) + 4 * (ts & 3);
  auto read_vf = [&](int buf, int st, uint4 (&vf)[4]) {
    const uint16_t* vsrc = &tl.v[buf][0][0] + v_lane + (16 * st) * kVRow;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const uint2 v0 = lds_read_tr16(vsrc + 32 * dt);
      const uint2 v1 = lds_read_tr16(vsrc + 8 * kVRow + 32 * dt);
      vf[dt] = make_uint4(v0.x, v0.y, v1.x, v1.y);
    }
  };

  // Softmax of tile j (scores s) and O^T += V^T P^T from V buffer `buf`, one 16-key k-step
  // at a time (register pressure).
  auto softmax_pv = [&](f32x16_t s, int j, int buf) {
    const float mref = mask_and_rescale(s, j);
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = fast_exp2(fmaf(s[8 * st + e], c, -mref));
      uint4 vf[4];
      if constexpr (PRECISE) {
        // B operand per k-step st (keys 16st + 8(e/4) + 4*h2 + e%4), each weight as
        // hi + mid + lo bf16 terms: both remainders are exact in fp32, so the three terms
        // carry the fp32 weight to ~2^-26 relative.
        uint32_t hw[4], mw[4], lw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          hw[e] = cvt_bf16x2(pv[2 * e], pv[2 * e + 1]);
          const float r0 = pv[2 * e] - bf16_lo(hw[e]), r1 = pv[2 * e + 1] - bf16_hi(hw[e]);
          mw[e] = cvt_bf16x2(r0, r1);
          lw[e] = cvt_bf16x2(r0 - bf16_lo(mw[e]), r1 - bf16_hi(mw[e]));
          lsum += pv[2 * e] + pv[2 * e + 1];
        }
        const uint4 phi = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        const uint4 pmid = make_uint4(mw[0], mw[1], mw[2], mw[3]);
        const uint4 plo = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        read_vf(buf, st, vf);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const bf16x8_t va = as_bf16x8(vf[dt]);
          o[dt] = mfma32(va, as_bf16x8(plo), o[dt]);
          o[dt] = mfma32(va, as_bf16x8(pmid), o[dt]);
          o[dt] = mfma32(va, as_bf16x8(phi), o[dt]);
        }
      } else {
        // bf16 weights, and the row sum of those bf16 values (the pipelined rounds' form)
        uint32_t hw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          hw[e] = cvt_bf16x2(pv[2 * e], pv[2 * e + 1]);
          lsum = add_bf16x2(hw[e], lsum);
        }
        const uint4 phi = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        read_vf(buf, st, vf);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[dt] = mfma32(as_bf16x8(vf[dt]), as_bf16x8(phi), o[dt]);
      }
      // one k-step's temporaries at a time (the one-wave key groups keep a tile in flight)
      if constexpr (RW == 1) __builtin_amdgcn_sched_barrier(0);
    }
  };

  if constexpr (RW == 1) {
    // Short prompts: every wave is a key group of its own with a single K and V buffer that
    // no other wave touches, so the rounds need no workgroup barrier.  A wave's LDS
    // instructions execute in issue order, so a tile may be stored over the previous one
    // right after that one's reads; compiler fences keep the order.  A wave loads and
    // computes its own tiles only.
    //  * bf16 mode, round j: S of tile j, store K(j+1); softmax and PV of tile j, store
    //    V(j+1); load tile j+2.  At most two tiles per wave (the prompts this form is chosen
    //    for) are all loaded in the prologue: one memory latency.
    //  * fp32 mode holds three q terms, so only K(j+1) is in flight during S of tile j and no
    //    tile during the softmax and PV; V(j+1) is loaded after them.
    if (my_tiles > 0 && !early0) {
      load_k(0, kr);
      load_v(0, vr);
    }
    if (my_tiles > 1 && !early1) {
      load_k(1, kn);
      if (!PRECISE) load_v(1, vn);
    }
    if (my_tiles > 0) {
      store_k(0, kr);
      store_v(0, vr, 0);
    }
    for (int j = 0; j < my_tiles; ++j) {
      asm volatile("" ::: "memory");
      const f32x16_t sj = qk(0);
      asm volatile("" ::: "memory");
      if constexpr (!PRECISE) {
        if (j + 1 < my_tiles) store_k(0, kn);
        softmax_pv(sj, j, 0);
        asm volatile("" ::: "memory");
        if (j + 1 < my_tiles) store_v(0, vn, j + 1);
        if (j + 2 < my_tiles) {
          load_k(j + 2, kn);
          load_v(j + 2, vn);
        }
      } else {
        if (j + 1 < my_tiles) store_k(0, kn);
        softmax_pv(sj, j, 0);
        asm volatile("" ::: "memory");
        if (j + 1 < my_tiles) {
          load_v(j + 1, vn);
          store_v(0, vn, j + 1);
        }
        if (j + 2 < my_tiles) load_k(j + 2, kn);
      }
    }
    lds_barrier();  // every wave's tiles are consumed before the merge reuses them
  } else if constexpr (!PRECISE) {
    // Register prefetch sets: set (j % DIST) holds K(j+2), V(j+1) at the start of round j.
    u32x4_t kr[DIST][NP], vr[DIST][NP];
    // Phases of one bf16 round, in issue order: LDS stores of the prefetched K(j+2), V(j+1);
    // global loads of K(j+2+DIST), V(j+1+DIST); the K fragments of S(j+1); mask / max /
    // rescale of tile j; the transposed V reads of tile j; S(j+1) MFMAs interleaved with
    // the weights of tile j (exp, bf16 pack, row sum); the PV MFMAs of tile j.
    auto round = [&]<int P>(int j, f32x16_t& s_cur, f32x16_t& s_nxt) {
      constexpr int S = DIST == 2 ? P : 0;
      store_k(P, kr[S]);
      store_v(P ^ 1, vr[S], j + 1);
      load_k(j + 2 + DIST, kr[S]);
      load_v(j + 1 + DIST, vr[S]);
      if (j >= my_tiles) return;  // uniform: this group has no tile j
      uint4 kf[8];
#pragma unroll
      for (int ks = 0; ks < 8; ++ks)
        kf[ks] = *reinterpret_cast<const uint4*>(&tl.k[P ^ 1][col][16 * ks + 8 * h2]);
      const float mref = mask_and_rescale(s_cur, j);
      uint4 vf[2][4];
      read_vf(P, 0, vf[0]);
      read_vf(P, 1, vf[1]);
      f32x16_t sn = {};
      uint32_t hw[8];  // bf16 weights of elements 2i, 2i+1 of s_cur
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        sn = mfma32(as_bf16x8(kf[ks]), as_bf16x8(qhi[ks]), sn);
        const float p0 = fast_exp2(fmaf(s_cur[2 * ks], c, -mref));
        const float p1 = fast_exp2(fmaf(s_cur[2 * ks + 1], c, -mref));
        hw[ks] = cvt_bf16x2(p0, p1);
        lsum = add_bf16x2(hw[ks], lsum);
      }
      s_nxt = sn;
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const uint4 ph = make_uint4(hw[4 * st], hw[4 * st + 1], hw[4 * st + 2], hw[4 * st + 3]);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[dt] = mfma32(as_bf16x8(vf[st][dt]), as_bf16x8(ph), o[dt]);
      }
      // Issue order: each dependent S MFMA followed by ~6 independent weight instructions
      // (which run while the MFMA executes), the V reads in two batches ahead of them, then
      // the PV MFMAs.
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (i % 4 == 0) __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);  // DS reads
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);                  // VALU
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);  // MFMA
    };
    // ---- prologue: K0, V0, K1 into LDS, S(0); the first DIST register sets are loaded in
    // the same burst (one memory round trip before the first round, not two) ----
    {
      u32x4_t k0[NP], v0[NP], k1[NP];
      load_k(0, k0);
      load_v(0, v0);
      load_k(1, k1);
#pragma unroll
      for (int d = 0; d < DIST; ++d) {
        load_k(2 + d, kr[d]);
        load_v(1 + d, vr[d]);
      }
      store_k(0, k0);
      store_v(0, v0, 0);
      store_k(1, k1);
    }
    lds_barrier();
    f32x16_t s0 = qk(0), s1;
    lds_barrier();  // K buffer 0 is refilled in round 0
    int j = 0;
    for (; j + 1 < n_rounds; j += 2) {
      round.template operator()<0>(j, s0, s1);
      lds_barrier();
      round.template operator()<1>(j + 1, s1, s0);
      lds_barrier();
    }
    if (j < n_rounds) {
      round.template operator()<0>(j, s0, s1);
      lds_barrier();
    }
  } else {
    // fp32 mode holds three q terms, so S is not pipelined (register budget of 2 waves/SIMD):
    // round j stores tile j+1, loads tile j+2, and computes S, softmax and PV of tile j.
    u32x4_t kr[NP], vr[NP];
    load_k(0, kr);
    load_v(0, vr);
    store_k(0, kr);
    store_v(0, vr, 0);
    load_k(1, kr);
    load_v(1, vr);
    lds_barrier();
    for (int j = 0; j < n_rounds; ++j) {
      store_k((j + 1) & 1, kr);
      store_v((j + 1) & 1, vr, j + 1);
      load_k(j + 2, kr);
      load_v(j + 2, vr);
      if (j < my_tiles) softmax_pv(qk(j & 1), j, j & 1);
      lds_barrier();
    }
  }

  // ---- merge the KG key groups through LDS.  A lane's 64 accumulator values (block dt,
  // element e: flat index 16*dt + e) form KG chunks of CS; wave (grp, rw) finishes chunk grp
  // of its query columns, and hands every other chunk to the wave that finishes it. ----
  lsum = xor32_sum(lsum);
  float* mo = reinterpret_cast<float*>(smem);  // [wave][KG - 1 chunks][CS values][64 lanes]
  float* mml = mo + 8 * (KG - 1) * CS * 64;    // [wave][m, l][64 lanes]
#pragma unroll
  for (int ch = 0; ch < KG; ++ch) {
    if (ch == grp) continue;  // uniform
    const int slot = ch < grp ? ch : ch - 1;
#pragma unroll
    for (int i = 0; i < CS; ++i)
      mo[((wave * (KG - 1) + slot) * CS + i) * 64 + lane] = o[(ch * CS + i) / 16][(ch * CS + i) % 16];
  }
  mml[(wave * 2) * 64 + lane] = m;
  mml[(wave * 2 + 1) * 64 + lane] = lsum;
  lds_barrier();
  float mg[KG], M = -INFINITY;
#pragma unroll
  for (int g = 0; g < KG; ++g) {
    mg[g] = mml[((g * RW + rw) * 2) * 64 + lane];
    M = fmaxf(M, mg[g]);
  }
  float L = 0.0f;
  float w[KG];
#pragma unroll
  for (int g = 0; g < KG; ++g) {
    w[g] = mg[g] == -INFINITY ? 0.0f : fast_exp2(mg[g] - M);
    L += w[g] * mml[((g * RW + rw) * 2 + 1) * 64 + lane];
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  if (q_valid) {
    // this wave's own chunk, weighted, plus the other groups' weighted chunks in group order
    float f[CS];
#pragma unroll
    for (int ch = 0; ch < KG; ++ch)
      if (ch == grp)
#pragma unroll
        for (int i = 0; i < CS; ++i) f[i] = o[(ch * CS + i) / 16][(ch * CS + i) % 16];
    float w_own = w[0];
#pragma unroll
    for (int g = 1; g < KG; ++g)
      if (grp == g) w_own = w[g];
#pragma unroll
    for (int i = 0; i < CS; ++i) f[i] *= w_own;
#pragma unroll
    for (int g = 0; g < KG; ++g) {
      if (g == grp) continue;
      const int slot = grp < g ? grp : grp - 1;
      const float* src = mo + ((g * RW + rw) * (KG - 1) + slot) * CS * 64 + lane;
#pragma unroll
      for (int i = 0; i < CS; ++i) f[i] += w[g] * src[i * 64];
    }
    // flat index 16*dt + 4*q4 + r holds dim 32*dt + 8*q4 + 4*h2 + r
    float* orow = a.out + (static_cast<long>(tq) * a.Hq + hq) * kDh + 4 * h2;
#pragma unroll
    for (int i = 0; i < CS / 4; ++i) {
      const int fl = grp * CS + 4 * i;
      *reinterpret_cast<float4*>(orow + 32 * (fl / 16) + 2 * (fl % 16)) =
          make_float4(f[4 * i] * inv, f[4 * i + 1] * inv, f[4 * i + 2] * inv, f[4 * i + 3] * inv);
    }
  }
  };  // run_block

  // Heaviest blocks first; paired: the heavy block n-1-i, then (after a barrier that frees
  // the merge area) the light block i, so every workgroup has about the same key count.
  run_block(a.n_tblocks - 1 - wi);
  if (RW > 1 && a.paired && wi < a.n_tblocks - 1 - wi) {  // RW = 1 grids are never paired
    __syncthreads();
    run_block(wi);
  }
}

template <int G, bool PRECISE>
int launch_rw(const PrefillArgs& args, int rw, hipStream_t stream) {
  const int n_work = args.paired ? (args.n_tblocks + 1) / 2 : args.n_tblocks;
  const dim3 grid(n_work * args.Hkv);
  if (rw == 4)
    hipLaunchKernelGGL((gqa_prefill_kernel<G, PRECISE, 4>), grid, dim3(kThreads), 0, stream, args);
  else if (rw == 2)
    hipLaunchKernelGGL((gqa_prefill_kernel<G, PRECISE, 2>), grid, dim3(kThreads), 0, stream, args);
  else
    hipLaunchKernelGGL((gqa_prefill_kernel<G, PRECISE, 1>), grid, dim3(kThreads), 0, stream, args);
  return check_launch("gqa_prefill_kernel");
}

template <int G>
int launch_g(PrefillArgs& args, bool precise, hipStream_t stream) {
  // 128 query rows per K/V tile when that still gives every CU two workgroups (heaviest-
  // first dispatch needs the second one to even out the causal triangle); measured on
  // MI355X: RW = 2 is faster at 2048 tokens x 8 kv heads, RW = 4 at 4096.
  // Prompts too short to give every CU an RW = 2 workgroup take RW = 1 (8 one-wave key
  // groups): twice the workgroups, half the rounds per workgroup.
  const int cus_q = device_cu_count();
  const int cus = cus_q > 0 ? cus_q : 256;
  const int blocks4 = (args.Tq + 4 * (32 / G) - 1) / (4 * (32 / G));
  const int blocks2 = (args.Tq + 2 * (32 / G) - 1) / (2 * (32 / G));
  const int rw = static_cast<long>(blocks4) * args.Hkv >= 2L * cus ? 4
                 : static_cast<long>(blocks2) * args.Hkv < cus     ? 1
                                                                    : 2;
  const int BT = rw * (32 / G);
  args.n_tblocks = (args.Tq + BT - 1) / BT;
  // Pairs of blocks (heavy n-1-i with light i) per workgroup once there are at least two
  // blocks per CU: one workgroup per CU instead of two back to back, and one prologue less.
  args.paired = rw > 1 && static_cast<long>(args.n_tblocks) * args.Hkv >= 2L * cus;
  return precise ? launch_rw<G, true>(args, rw, stream) : launch_rw<G, false>(args, rw, stream);
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
  if (mode != ORATOR_PREFILL_FP32 && mode != ORATOR_PREFILL_BF16)
    return fail(ORATOR_ERR_INVALID, "gqa_prefill: unknown precision mode");
  if (capacity <= 0) return fail(ORATOR_ERR_INVALID, "gqa_prefill: capacity must be > 0");
  if (!(scale > 0.0f)) return fail(ORATOR_ERR_INVALID, "gqa_prefill: scale must be > 0");
  if (Dh != kDh || !(G == 1 || G == 2 || G == 4)) {
    // head sizes and groups the MFMA kernels are not built for: the generic kernel (fp32
    // arithmetic in either mode), any Dh up to 1024
    if (Dh > 1024) return fail(ORATOR_ERR_UNSUPPORTED, "gqa_prefill: head size above 1024");
    int shift = 0;
    if (page_table) {
      shift = ilog2_exact(page_size);
      if (shift < 0 || max_pages <= 0)
        return fail(ORATOR_ERR_INVALID, "gqa_prefill: page_size must be a power of two");
      if (static_cast<long>(max_pages) * page_size < capacity)
        return fail(ORATOR_ERR_CAPACITY, "gqa_prefill: capacity exceeds max_pages*page_size");
    }
    return launch_prefill_generic(q, q_bf16, kpool, vpool, page_table, max_pages, shift, out, Tq,
                                  Hq, Hkv, Dh, d_pos0, capacity, scale, stream);
  }
  // the LDS page-row table of a paged cache covers 16384 keys; contiguous rows are arithmetic
  if (page_table && capacity > 16 * kMaxRowGroups)
    return fail(ORATOR_ERR_UNSUPPORTED, "gqa_prefill: paged caches hold at most 16384 keys");
  // Long bf16 prompts over a contiguous cache: the stream-K kernel (prefill_sk.hip), where it
  // measured faster on MI355X (Tq >= 2048 for GQA groups 1 and 2; below that, and for group
  // 4, its per-segment set-up and partial merges cost more than the work imbalance it
  // removes).  Its buffer offsets are 32-bit.
  if (mode == ORATOR_PREFILL_BF16 && !page_table && Tq >= kSkMinTokens && G <= 2 &&
      static_cast<long>(Hkv) * ((Tq + 128 / G - 1) / (128 / G)) <= kArriveCounters &&
      static_cast<long>(Tq) * Hq * kDh * 2 < (1L << 31) &&
      static_cast<long>(capacity) * Hkv * kDh * 2 < (1L << 31))
    return launch_prefill_sk(q, q_bf16, kpool, vpool, out, Tq, Hq, Hkv, d_pos0, capacity, scale,
                             stream);
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
