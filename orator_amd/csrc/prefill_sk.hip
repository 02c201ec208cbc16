// Causal GQA prefill attention for long prompts, bf16 mode, contiguous bf16 cache (gfx950).
//
// Same operation and semantics as the kernels in prefill_attn.hip (GqaCacheAttnKernel,
// src/model/asr_text_decoder.cu:88-142: query row t at absolute position pos0 + t attends keys
// [0, pos0 + t]; online softmax; out = acc / l), q and the softmax weights rounded to bf16,
// fp32 accumulation.  What differs is the work split, built for one wave per SIMD:
//
//  * a workgroup is 4 wave64s, one per SIMD, so each wave owns the whole 512-entry register
//    file: 64 query columns per wave (two 32x32 MFMA blocks: Q^T 64 registers, O^T 128
//    accumulators), so every K fragment and every V^T fragment read from LDS feeds two MFMAs
//    (half the LDS reads per MFMA of a 32-column wave);
//  * waves = 2 row waves (64 columns each: a block of 2 * 64 / G tokens x G heads) x 2 key
//    groups (even / odd 32-key tiles); the two row waves of a key group share its tiles;
//  * stream-K balance: per kv head, the blocks' key tiles are listed in heavy / light pair
//    order (the last block, the first, the second last, ...) and the list is cut into equal
//    contiguous ranges, one per workgroup (the kv head fastest in the grid, so a head's
//    workgroups share an XCD).  A workgroup runs the blocks its range touches as segments; a
//    block cut by a range boundary leaves one partial (m, l, unnormalised O) per workgroup in
//    the workspace, and the last workgroup to finish it (an arrival counter) merges them.
//    Partials and counters are agent-scope atomic accesses (coherent across the XCDs' L2s
//    without an L2 write-back).
//  * K and V tiles go from memory straight into LDS rings of four stages (LDS-DMA, three
//    rounds ahead of their use); per round a key group computes S^T = K Q^T of its next tile
//    interleaved with the softmax of the current one, then O^T += V^T P^T (V^T by
//    transposing LDS reads).  The softmax reference is fixed per segment (the accumulators
//    are never rescaled in the loop); a score more than 2^64 above it makes the workgroup
//    redo the segment with the maxima it has seen.
#include <algorithm>

#include "common.hpp"
#include "internal.hpp"
#include "mfma_tile.hpp"

namespace orator_hip {
namespace {

constexpr int kSkDh = 128;
constexpr int kSkBN = 32;                // keys per tile
constexpr int kSkThreads = 256;          // 4 wave64s, one per SIMD
constexpr float kSkSlack = 64.0f;        // log2 headroom of the softmax reference
// A cut block's partial, one slot: each wave (row wave rw, key group g) writes the 64 O^T
// values it finishes per lane as 16 lane-contiguous float4 (o[rw][g][16][64 lanes][4]), then
// m and l of its two columns ([rw][m0, m1, l0, l1][64 lanes], key group 0 only).  Every
// workgroup's wave (rw, g) maps lanes to the same columns and dims of a block, so the merging
// workgroup reads the other slots lane for lane.
constexpr int kSkPartO = 2 * 2 * 16 * 64 * 4;  // floats
constexpr int kSkPartSlot = kSkPartO + 2 * 4 * 64;
constexpr int kSkPartCoherent = 16;  // buffer cache policy sc1: coherent across the XCDs

struct SkArgs {
  const float* q;          // [Tq, Hq, Dh] fp32 (rounded to bf16 here), or
  const uint16_t* q_bf16;  // [Tq, Hq, Dh] bf16
  const uint16_t* kc;      // [capacity][Hkv][Dh] bf16
  const uint16_t* vc;
  const int* pos0p;
  float* out;              // [Tq, Hq, Dh] fp32
  float* part;             // [gridDim.x][2 slots][kSkPartSlot]
  unsigned* arrive;        // [Hkv][n_blocks] kCounterStride apart, zero between launches
  int Tq, Hq, Hkv, capacity;
  int n_blocks;            // token blocks per kv head
  int wgs;                 // workgroups per kv head
  float c;                 // scale * log2(e)
};


__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int u = __shfl_up(v, d);
    if (lane >= d) v += u;
  }
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) v += __shfl_xor(v, d);
  return v;
}

// Inline-asm MFMAs: Q^T (the S product's B operand) and the O^T accumulators stay in AGPRs
// (the compiler's own MFMA selection kept Q in VGPRs and copied it out of AGPRs at every use).
// The hardware does not interlock these; the wait states are placed by hand:
//  * every MFMA is preceded by s_nop 1: an operand written by a VALU instruction needs 2 wait
//    states before an MFMA reads it;
//  * a VALU (or LDS, memory) read of an MFMA result needs 12 wait states after the MFMA
//    (8-pass XDL on gfx950): given by mfma_result_guard() before such reads (the softmax of a
//    score tile, the rescale and the merge of the accumulators);
//  * a chain of MFMAs accumulating into the same registers needs none.
__device__ __forceinline__ void mfma_s0(f32x16_t& d, const u32x4_t& a, const u32x4_t& b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "a"(b));
}
__device__ __forceinline__ void mfma_s(f32x16_t& d, const u32x4_t& a, const u32x4_t& b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "a"(b));
}
__device__ __forceinline__ void mfma_o(f32x16_t& d, const u32x4_t& a, const u32x4_t& b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(d) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_result_guard() { asm volatile("s_nop 7\n\ts_nop 4" ::); }

// XOR swizzle of the 16-byte chunks of a 256-byte tile row (LDS-DMA writes 1 KB blocks of
// four unpadded rows): chunk c of row r sits at chunk c ^ swz(r).  The 32 K rows of an MFMA
// A-fragment read (16 rows per pass, one chunk each) and the 4 rows x 2 chunks of a
// transposing V read land in distinct bank groups.
__device__ __forceinline__ int swz(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }

// Maximum of the 16 scores of a lane's column: seven v_max3_f32 and a v_max_f32 (fmaxf
// compiled to two-operand maxima plus NaN-quieting copies of every operand).
__device__ __forceinline__ float max16(const f32x16_t& s) {
  float v;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(v) : "v"(s[0]), "v"(s[1]), "v"(s[2]));
#pragma unroll
  for (int e = 3; e < 15; e += 2)
    asm("v_max3_f32 %0, %0, %1, %2" : "+v"(v) : "v"(s[e]), "v"(s[e + 1]));
  asm("v_max_f32 %0, %0, %1" : "+v"(v) : "v"(s[15]));
  return v;
}

template <int G>
__global__ __launch_bounds__(kSkThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gqa_prefill_sk_kernel(SkArgs a) {
  constexpr int TW = 64 / G;   // tokens per row wave
  constexpr int BT = 2 * TW;   // tokens per block
  // K and V rings of kSkStages tiles per key group, each stage its own object (the wait
  // counter pass separates LDS-DMA writes into one stage from reads of another only for
  // distinct objects).  [key group][32 rows][128 dims], rows unpadded, chunks swizzled.
  __shared__ __align__(16) uint16_t ks0[2][kSkBN][kSkDh], ks1[2][kSkBN][kSkDh];
  __shared__ __align__(16) uint16_t ks2[2][kSkBN][kSkDh], ks3[2][kSkBN][kSkDh];
  __shared__ __align__(16) uint16_t vs0[2][kSkBN][kSkDh], vs1[2][kSkBN][kSkDh];
  __shared__ __align__(16) uint16_t vs2[2][kSkBN][kSkDh], vs3[2][kSkBN][kSkDh];
  __shared__ int s_last;
  __shared__ int s_restart;
  // key-group merge: 16 values per lane and wave per pass, and m / l of every wave
  __shared__ float4 s_xo[4][4][64];
  __shared__ float s_xml[4][4][64];
  auto kst = [&]<int S>() -> uint16_t* {
    if constexpr (S == 0) return &ks0[0][0][0];
    else if constexpr (S == 1) return &ks1[0][0][0];
    else if constexpr (S == 2) return &ks2[0][0][0];
    else return &ks3[0][0][0];
  };
  auto vst = [&]<int S>() -> uint16_t* {
    if constexpr (S == 0) return &vs0[0][0][0];
    else if constexpr (S == 1) return &vs1[0][0][0];
    else if constexpr (S == 2) return &vs2[0][0][0];
    else return &vs3[0][0][0];
  };

  const int kvh = blockIdx.x % a.Hkv;
  const int wg = blockIdx.x / a.Hkv;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 1;  // key group
  const int rw = wave & 1;    // row wave
  const int j32 = lane & 31, h2 = lane >> 5;

  const int pos0 = *a.pos0p;
  const int n = a.n_blocks;
  auto block_keys = [&](int b) { return min(pos0 + min((b + 1) * BT, a.Tq), a.capacity); };
  auto block_of = [&](int p) { return (p & 1) ? (p >> 1) : n - 1 - (p >> 1); };
  auto tiles_at = [&](int p) { return (block_keys(block_of(p)) + kSkBN - 1) / kSkBN; };

  // ---- this workgroup's range of the kv head's tile list, and its first block ----
  int U = 0;
  for (int p0 = 0; p0 < n; p0 += 64) {
    const int p = p0 + lane;
    U += wave_sum_i(p < n ? tiles_at(p) : 0);
  }
  U = __builtin_amdgcn_readfirstlane(U);
  const int per = (U + a.wgs - 1) / a.wgs;
  const int r0 = wg * per, r1 = min(r0 + per, U);
  if (r0 >= r1) return;  // uniform: nothing to do
  int p_cur = 0, excl = 0;
  for (int p0 = 0;; p0 += 64) {
    const int p = p0 + lane;
    const int t = p < n ? tiles_at(p) : 0;
    const int incl = excl + wave_incl_scan(t, lane);
    const uint64_t hit = __builtin_amdgcn_ballot_w64(p < n && incl > r0);
    if (hit) {
      const int l = __builtin_ctzll(hit);
      p_cur = p0 + l;
      excl = __builtin_amdgcn_readlane(incl, l) - __builtin_amdgcn_readlane(t, l);
      break;
    }
    excl = __builtin_amdgcn_readlane(incl, 63);
  }
  p_cur = __builtin_amdgcn_readfirstlane(p_cur);
  excl = __builtin_amdgcn_readfirstlane(excl);
  if (tid == 0) s_restart = 0;
  __syncthreads();

  // ---- per-lane LDS and memory addresses (fixed for the kernel) ----
  const uint32_t row_bytes = static_cast<uint32_t>(a.Hkv) * kSkDh * 2;
  // LDS-DMA: the wave fills rows 16 rw .. +15 of its group's tile, four rows (1 KB) per
  // instruction; lane l writes chunk l & 15 of row 4 i + l / 16, fetching the chunk that the
  // swizzle puts there
  uint32_t dma_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 16 * rw + 4 * i + (lane >> 4);
    dma_off[i] = r * row_bytes + kvh * kSkDh * 2 + (((lane & 15) ^ swz(r)) << 4);
  }
  const uint32_t grp_off = grp * kSkBN * kSkDh * 2;  // bytes: this group's half of a stage
  // K A-fragment of k-step ks: row j32, chunk 8 h2 + ks (the dim order q's B operand uses)
  uint32_t k_addr[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks)
    k_addr[ks] = grp_off + j32 * kSkDh * 2 + (((8 * h2 + ks) ^ swz(j32)) << 4);
  // V^T A-fragment of (16-key step st, 32-dim block dt): transposed reads of rows
  // 4 (tg >> 1) + (ts >> 2) (+8 for the second read, +16 st), dims 32 dt + 16 (tg & 1) + 4 (ts & 3)
  const int tg = lane >> 4, ts = lane & 15;
  uint32_t v_addr[2][4];  // [second read][dt]; st adds 16 rows
#pragma unroll
  for (int hh = 0; hh < 2; ++hh)
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const int r = 4 * (tg >> 1) + (ts >> 2) + 8 * hh;
      const int col = 32 * dt + 16 * (tg & 1) + 4 * (ts & 3);
      v_addr[hh][dt] = grp_off + r * kSkDh * 2 + (((col >> 3) ^ swz(r)) << 4) + ((col & 7) << 1);
    }
  const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.q_bf16), 0,
      static_cast<uint32_t>(a.Tq) * static_cast<uint32_t>(a.Hq) * kSkDh * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
      a.part, 0, static_cast<uint32_t>(gridDim.x * 2 * kSkPartSlot * 4), 0x00020000);

  // One segment: the part [t0, t1) of block p_cur that this workgroup's range holds.  Returns
  // whether the range goes on into the next block.  (Called in straight-line code for the
  // first two segments: inside a loop the register allocator spilled the accumulators.)
  auto segment = [&](bool first_seg) -> bool {
    const int tiles = tiles_at(p_cur);
    const int t0 = max(r0 - excl, 0), t1 = min(r1 - excl, tiles);
    const int b = block_of(p_cur);
    const int t_blk = b * BT;
    const int n_keys = block_keys(b);
    const int mask_from = min(pos0 + t_blk, n_keys - 1);  // tiles past this key need the mask
    const int n_my = t1 - t0 > grp ? (t1 - t0 - grp + 1) / 2 : 0;  // this group's tiles
    const int rounds = (t1 - t0 + 1) / 2;
    if (!first_seg) __syncthreads();  // the previous segment's merge area is free

    // K and V of the block's keys only: rows from n_keys on read as zeros (no V row past the
    // block's keys may hold a non-finite value: its weight is 0, and 0 * inf must not occur)
    const uint32_t kv_bytes = static_cast<uint32_t>(n_keys) * row_bytes;
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.kc), 0, kv_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.vc), 0, kv_bytes, 0x00020000);

    // ---- this wave's 64 query columns: block cb = 0, 1 of 32, column j32 ----
    int tq[2], hq[2], qlim[2];
    bool qv[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int f = 32 * cb + j32;
      tq[cb] = t_blk + rw * TW + f % TW;
      hq[cb] = kvh * G + f / TW;
      qv[cb] = tq[cb] < a.Tq;
      qlim[cb] = min(pos0 + tq[cb], n_keys - 1);
    }

    // Group-local tile j (block tile t0 + grp + 2 j) into ring stage S: four 1 KB LDS-DMA
    // loads each of K and V per wave.  Tiles past this group's last are issued too (as
    // loads past the buffer range: no memory traffic), so every round issues the same count
    // and the wait counts below stay exact.
    auto dma_k = [&]<int S>(int j) {
      const uint32_t soff = j < n_my ? (t0 + grp + 2 * j) * kSkBN * row_bytes : kv_bytes;
      uint16_t* dst = kst.template operator()<S>() + (grp_off >> 1) + 16 * rw * kSkDh;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            krs, (__attribute__((address_space(3))) void*)(dst + 4 * i * kSkDh), 16, dma_off[i],
            soff, 0, 0);
    };
    auto dma_v = [&]<int S>(int j) {
      const uint32_t soff = j < n_my ? (t0 + grp + 2 * j) * kSkBN * row_bytes : kv_bytes;
      uint16_t* dst = vst.template operator()<S>() + (grp_off >> 1) + 16 * rw * kSkDh;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            vrs, (__attribute__((address_space(3))) void*)(dst + 4 * i * kSkDh), 16, dma_off[i],
            soff, 0, 0);
    };

    // q^T, B operand of k-step ks: dims 64 h2 + 8 ks .. +7, held in AGPRs
    u32x4_t qf[2][8];

    // Softmax reference per column: fixed for an attempt at the segment (the accumulators are
    // never rescaled inside the rounds -- C++ arithmetic on them there made the compiler keep
    // VGPR copies of all 128).  A column's reference is its first finite tile maximum (moving
    // it from -inf is free: nothing has been accumulated); a later tile more than 2^kSkSlack
    // above it (weights up to 2^64 stay finite in bf16 and fp32) makes the workgroup redo the
    // segment with every wave's running maxima as references.  Scores of RMS-normed q and k
    // are bounded far below that; the redo is for arbitrary inputs.
    f32x16_t o[2][4];
    float m[2], mseen[2], lsum[2];
    float mhint[2] = {-INFINITY, -INFINITY};
    const float c = a.c;

    // causal / capacity mask of tile j's scores, the reference check, and the reference
    // subtracted from the scores (0 while a column has seen no finite score)
    float mref[2];  // reference subtracted from the current tile's scores
    auto mask_and_check = [&](f32x16_t (&s)[2], int j) {
      const int k0 = (t0 + grp + 2 * j) * kSkBN;
      if (k0 + kSkBN - 1 > mask_from) {  // uniform
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int key = k0 + 8 * (e >> 2) + 4 * h2 + (e & 3);
            if (key > qlim[cb]) s[cb][e] = -INFINITY;
          }
      }
      float mx[2];
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        mx[cb] = xor32_max(max16(s[cb])) * c;
        if (m[cb] == -INFINITY) m[cb] = mx[cb];
        mseen[cb] = fmaxf(mseen[cb], mx[cb]);
      }
      if (__builtin_amdgcn_ballot_w64(mx[0] > m[0] + kSkSlack || mx[1] > m[1] + kSkSlack))
        s_restart = 1;
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) mref[cb] = m[cb] == -INFINITY ? 0.0f : m[cb];
    };

    // One round j: S(j + 1) from K stage (j + 1) % 4, PV of tile j from V stage j % 4 (R =
    // j % 4); the scores of tile j in s_cur, those of tile j + 1 into s_nxt.  The round ends
    // waiting for this wave's loads of K(j + 2), V(j + 1) (issued in round j - 2) and a barrier.
    auto round = [&]<int R>(int j, f32x16_t (&s_cur)[2], f32x16_t (&s_nxt)[2]) {
      constexpr int SV = R % 4, SK = (R + 1) % 4;
      if (j < n_my) {  // uniform: this group has tile j
        // the K fragments first (at most 15 LDS reads may be outstanding per wave: the V^T
        // reads go out in the first slots below)
        u32x4_t kf[8];
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
          kf[ks] = *reinterpret_cast<const u32x4_t*>(
              reinterpret_cast<const char*>(kst.template operator()<SK>()) + k_addr[ks]);
        u32x4_t vf[2][4];
        auto read_v = [&](int st, int dt) {
          const uint16_t* vb = vst.template operator()<SV>() + 16 * st * kSkDh;
          const uint2 x0 = lds_read_tr16(reinterpret_cast<const uint16_t*>(
              reinterpret_cast<const char*>(vb) + v_addr[0][dt]));
          const uint2 x1 = lds_read_tr16(reinterpret_cast<const uint16_t*>(
              reinterpret_cast<const char*>(vb) + v_addr[1][dt]));
          vf[st][dt] = u32x4_t{x0.x, x0.y, x1.x, x1.y};
        };
        // Weights of tile j: p = 2^(s c - mref) for element e of column block cb; pairs packed
        // to bf16 (pk[cb][st] holds elements 8 st .. 8 st + 7: the PV B operand of 16-key step
        // st) and summed.
        float pv[2][16];
        u32x4_t pk[2][2];
        auto expw = [&](int cb, int e) { pv[cb][e] = fast_exp2(fmaf(s_cur[cb][e], c, -mref[cb])); };
        auto pack = [&](int cb, int e) {
          const uint32_t w = cvt_bf16x2(pv[cb][e], pv[cb][e + 1]);
          pk[cb][e >> 3][(e & 7) >> 1] = w;
          lsum[cb] = add_bf16x2(w, lsum[cb]);
        };
        __builtin_amdgcn_sched_barrier(0);
        // 32 slots, one MFMA each with ~30 cycles of independent VALU behind it (a lone wave on
        // its SIMD issues an MFMA into a busy matrix pipe only by stalling, VALU included):
        //  slots 0..15  S(j + 1), k-step i / 2, column block i % 2;
        //  slots 16..31 PV of tile j, 16-key step (i - 16) / 8, dims block ((i - 16) / 2) % 4,
        //               column block i % 2.
        // Exponentials: elements 0..7 of both column blocks in slots 0..7 (two per slot),
        // elements 8..15 of block 0 in slots 8..15 and of block 1 in slots 16..23 (one per
        // slot); each pair is packed two slots after its second exponential.  V^T reads in
        // slots 0..7, the LDS-DMA of later tiles in slots 24 and 28.
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          if (i < 16) {
            const int ks = i >> 1, cb = i & 1;
            if (ks == 0)
              mfma_s0(s_nxt[cb], kf[0], qf[cb][0]);
            else
              mfma_s(s_nxt[cb], kf[ks], qf[cb][ks]);
          } else {
            const int st = (i - 16) >> 3, dt = ((i - 16) >> 1) & 3, cb = i & 1;
            o[cb][dt] = mfma32(__builtin_bit_cast(bf16x8_t, vf[st][dt]),
                               __builtin_bit_cast(bf16x8_t, pk[cb][st]), o[cb][dt]);
          }
          if (i < 8) read_v(i >> 2, i & 3);
          if (i < 8) {  // elements 2 (i / 2) + {0, 1} of block i % 2
            expw(i & 1, 2 * (i >> 1));
            expw(i & 1, 2 * (i >> 1) + 1);
          } else if (i < 24) {  // element 8 + (i - 8) % 8 of block (i - 8) / 8
            expw((i - 8) >> 3, 8 + ((i - 8) & 7));
          }
          if (i >= 2 && i < 10) pack((i - 2) & 1, 2 * ((i - 2) >> 1));
          if (i >= 11 && i <= 17 && ((i - 11) & 1) == 0) pack(0, 8 + (i - 11));
          if (i >= 19 && i <= 23 && ((i - 19) & 1) == 0) pack(1, 8 + (i - 19));
          if (i == 24) pack(1, 14);
          if (i == 24) dma_k.template operator()<SV>(j + 4);
          if (i == 28) dma_v.template operator()<(R + 3) % 4>(j + 3);
          __builtin_amdgcn_sched_barrier(0);
        }
        // mask, maximum and reference check of tile j + 1, under the last PV MFMAs
        if (j + 1 < n_my) {
          mfma_result_guard();  // s_nxt came out of MFMAs
          mask_and_check(s_nxt, j + 1);
        }
      } else {
        dma_k.template operator()<SV>(j + 4);
        dma_v.template operator()<(R + 3) % 4>(j + 3);
      }
      // vmcnt(16): this wave's K(j + 2), V(j + 1) (issued three rounds back) landed
      __builtin_amdgcn_s_waitcnt(0x4f70);
      __builtin_amdgcn_s_barrier();
    };

    for (;;) {  // attempts at the segment (a second one only after a reference check failed)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[cb][dt][e] = 0.0f;
        m[cb] = mseen[cb] = mhint[cb];
        lsum[cb] = 0.0f;
      }
      // ---- prologue: K0..K3 and V0..V2 by LDS-DMA into stages 0..3, S(0).  Round j loads
      // K(j + 4) into K(j)'s stage and V(j + 3) into V(j - 1)'s (both last read in round
      // j - 1, before its closing barrier), three rounds ahead of their use ----
      // bf16 q goes out right after K0 (by LDS-DMA: 4 rows of 256 bytes per instruction, where
      // per-lane 16-byte loads of a column's dims touched a cache line per lane), and S(0)
      // waits for those two only.  The row wave's q is staged in the stage-3 V ring (row wave
      // 0; V3 is first loaded in round 0) or the merge area (row wave 1), one 32-column block
      // per key-group wave.  fp32 q is converted as it arrives, so its loads go out last.
      dma_k.template operator()<0>(0);
      if (a.q_bf16) {  // uniform
        uint32_t qoff[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int r = 4 * i + (lane >> 4);
          const int f = 32 * grp + r;
          const int t = min(t_blk + rw * TW + f % TW, a.Tq - 1);
          qoff[i] = static_cast<uint32_t>((t * a.Hq + kvh * G + f / TW) * kSkDh * 2) +
                    (((lane & 15) ^ swz(r)) << 4);
        }
        auto dma_q = [&](uint16_t* region) {
          uint16_t* dst = region + grp * kSkBN * kSkDh;
#pragma unroll
          for (int i = 0; i < 8; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                qrs, (__attribute__((address_space(3))) void*)(dst + 4 * i * kSkDh), 16, qoff[i],
                0, 0, 0);
        };
        if (rw == 0)
          dma_q(&vs3[0][0][0]);
        else
          dma_q(reinterpret_cast<uint16_t*>(&s_xo[0][0][0]));
      }
      dma_k.template operator()<1>(1);
      dma_v.template operator()<0>(0);
      if (!a.q_bf16) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          const long qoff =
              (static_cast<long>(min(tq[cb], a.Tq - 1)) * a.Hq + hq[cb]) * kSkDh + 64 * h2;
#pragma unroll
          for (int ks = 0; ks < 8; ++ks) {
            const float4 x0 = *reinterpret_cast<const float4*>(a.q + qoff + 8 * ks);
            const float4 x1 = *reinterpret_cast<const float4*>(a.q + qoff + 8 * ks + 4);
            qf[cb][ks] = u32x4_t{cvt_bf16x2(x0.x, x0.y), cvt_bf16x2(x0.z, x0.w),
                                 cvt_bf16x2(x1.x, x1.y), cvt_bf16x2(x1.z, x1.w)};
          }
        }
      }
      // vmcnt(8): K0 and q landed (K1, V0 may be in flight); K0's rows and the q blocks come
      // from both waves of a key group / row wave
      __builtin_amdgcn_s_waitcnt(0x0f78);
      __builtin_amdgcn_s_barrier();
      if (a.q_bf16) {  // q^T fragments: the K fragment addresses of rows (columns) j32
        auto read_q = [&](const uint16_t* region) {
#pragma unroll
          for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int ks = 0; ks < 8; ++ks)
              qf[cb][ks] = *reinterpret_cast<const u32x4_t*>(
                  reinterpret_cast<const char*>(region) + cb * kSkBN * kSkDh * 2 +
                  (k_addr[ks] - grp_off));
        };
        if (rw == 0)
          read_q(&vs3[0][0][0]);
        else
          read_q(reinterpret_cast<const uint16_t*>(&s_xo[0][0][0]));
      }
      // the other tiles of the prologue queue behind K0 and q (the loads of one CU go through
      // its memory pipeline at about 1 KB per 16 cycles): issued once those two are in
      dma_k.template operator()<2>(2);
      dma_v.template operator()<1>(1);
      dma_k.template operator()<3>(3);
      dma_v.template operator()<2>(2);
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)  // tokens past the prompt: q = 0 (never stored)
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
          if (!qv[cb]) qf[cb][ks] = u32x4_t{0, 0, 0, 0};
          asm volatile("" : "+a"(qf[cb][ks]));
        }
      f32x16_t sA[2], sB[2];
      if (n_my > 0) {
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
          const u32x4_t kf = *reinterpret_cast<const u32x4_t*>(
              reinterpret_cast<const char*>(&ks0[0][0][0]) + k_addr[ks]);
          if (ks == 0) {
            mfma_s0(sA[0], kf, qf[0][0]);
            mfma_s0(sA[1], kf, qf[1][0]);
          } else {
            mfma_s(sA[0], kf, qf[0][ks]);
            mfma_s(sA[1], kf, qf[1][ks]);
          }
        }
      }
      if (n_my > 0) {
        mfma_result_guard();
        mask_and_check(sA, 0);
      }
      // vmcnt(16), lgkmcnt(0): K1 and V0 landed (round 0 reads them), this wave's K0 reads
      // done
      __builtin_amdgcn_s_waitcnt(0x4070);
      __builtin_amdgcn_s_barrier();
      for (int j = 0; j < rounds; j += 4) {
        round.template operator()<0>(j, sA, sB);
        if (j + 1 >= rounds) break;
        round.template operator()<1>(j + 1, sB, sA);
        if (j + 2 >= rounds) break;
        round.template operator()<2>(j + 2, sA, sB);
        if (j + 3 >= rounds) break;
        round.template operator()<3>(j + 3, sB, sA);
      }
      // every LDS-DMA write (the rounds' loads past the end included) lands before the merge
      // area reuses the rings
      __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
      __syncthreads();
      if (!s_restart) break;  // uniform: read after the barrier above
      // redo with every column's maximum so far as its reference
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) mhint[cb] = mseen[cb];
      __syncthreads();  // every wave has read the flag
      if (tid == 0) s_restart = 0;
      __syncthreads();
    }
    mfma_result_guard();  // the accumulators came out of MFMAs

    // ---- merge the two key groups through LDS: wave (grp, rw) finishes dims 64 grp .. of
    // its columns (blocks dt = KD, KD + 1 of the accumulators) and hands the other half to the
    // partner wave (1 - grp, rw).  KD is a template argument: a run-time index into the
    // accumulators would put them in scratch memory. ----
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) lsum[cb] = xor32_sum(lsum[cb]);
    const int pw = (1 - grp) * 2 + rw;
    auto finish = [&]<int KD>() {
      constexpr int GD = 2 - KD;  // the half handed over
      // m and l of every wave and the 64 accumulator values each wave hands over (lane-
      // contiguous float4s in a K ring stage of its own: the rings are idle once the rounds'
      // loads have landed, and the next segment's first LDS-DMA waits behind the barrier at
      // its start), one barrier, then the partner's half folded in: one barrier where a
      // 16 KB area passed one 16-value block at a time needed eight
      float4* const xo_mine = reinterpret_cast<float4*>(
          wave == 0 ? &ks0[0][0][0] : wave == 1 ? &ks1[0][0][0] : wave == 2 ? &ks2[0][0][0]
                                                                              : &ks3[0][0][0]);
      const float4* const xo_part = reinterpret_cast<const float4*>(
          pw == 0 ? &ks0[0][0][0] : pw == 1 ? &ks1[0][0][0] : pw == 2 ? &ks2[0][0][0]
                                                                      : &ks3[0][0][0]);
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        s_xml[wave][cb][lane] = m[cb];
        s_xml[wave][2 + cb][lane] = lsum[cb];
      }
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4)
            xo_mine[((cb * 2 + i) * 4 + q4) * 64 + lane] =
                make_float4(o[cb][GD + i][4 * q4], o[cb][GD + i][4 * q4 + 1],
                            o[cb][GD + i][4 * q4 + 2], o[cb][GD + i][4 * q4 + 3]);
      float M[2], L[2], wo[2], wp[2];
      __syncthreads();
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const float mp = s_xml[pw][cb][lane];
        const float lp = s_xml[pw][2 + cb][lane];
        M[cb] = fmaxf(m[cb], mp);
        wo[cb] = m[cb] == -INFINITY ? 0.0f : fast_exp2(m[cb] - M[cb]);
        wp[cb] = mp == -INFINITY ? 0.0f : fast_exp2(mp - M[cb]);
        // in key-group order, so both waves of a row wave hold the same L
        L[cb] = grp == 0 ? wo[cb] * lsum[cb] + wp[cb] * lp : wp[cb] * lp + wo[cb] * lsum[cb];
      }
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const float4 x = xo_part[((cb * 2 + i) * 4 + q4) * 64 + lane];
            o[cb][KD + i][4 * q4] = wo[cb] * o[cb][KD + i][4 * q4] + wp[cb] * x.x;
            o[cb][KD + i][4 * q4 + 1] = wo[cb] * o[cb][KD + i][4 * q4 + 1] + wp[cb] * x.y;
            o[cb][KD + i][4 * q4 + 2] = wo[cb] * o[cb][KD + i][4 * q4 + 2] + wp[cb] * x.z;
            o[cb][KD + i][4 * q4 + 3] = wo[cb] * o[cb][KD + i][4 * q4 + 3] + wp[cb] * x.w;
          }

      // ---- whole block: normalise and store; cut block: a partial, and the last
      // workgroup to finish the block merges the partials ----
      bool store_out = t0 == 0 && t1 == tiles;
      if (!store_out) {
        const int w1 = excl / per, w2 = (excl + tiles - 1) / per;
        const int slot = blockIdx.x * 2 + (first_seg ? 0 : 1);
        // slot offsets in bytes: this wave's O block, and its row wave's m / l block
        const uint32_t o_off = static_cast<uint32_t>(slot * kSkPartSlot +
                                                     ((rw * 2 + grp) * 16 * 64 + lane) * 4) * 4;
        const uint32_t ml_off =
            static_cast<uint32_t>(slot * kSkPartSlot + kSkPartO + rw * 4 * 64 + lane) * 4;
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
              const int f4 = (cb * 2 + i) * 4 + q4;
              const f32x16_t& ov = o[cb][KD + i];
              const u32x4_t v = {__float_as_uint(ov[4 * q4]), __float_as_uint(ov[4 * q4 + 1]),
                                 __float_as_uint(ov[4 * q4 + 2]), __float_as_uint(ov[4 * q4 + 3])};
              __builtin_amdgcn_raw_buffer_store_b128(v, prs, o_off + f4 * 64 * 16, 0,
                                                     kSkPartCoherent);
            }
        if (KD == 0) {
#pragma unroll
          for (int cb = 0; cb < 2; ++cb) {
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(M[cb]), prs,
                                                  ml_off + cb * 64 * 4, 0, kSkPartCoherent);
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(L[cb]), prs,
                                                  ml_off + (2 + cb) * 64 * 4, 0, kSkPartCoherent);
          }
        }
        // every thread's partial stores are complete at the coherent level before the count
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0) {
          unsigned* ctr = a.arrive + (static_cast<long>(kvh) * n + b) * kCounterStride;
          const unsigned prev =
              __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          const int last = prev + 1 == static_cast<unsigned>(w2 - w1 + 1);
          if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          s_last = last;
        }
        __syncthreads();
        store_out = s_last;
        if (store_out) {
          // fold in the other workgroups' partials of this block
          for (int wo = w1; wo <= w2; ++wo) {
            if (wo == wg) continue;
            const int oslot = (kvh + a.Hkv * wo) * 2 + ((wo == w1 && excl > w1 * per) ? 1 : 0);
            const uint32_t oo = static_cast<uint32_t>(oslot * kSkPartSlot +
                                                      ((rw * 2 + grp) * 16 * 64 + lane) * 4) * 4;
            const uint32_t om =
                static_cast<uint32_t>(oslot * kSkPartSlot + kSkPartO + rw * 4 * 64 + lane) * 4;
            // the slot's 20 loads all go out before the first use: one memory latency per slot
            float mp[2], lp[2];
            u32x4_t pv[16];
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
              mp[cb] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                  prs, om + cb * 64 * 4, 0, kSkPartCoherent));
              lp[cb] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                  prs, om + (2 + cb) * 64 * 4, 0, kSkPartCoherent));
            }
#pragma unroll
            for (int f4 = 0; f4 < 16; ++f4)
              pv[f4] = __builtin_amdgcn_raw_buffer_load_b128(prs, oo + f4 * 64 * 16, 0,
                                                             kSkPartCoherent);
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
              const float Mn = fmaxf(M[cb], mp[cb]);
              const float wm = M[cb] == -INFINITY ? 0.0f : fast_exp2(M[cb] - Mn);
              const float wp = mp[cb] == -INFINITY ? 0.0f : fast_exp2(mp[cb] - Mn);
              M[cb] = Mn;
              L[cb] = wm * L[cb] + wp * lp[cb];
#pragma unroll
              for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                  const u32x4_t& v = pv[(cb * 2 + i) * 4 + q4];
#pragma unroll
                  for (int e = 0; e < 4; ++e)
                    o[cb][KD + i][4 * q4 + e] =
                        wm * o[cb][KD + i][4 * q4 + e] + wp * __uint_as_float(v[e]);
                }
            }
          }
        }
      }
      if (store_out) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          if (!qv[cb]) continue;
          const float inv = L[cb] > 0.0f ? 1.0f / L[cb] : 0.0f;
          float* orow = a.out + (static_cast<long>(tq[cb]) * a.Hq + hq[cb]) * kSkDh + 4 * h2;
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4)
              *reinterpret_cast<float4*>(orow + 32 * (KD + i) + 8 * q4) = make_float4(
                  o[cb][KD + i][4 * q4] * inv, o[cb][KD + i][4 * q4 + 1] * inv,
                  o[cb][KD + i][4 * q4 + 2] * inv, o[cb][KD + i][4 * q4 + 3] * inv);
        }
      }
    };
    if (grp == 0)
      finish.template operator()<0>();
    else
      finish.template operator()<2>();

    excl += tiles;
    ++p_cur;
    return excl < r1 && p_cur < n;
  };
  if (segment(true) && segment(false))
    while (segment(false)) {
    }
}

}  // namespace

// Long-prompt bf16 prefill over a contiguous cache (see the header).  The caller has checked
// Dh = 128, G in {1, 2, 4}, the pointers and the capacity.
int launch_prefill_sk(const float* q, const uint16_t* q_bf16, const uint16_t* kc,
                      const uint16_t* vc, float* out, int Tq, int Hq, int Hkv,
                      const int* d_pos0, int capacity, float scale, hipStream_t stream) {
  const int G = Hq / Hkv;
  const int cus_q = device_cu_count();
  const int cus = cus_q > 0 ? cus_q : 256;
  SkArgs a{};
  a.q = q;
  a.q_bf16 = q ? nullptr : q_bf16;
  a.kc = kc;
  a.vc = vc;
  a.pos0p = d_pos0;
  a.out = out;
  a.Tq = Tq;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.capacity = capacity;
  const int BT = 2 * 64 / G;
  a.n_blocks = (Tq + BT - 1) / BT;
  a.wgs = std::max(1, cus / Hkv);
  a.c = scale * 1.4426950408889634f;
  if (static_cast<long>(Hkv) * a.n_blocks > kArriveCounters)
    return fail(ORATOR_ERR_UNSUPPORTED, "gqa_prefill: too many token blocks for the counters");
  const int grid = Hkv * a.wgs;
  const size_t part_bytes =
      static_cast<size_t>(grid) * 2 * kSkPartSlot * sizeof(float);
  a.part = static_cast<float*>(workspace(stream, part_bytes, kWsPrefill));
  if (!a.part) return ORATOR_ERR_HIP;
  if (int rc = zeroed_counters(stream, kWsPrefillArrive, &a.arrive)) return rc;
  if (G == 1)
    hipLaunchKernelGGL((gqa_prefill_sk_kernel<1>), dim3(grid), dim3(kSkThreads), 0, stream, a);
  else if (G == 2)
    hipLaunchKernelGGL((gqa_prefill_sk_kernel<2>), dim3(grid), dim3(kSkThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((gqa_prefill_sk_kernel<4>), dim3(grid), dim3(kSkThreads), 0, stream, a);
  return check_launch("gqa_prefill_sk_kernel");
}

}  // namespace orator_hip
