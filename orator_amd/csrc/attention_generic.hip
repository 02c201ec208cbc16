// Generic GQA attention for the shapes the MFMA prefill and split-K decode kernels are not
// built for: any head size up to 1024 and any Hq that is a multiple of Hkv.
//
// The reference's attention entry points take such shapes:
//  * asr_ops::GqaAttention (include/model/asr_ops.cuh:50-56, src/model/asr_ops.cu:113-195,
//    237-295): fp32 self-attention, any power-of-two head_dim up to 1024;
//  * GqaCacheAttnKernel (src/model/asr_text_decoder.cu:83-142): prefill over a bf16 cache,
//    any Dh <= 256 (qreg[8] of a 32-lane warp), any group;
//  * GqaDecodeAttnKernel (src/model/asr_text_decoder.cu:149-213): decode over a bf16 cache,
//    blockDim = Dh, any group.
// The fast kernels serve Dh 128 (prefill) and Dh 64 / 128 (decode) with Hq / Hkv in {1, 2, 4};
// every other shape runs here, with the same semantics: row r of q head h attends a key range
// of kv head h / (Hq / Hkv) -- [0, r] or [0, T) for self-attention, [0, pos0 + r] for a
// prefill, the stream's keys for a decode -- fp32 scores scaled after the dot, an online
// softmax, out = acc / l (0 when l = 0).
//
// One workgroup = (row, q head), 4 wave64s striding over the keys.  A key is covered by
// L = min(DHP, 64) lanes holding DHP / L elements each (element d = e * L + lane: coalesced
// rows; DHP is Dh rounded up to a power of two, elements d >= Dh are zero), so a wave takes
// 64 / L keys per step; each key slot keeps its own online-softmax state, merged across slots
// and waves in LDS at the end.
#include <math.h>

#include "common.hpp"
#include "internal.hpp"

namespace orator_hip {
namespace {

constexpr int kGenWaves = 4;

enum { kRowsSelf = 0, kRowsPrefill = 1, kRowsDecode = 2 };

struct GenericArgs {
  const void* q;  // [rows][Hq][Dh], fp32 or bf16 bits
  const void* k;  // key / value rows [.][Hkv][Dh], fp32 or bf16 bits
  const void* v;
  float* out;     // [rows][Hq][Dh]
  const int* page_table;  // paged caches: [streams][max_pages]
  int max_pages;
  int page_shift;
  long stream_stride;  // contiguous decode caches: elements between streams
  int rows, Hq, Hkv, Dh;
  float scale_log2e;
  int row_mode;  // kRowsSelf / kRowsPrefill / kRowsDecode
  int causal;    // self-attention
  const int* pos;  // prefill: pos0 (one word); decode: [streams]
  int pos_mode;    // decode, as DecodeProblem::pos_mode (0 .. 3)
  const int* seg_start;
  const int* seg_end;
  int capacity;
  // decode append (pos_mode 0): key pos[b] of stream b is the bf16 rounding of these rows
  // ([streams][Hkv][Dh] fp32), not the cache's
  const float* k_new;
  const float* v_new;
};

template <typename T>
__device__ __forceinline__ float elem(const T* p, long i) {
  if constexpr (sizeof(T) == 2)
    return bf16_to_f32(p[i]);
  else
    return p[i];
}

template <int DHP, typename QT, typename KV>
__global__ __launch_bounds__(64 * kGenWaves) void gqa_attention_generic_kernel(GenericArgs a) {
  constexpr int L = DHP < kWave ? DHP : kWave;  // lanes per key
  constexpr int KPI = kWave / L;                // keys per wave step
  constexpr int E = DHP / L;                    // elements per lane
  constexpr int NS = kGenWaves * KPI;           // key slots per workgroup
  __shared__ float s_ml[NS][2];
  __shared__ float s_o[NS][DHP];

  const int i = blockIdx.x;
  const int h = blockIdx.y;
  const int kvh = h / (a.Hq / a.Hkv);
  const int Dh = a.Dh;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane / L;  // key slot within the wave
  const int li = lane % L;
  const int slot = wave * KPI + sub;

  // the row's stream and key range [key0, key0 + S)
  int b = 0, key0 = 0, S;
  int new_key = -1;  // decode append: the key read from k_new / v_new
  if (a.row_mode == kRowsSelf) {
    S = a.causal ? i + 1 : a.rows;
  } else if (a.row_mode == kRowsPrefill) {
    S = min(*a.pos + i + 1, a.capacity);
  } else {
    b = i;
    if (a.pos_mode == 3) {
      key0 = min(max(a.seg_start[b], 0), a.capacity);
      S = min(max(a.seg_end[b], key0), a.capacity) - key0;
    } else {
      const int pb = a.pos_mode == 0 ? a.pos[b] : 0;
      S = a.pos_mode == 0 ? pb + 1 : (a.pos_mode == 1 ? b + 1 : a.capacity);
      S = min(S, a.capacity);
      if (a.k_new && S == pb + 1) new_key = S - 1;
    }
  }

  const QT* qp = static_cast<const QT*>(a.q) + (static_cast<long>(i) * a.Hq + h) * Dh;
  float qr[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int d = e * L + li;
    qr[e] = d < Dh ? elem(qp, d) : 0.0f;
  }
  const KV* kp = static_cast<const KV*>(a.k);
  const KV* vp = static_cast<const KV*>(a.v);
  const long rs = static_cast<long>(a.Hkv) * Dh;
  const long sbase = a.page_table ? 0 : static_cast<long>(b) * a.stream_stride;
  const float* kn = new_key >= 0 ? a.k_new + (static_cast<long>(b) * a.Hkv + kvh) * Dh : nullptr;
  const float* vn = new_key >= 0 ? a.v_new + (static_cast<long>(b) * a.Hkv + kvh) * Dh : nullptr;

  float m = -INFINITY, l = 0.0f, acc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.0f;
  for (int j0 = wave * KPI; j0 < S; j0 += NS) {
    const int jj = j0 + sub;
    const int j = key0 + min(jj, S - 1);  // an in-range key; slots past S get weight 0
    bool valid = jj < S;
    long row = j;
    if (a.page_table) {
      const int page = a.page_table[static_cast<long>(b) * a.max_pages + (j >> a.page_shift)];
      row = (static_cast<long>(page) << a.page_shift) + (j & ((1 << a.page_shift) - 1));
      valid = valid && (page >= 0 || j == new_key);  // an unmapped page is never read
    }
    const bool fresh = j == new_key;
    const long off = sbase + row * rs + static_cast<long>(kvh) * Dh;
    float kv[E], vv[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int d = e * L + li;
      kv[e] = 0.0f;
      vv[e] = 0.0f;
      if (d < Dh) {
        if (fresh) {  // the bf16 value the cache will hold
          kv[e] = bf16_to_f32(f32_to_bf16(kn[d]));
          vv[e] = bf16_to_f32(f32_to_bf16(vn[d]));
        } else if (valid) {
          kv[e] = elem(kp, off + d);
          vv[e] = elem(vp, off + d);
        }
      }
    }
    float dot = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) dot = fmaf(qr[e], kv[e], dot);
#pragma unroll
    for (int o = 1; o < L; o <<= 1) dot += __shfl_xor(dot, o);
    const float s = valid ? dot * a.scale_log2e : -INFINITY;
    const float mn = fmaxf(m, s);
    const float mr = mn == -INFINITY ? 0.0f : mn;
    const float corr = fast_exp2(m - mr);
    const float p = fast_exp2(s - mr);
    l = l * corr + p;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = fmaf(p, vv[e], acc[e] * corr);
    m = mn;
  }
  if (li == 0) {
    s_ml[slot][0] = m;
    s_ml[slot][1] = l;
  }
#pragma unroll
  for (int e = 0; e < E; ++e) s_o[slot][e * L + li] = acc[e];
  __syncthreads();
  for (int d = threadIdx.x; d < Dh; d += 64 * kGenWaves) {
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
    a.out[(static_cast<long>(i) * a.Hq + h) * Dh + d] = lv > 0.0f ? ov * (1.0f / lv) : 0.0f;
  }
}

template <int DHP>
int launch_dhp(const GenericArgs& a, bool q_bf16, bool kv_bf16, hipStream_t s) {
  const dim3 grid(a.rows, a.Hq), block(64 * kGenWaves);
  if (kv_bf16) {
    if (q_bf16)
      hipLaunchKernelGGL((gqa_attention_generic_kernel<DHP, uint16_t, uint16_t>), grid, block, 0,
                         s, a);
    else
      hipLaunchKernelGGL((gqa_attention_generic_kernel<DHP, float, uint16_t>), grid, block, 0, s,
                         a);
  } else {
    hipLaunchKernelGGL((gqa_attention_generic_kernel<DHP, float, float>), grid, block, 0, s, a);
  }
  return check_launch("gqa_attention_generic_kernel");
}

// Dh rounded up to a power of two (Dh in [1, 1024]).
int launch_generic(const GenericArgs& a, bool q_bf16, bool kv_bf16, hipStream_t s) {
  if (a.rows <= 0 || a.Hq <= 0) return ORATOR_OK;
  if (a.Hq > 65535) return fail(ORATOR_ERR_UNSUPPORTED, "gqa attention: at most 65535 q heads");
  if (a.Dh < 1 || a.Dh > 1024)
    return fail(ORATOR_ERR_UNSUPPORTED, "gqa attention: head size must be in [1, 1024]");
  int dhp = 1;
  while (dhp < a.Dh) dhp <<= 1;
  switch (dhp) {
    case 1: return launch_dhp<1>(a, q_bf16, kv_bf16, s);
    case 2: return launch_dhp<2>(a, q_bf16, kv_bf16, s);
    case 4: return launch_dhp<4>(a, q_bf16, kv_bf16, s);
    case 8: return launch_dhp<8>(a, q_bf16, kv_bf16, s);
    case 16: return launch_dhp<16>(a, q_bf16, kv_bf16, s);
    case 32: return launch_dhp<32>(a, q_bf16, kv_bf16, s);
    case 64: return launch_dhp<64>(a, q_bf16, kv_bf16, s);
    case 128: return launch_dhp<128>(a, q_bf16, kv_bf16, s);
    case 256: return launch_dhp<256>(a, q_bf16, kv_bf16, s);
    case 512: return launch_dhp<512>(a, q_bf16, kv_bf16, s);
    default: return launch_dhp<1024>(a, q_bf16, kv_bf16, s);
  }
}

// The decode append's cache write for the generic path: stream b's new K/V rows ([B][Hkv][Dh]
// fp32) stored as bf16 (round to nearest even) at position pos[b], as the fused append
// kernels store them: not written when pos[b] is outside [0, capacity), when its page-table
// entry is unmapped (< 0), or when its pool row is at or past pool_rows.
__global__ __launch_bounds__(256) void append_write_kernel(const float* __restrict__ k_new,
                                                           const float* __restrict__ v_new,
                                                           uint16_t* kpool, uint16_t* vpool,
                                                           GenericArgs a, long pool_rows) {
  const long idx = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  const long per_stream = static_cast<long>(a.Hkv) * a.Dh;
  if (idx >= per_stream * a.rows) return;
  const int b = static_cast<int>(idx / per_stream);
  const long hd = idx % per_stream;  // kv head * Dh + d
  const int pos = a.pos[b];
  if (pos < 0 || pos >= a.capacity) return;
  long off;
  if (a.page_table) {
    const int page = a.page_table[static_cast<long>(b) * a.max_pages + (pos >> a.page_shift)];
    const long row = (static_cast<long>(page) << a.page_shift) + (pos & ((1 << a.page_shift) - 1));
    if (page < 0 || row >= pool_rows) return;
    off = row * per_stream + hd;
  } else {
    off = static_cast<long>(b) * a.stream_stride + static_cast<long>(pos) * per_stream + hd;
  }
  kpool[off] = f32_to_bf16(k_new[idx]);
  vpool[off] = f32_to_bf16(v_new[idx]);
}

}  // namespace

int launch_gqa_attention_generic(const float* q, const float* k, const float* v, float* out,
                                 int T, int Hq, int Hkv, int Dh, float scale, bool causal,
                                 hipStream_t s) {
  GenericArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.rows = T;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.Dh = Dh;
  a.scale_log2e = scale * 1.4426950408889634f;
  a.row_mode = kRowsSelf;
  a.causal = causal ? 1 : 0;
  a.capacity = T;
  return launch_generic(a, false, false, s);
}

int launch_prefill_generic(const float* q, const uint16_t* q_bf16, const uint16_t* kpool,
                           const uint16_t* vpool, const int* page_table, int max_pages,
                           int page_shift, float* out, int Tq, int Hq, int Hkv, int Dh,
                           const int* d_pos0, int capacity, float scale, hipStream_t s) {
  GenericArgs a{};
  a.q = q ? static_cast<const void*>(q) : static_cast<const void*>(q_bf16);
  a.k = kpool;
  a.v = vpool;
  a.out = out;
  a.page_table = page_table;
  a.max_pages = max_pages;
  a.page_shift = page_shift;
  a.rows = Tq;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.Dh = Dh;
  a.scale_log2e = scale * 1.4426950408889634f;
  a.row_mode = kRowsPrefill;
  a.pos = d_pos0;
  a.capacity = capacity;
  return launch_generic(a, q == nullptr, true, s);
}

int launch_decode_generic(const DecodeProblem& p, int page_shift, hipStream_t s) {
  GenericArgs a{};
  a.q = p.q;
  a.k = p.kpool;
  a.v = p.vpool;
  a.out = p.out;
  a.page_table = p.page_table;
  a.max_pages = p.max_pages;
  a.page_shift = page_shift;
  a.stream_stride = p.stream_stride;
  a.rows = p.B;
  a.Hq = p.Hq;
  a.Hkv = p.Hkv;
  a.Dh = p.Dh;
  a.scale_log2e = p.scale * 1.4426950408889634f;
  a.row_mode = kRowsDecode;
  a.pos = p.pos;
  a.pos_mode = p.pos_mode;
  a.seg_start = p.seg_start;
  a.seg_end = p.seg_end;
  a.capacity = p.capacity;
  a.k_new = p.k_new;
  a.v_new = p.v_new;
  if (int rc = launch_generic(a, false, !p.kv_f32, s)) return rc;
  if (!p.k_new) return ORATOR_OK;
  // the appended rows were attended from k_new / v_new; now the cache gets them
  const long n = static_cast<long>(p.B) * p.Hkv * p.Dh;
  hipLaunchKernelGGL(append_write_kernel, dim3((n + 255) / 256), dim3(256), 0, s, p.k_new,
                     p.v_new, const_cast<uint16_t*>(static_cast<const uint16_t*>(p.kpool)),
                     const_cast<uint16_t*>(static_cast<const uint16_t*>(p.vpool)), a,
                     p.pool_rows);
  return check_launch("append_write_kernel");
}

}  // namespace orator_hip
