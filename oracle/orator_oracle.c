/*
 * orator_oracle.c -- CPU restatement of Orator's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels, never part of the
 * product path (see orator_oracle.h).  Built with -O3 -ffp-contract=off, no fast-math and
 * no SIMD intrinsics, so the fp32 operation order of every output is the one written here
 * (the compiler may only run independent outputs side by side, as in orc_linear_bf16).
 *
 * Pinning (what checks each function, all in tests/test_oracle.py):
 *   orc_f32_to_bf16         known-answer values + torch's RNE bf16 cast, bit-exact
 *   orc_rms_norm            reference fixture recipe (tools/dump/dump_asr_ops.py:41-52)
 *                           recomputed with torch; scale invariance; constant rows
 *   orc_rope_interleaved    reference fixture recipe (dump_asr_ops.py:55-75) with torch
 *   orc_rope_half           torch rotate_half formula in fp64; pos=0 identity; pair norms;
 *                           relative-position invariance of q.k
 *   orc_swiglu              reference fixture recipe (dump_asr_ops.py:78-88) with torch
 *   orc_kv_write(_paged)    bf16 bit-exactness; paged == contiguous for identity tables
 *   orc_gqa_attention       reference fixture recipe (dump_asr_ops.py:91-110): torch SDPA
 *                           with repeat_interleave'd K/V; fp64 truth
 *   orc_gqa_prefill(_paged) torch SDPA on the bf16-decoded cache with a pos0 offset mask;
 *                           split-prefill equivalence; S=1 -> v0; identical keys -> mean(V)
 *   orc_gqa_decode(_paged)  equals the last row of a causal prefill; page permutation
 *                           invariance; fp64 truth
 *   orc_build_pos_emb       closed form sin/cos in fp64
 *   orc_relpos_attention    closed-form rel shift BD[T-1-i+j] (fp64 truth); u=v=0,P=0
 *                           reduces to torch SDPA (non-causal MHA); key masking
 *   orc_sgemm(_batched)     the reference's own test pattern (test_gemm_batched.cu:12-61)
 *                           against fp64 numpy matmul
 *   orc_argmax_banned       numpy argmax with bans; the reference tie rule on planted ties
 *   orc_linear_bf16         fp64 numpy matmul of the bf16-decoded operands; GELU against
 *                           math.erf; ReLU; bias
 *   orc_layer_norm,         torch F.layer_norm / F.glu / F.conv1d(groups=C) + F.batch_norm
 *   orc_glu_mask,           (eval) + F.silu in fp64; the composed Conformer layer against the
 *   orc_dwconv_bn_silu      same torch routines with the rel-pos core from orc_relpos_attention
 *   orc_masked_mha          torch SDPA with a key-padding mask; == orc_relpos_attention with
 *                           u = v = 0 and P = 0; valid_len 0 -> mean of V
 *   orc_window_attention    full windows == orc_gqa_attention non-causal (torch SDPA pinned);
 *                           block-diagonal windows == per-segment SDPA; empty window -> 0;
 *                           fp64 softmax brute force
 */
#include "orator_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* bf16                                                                      */
/* ------------------------------------------------------------------------- */

/* Round-to-nearest-even, as the host restatement at test/unit/model/test_asr_gemm.cc:21-27
 * and __float2bfloat16 at src/model/asr_text_decoder.cu:75-76 (finite inputs). */
uint16_t orc_f32_to_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, sizeof(u));
  const uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

/* bits << 16 (src/model/asr_text_decoder.cu:79-81, include/model/gemm.cuh:285-287). */
float orc_bf16_to_f32(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, sizeof(f));
  return f;
}

void orc_f32_to_bf16_n(const float* in, uint16_t* out, long n) {
  for (long i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(in[i]);
}

void orc_bf16_to_f32_n(const uint16_t* in, float* out, long n) {
  for (long i = 0; i < n; ++i) out[i] = orc_bf16_to_f32(in[i]);
}

/* ------------------------------------------------------------------------- */
/* a1 RMSNorm -- src/model/asr_ops.cu:21-51                                   */
/* 256 thread-strided fp32 partial sums, then a halving tree; inv computed    */
/* once per row; y = (x*inv)*w.                                               */
/* ------------------------------------------------------------------------- */
void orc_rms_norm(const float* x, const float* w, float* out, int rows, int dim, float eps) {
  enum { kThreads = 256 };
  float red[kThreads];
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (size_t)r * dim;
    float* yr = out + (size_t)r * dim;
    for (int t = 0; t < kThreads; ++t) {
      float local = 0.0f;
      for (int d = t; d < dim; d += kThreads) local += xr[d] * xr[d];
      red[t] = local;
    }
    for (int s = kThreads / 2; s > 0; s >>= 1)
      for (int t = 0; t < s; ++t) red[t] += red[t + s];
    const float ms = red[0] / (float)dim + eps;
    const float inv = (float)(1.0 / sqrt((double)ms)); /* correctly rounded rsqrtf */
    for (int d = 0; d < dim; ++d) yr[d] = xr[d] * inv * w[d];
  }
}

/* ------------------------------------------------------------------------- */
/* a2/a3 RoPE -- src/model/asr_ops.cu:57-75 (interleaved), 92-111 (half)      */
/* inv_freq = powf(base, -2j/Dh) with the exponent formed in fp32; the angle  */
/* pos*inv_freq is an fp32 product.  pow/sin/cos are evaluated in fp64 and    */
/* rounded once, i.e. the correctly rounded values the fp32 library calls     */
/* approximate.                                                               */
/* ------------------------------------------------------------------------- */
float orc_rope_inv_freq(float base, int j, int head_dim) {
  const float e = -2.0f * (float)j / (float)head_dim;
  return (float)pow((double)base, (double)e);
}

void orc_rope_half(float* x, const int* pos, int n_tokens, int n_heads, int head_dim,
                   float base) {
  const int half = head_dim / 2;
  for (int t = 0; t < n_tokens; ++t) {
    const float p = (float)pos[t];
    for (int h = 0; h < n_heads; ++h) {
      float* xr = x + ((size_t)t * n_heads + h) * head_dim;
      for (int j = 0; j < half; ++j) {
        const float angle = p * orc_rope_inv_freq(base, j, head_dim);
        const float c = (float)cos((double)angle);
        const float s = (float)sin((double)angle);
        const float a = xr[j];
        const float b = xr[j + half];
        xr[j] = a * c - b * s;
        xr[j + half] = b * c + a * s;
      }
    }
  }
}

void orc_rope_interleaved(float* x, const int* pos, int n_tokens, int n_heads, int head_dim,
                          float base) {
  const int half = head_dim / 2;
  for (int t = 0; t < n_tokens; ++t) {
    const float p = (float)pos[t];
    for (int h = 0; h < n_heads; ++h) {
      float* xr = x + ((size_t)t * n_heads + h) * head_dim;
      for (int i = 0; i < half; ++i) {
        const float angle = p * orc_rope_inv_freq(base, i, head_dim);
        const float c = (float)cos((double)angle);
        const float s = (float)sin((double)angle);
        const float a = xr[2 * i];
        const float b = xr[2 * i + 1];
        xr[2 * i] = a * c - b * s;
        xr[2 * i + 1] = a * s + b * c;
      }
    }
  }
}

/* SwiGLU -- src/model/asr_ops.cu:80-87: (g / (1 + expf(-g))) * u */
void orc_swiglu(const float* gate, const float* up, float* out, int n) {
  for (int i = 0; i < n; ++i) {
    const float g = gate[i];
    out[i] = (g / (1.0f + expf(-g))) * up[i];
  }
}

/* ------------------------------------------------------------------------- */
/* a4 KV write -- src/model/asr_text_decoder.cu:62-77                         */
/* ------------------------------------------------------------------------- */
void orc_kv_write(const float* k, const float* v, uint16_t* kc, uint16_t* vc, int Tq, int Hkv,
                  int Dh, int pos0) {
  const long total = (long)Tq * Hkv * Dh;
  for (long idx = 0; idx < total; ++idx) {
    const int d = (int)(idx % Dh);
    const int h = (int)((idx / Dh) % Hkv);
    const int t = (int)(idx / ((long)Dh * Hkv));
    const long dst = ((long)(pos0 + t) * Hkv + h) * Dh + d;
    kc[dst] = orc_f32_to_bf16(k[idx]);
    vc[dst] = orc_f32_to_bf16(v[idx]);
  }
}

/* Paged form: absolute position P lives in page page_table[P / page_size], row
 * P % page_size; a page holds [page_size, Hkv, Dh].  With page_table[i] = i this is
 * exactly the contiguous layout above. */
static inline long paged_row(const int* page_table, int page_size, int pos, int Hkv, int h,
                             int Dh) {
  const long page = page_table[pos / page_size];
  return ((page * page_size + pos % page_size) * Hkv + h) * (long)Dh;
}

void orc_kv_write_paged(const float* k, const float* v, uint16_t* kpool, uint16_t* vpool,
                        const int* page_table, int page_size, int Tq, int Hkv, int Dh, int pos0) {
  for (int t = 0; t < Tq; ++t)
    for (int h = 0; h < Hkv; ++h) {
      const long dst = paged_row(page_table, page_size, pos0 + t, Hkv, h, Dh);
      const float* ks = k + ((size_t)t * Hkv + h) * Dh;
      const float* vs = v + ((size_t)t * Hkv + h) * Dh;
      for (int d = 0; d < Dh; ++d) {
        kpool[dst + d] = orc_f32_to_bf16(ks[d]);
        vpool[dst + d] = orc_f32_to_bf16(vs[d]);
      }
    }
}

/* ------------------------------------------------------------------------- */
/* a5 prefill attention -- src/model/asr_text_decoder.cu:88-142               */
/* Row t (absolute position pos0+t) attends keys [0, pos0+t]; online softmax  */
/* from m = -1e30 with expf; out = acc * (1/l), or 0 when l == 0.             */
/* ------------------------------------------------------------------------- */
typedef struct {
  const int* page_table; /* NULL => contiguous */
  int page_size;
} kv_map;

static inline long kv_row(kv_map m, int j, int Hkv, int kvh, int Dh) {
  if (!m.page_table) return ((long)j * Hkv + kvh) * Dh;
  return paged_row(m.page_table, m.page_size, j, Hkv, kvh, Dh);
}

static void prefill_rows(const float* q, const uint16_t* kc, const uint16_t* vc, kv_map map,
                         float* out, int Tq, int Hq, int Hkv, int Dh, int pos0, float scale,
                         long pair_begin, long pair_end) {
  (void)Tq;
  const int group = Hq / Hkv;
  float* acc = (float*)malloc(sizeof(float) * (size_t)Dh);
  for (long pair = pair_begin; pair < pair_end; ++pair) {
    const int t = (int)(pair / Hq);
    const int h = (int)(pair % Hq);
    const int kvh = h / group;
    const float* qrow = q + ((size_t)t * Hq + h) * Dh;
    float m = -1e30f, l = 0.0f;
    for (int d = 0; d < Dh; ++d) acc[d] = 0.0f;
    const int jmax = pos0 + t;
    for (int j = 0; j <= jmax; ++j) {
      const long r = kv_row(map, j, Hkv, kvh, Dh);
      float dot = 0.0f;
      for (int d = 0; d < Dh; ++d) dot += qrow[d] * orc_bf16_to_f32(kc[r + d]);
      const float score = dot * scale;
      const float nm = fmaxf(m, score);
      const float corr = expf(m - nm);
      const float p = expf(score - nm);
      l = l * corr + p;
      for (int d = 0; d < Dh; ++d) acc[d] = acc[d] * corr + p * orc_bf16_to_f32(vc[r + d]);
      m = nm;
    }
    const float invl = (l > 0.0f) ? 1.0f / l : 0.0f;
    float* orow = out + ((size_t)t * Hq + h) * Dh;
    for (int d = 0; d < Dh; ++d) orow[d] = acc[d] * invl;
  }
  free(acc);
}

void orc_gqa_prefill(const float* q, const uint16_t* kc, const uint16_t* vc, float* out, int Tq,
                     int Hq, int Hkv, int Dh, int pos0, float scale) {
  kv_map map = {NULL, 0};
  prefill_rows(q, kc, vc, map, out, Tq, Hq, Hkv, Dh, pos0, scale, 0, (long)Tq * Hq);
}

void orc_gqa_prefill_paged(const float* q, const uint16_t* kpool, const uint16_t* vpool,
                           const int* page_table, int page_size, float* out, int Tq, int Hq,
                           int Hkv, int Dh, int pos0, float scale) {
  kv_map map = {page_table, page_size};
  prefill_rows(q, kpool, vpool, map, out, Tq, Hq, Hkv, Dh, pos0, scale, 0, (long)Tq * Hq);
}

/* ------------------------------------------------------------------------- */
/* a6 decode attention -- src/model/asr_text_decoder.cu:149-213               */
/* S = pos+1 keys; pass 1 scores = scale*dot; max; e = expf(s-max); sum;      */
/* pass 2 out[d] = (sum_j e_j v_j[d]) * (1/sum).                              */
/* ------------------------------------------------------------------------- */
static void decode_head(const float* qh, const uint16_t* kc, const uint16_t* vc, kv_map map,
                        float* oh, int S, int Hkv, int kvh, int Dh, float scale, float* sc) {
  for (int j = 0; j < S; ++j) {
    const long r = kv_row(map, j, Hkv, kvh, Dh);
    float dot = 0.0f;
    for (int e = 0; e < Dh; ++e) dot += qh[e] * orc_bf16_to_f32(kc[r + e]);
    sc[j] = dot * scale;
  }
  float m = -1e30f;
  for (int j = 0; j < S; ++j) m = fmaxf(m, sc[j]);
  float sum = 0.0f;
  for (int j = 0; j < S; ++j) {
    sc[j] = expf(sc[j] - m);
    sum += sc[j];
  }
  const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  /* Per output dim the sum still runs over j in order; j is the outer loop only so
   * each V row is read once. */
  for (int d = 0; d < Dh; ++d) oh[d] = 0.0f;
  for (int j = 0; j < S; ++j) {
    const uint16_t* vr = vc + kv_row(map, j, Hkv, kvh, Dh);
    for (int d = 0; d < Dh; ++d) oh[d] += sc[j] * orc_bf16_to_f32(vr[d]);
  }
  for (int d = 0; d < Dh; ++d) oh[d] *= inv;
}

void orc_gqa_decode(const float* q, const uint16_t* kc, const uint16_t* vc, float* out, int Hq,
                    int Hkv, int Dh, int pos, float scale) {
  kv_map map = {NULL, 0};
  const int S = pos + 1;
  float* sc = (float*)malloc(sizeof(float) * (size_t)S);
  const int group = Hq / Hkv;
  for (int h = 0; h < Hq; ++h)
    decode_head(q + (size_t)h * Dh, kc, vc, map, out + (size_t)h * Dh, S, Hkv, h / group, Dh,
                scale, sc);
  free(sc);
}

typedef struct {
  const float* q;
  const uint16_t* kpool;
  const uint16_t* vpool;
  const int* page_table;
  int max_pages, page_size;
  const int* pos;
  float* out;
  int B, Hq, Hkv, Dh;
  float scale;
  long begin, end; /* (b, h) pair range */
} decode_job;

static void* decode_worker(void* arg) {
  decode_job* jb = (decode_job*)arg;
  const int group = jb->Hq / jb->Hkv;
  int max_s = 1;
  for (int b = 0; b < jb->B; ++b)
    if (jb->pos[b] + 1 > max_s) max_s = jb->pos[b] + 1;
  float* sc = (float*)malloc(sizeof(float) * (size_t)max_s);
  for (long pair = jb->begin; pair < jb->end; ++pair) {
    const int b = (int)(pair / jb->Hq);
    const int h = (int)(pair % jb->Hq);
    kv_map map = {jb->page_table + (size_t)b * jb->max_pages, jb->page_size};
    const size_t off = ((size_t)b * jb->Hq + h) * jb->Dh;
    decode_head(jb->q + off, jb->kpool, jb->vpool, map, jb->out + off, jb->pos[b] + 1, jb->Hkv,
                h / group, jb->Dh, jb->scale, sc);
  }
  free(sc);
  return NULL;
}

void orc_gqa_decode_paged_mt(const float* q, const uint16_t* kpool, const uint16_t* vpool,
                             const int* page_table, int max_pages, int page_size, const int* pos,
                             float* out, int B, int Hq, int Hkv, int Dh, float scale,
                             int n_threads) {
  const long pairs = (long)B * Hq;
  if (n_threads < 1) n_threads = 1;
  if (n_threads > pairs) n_threads = (int)pairs;
  decode_job* jobs = (decode_job*)calloc((size_t)n_threads, sizeof(decode_job));
  pthread_t* th = (pthread_t*)calloc((size_t)n_threads, sizeof(pthread_t));
  for (int i = 0; i < n_threads; ++i) {
    decode_job j = {q, kpool, vpool, page_table, max_pages, page_size, pos, out,
                    B, Hq, Hkv, Dh, scale, pairs * i / n_threads, pairs * (i + 1) / n_threads};
    jobs[i] = j;
  }
  if (n_threads == 1) {
    decode_worker(&jobs[0]);
  } else {
    for (int i = 0; i < n_threads; ++i) pthread_create(&th[i], NULL, decode_worker, &jobs[i]);
    for (int i = 0; i < n_threads; ++i) pthread_join(th[i], NULL);
  }
  free(jobs);
  free(th);
}

void orc_gqa_decode_paged(const float* q, const uint16_t* kpool, const uint16_t* vpool,
                          const int* page_table, int max_pages, int page_size, const int* pos,
                          float* out, int B, int Hq, int Hkv, int Dh, float scale) {
  orc_gqa_decode_paged_mt(q, kpool, vpool, page_table, max_pages, page_size, pos, out, B, Hq,
                          Hkv, Dh, scale, 1);
}

typedef struct {
  const float* q;
  const uint16_t* kc;
  const uint16_t* vc;
  float* out;
  int Tq, Hq, Hkv, Dh, pos0;
  float scale;
  long begin, end;
} prefill_job;

/* begin = thread index, end = thread count: pairs are dealt round-robin. */
static void* prefill_worker(void* arg) {
  prefill_job* jb = (prefill_job*)arg;
  kv_map map = {NULL, 0};
  const long pairs = (long)jb->Tq * jb->Hq;
  for (long pair = jb->begin; pair < pairs; pair += jb->end)
    prefill_rows(jb->q, jb->kc, jb->vc, map, jb->out, jb->Tq, jb->Hq, jb->Hkv, jb->Dh, jb->pos0,
                 jb->scale, pair, pair + 1);
  return NULL;
}

void orc_gqa_prefill_mt(const float* q, const uint16_t* kc, const uint16_t* vc, float* out,
                        int Tq, int Hq, int Hkv, int Dh, int pos0, float scale, int n_threads) {
  const long pairs = (long)Tq * Hq;
  if (n_threads < 1) n_threads = 1;
  if (n_threads > pairs) n_threads = (int)pairs;
  prefill_job* jobs = (prefill_job*)calloc((size_t)n_threads, sizeof(prefill_job));
  pthread_t* th = (pthread_t*)calloc((size_t)n_threads, sizeof(pthread_t));
  /* Causal rows grow with t: deal pairs round-robin so each thread gets early and late rows. */
  for (int i = 0; i < n_threads; ++i) {
    prefill_job j = {q, kc, vc, out, Tq, Hq, Hkv, Dh, pos0, scale, i, n_threads};
    jobs[i] = j;
  }
  if (n_threads == 1) {
    prefill_worker(&jobs[0]);
  } else {
    for (int i = 0; i < n_threads; ++i) pthread_create(&th[i], NULL, prefill_worker, &jobs[i]);
    for (int i = 0; i < n_threads; ++i) pthread_join(th[i], NULL);
  }
  free(jobs);
  free(th);
}

/* ------------------------------------------------------------------------- */
/* a7 fp32 GQA self-attention -- src/model/asr_ops.cu:130-195, 252-295         */
/* ------------------------------------------------------------------------- */
void orc_gqa_attention(const float* q, const float* k, const float* v, float* out, int T, int Hq,
                       int Hkv, int Dh, float scale, int causal) {
  const int group = Hq / Hkv;
  float* acc = (float*)malloc(sizeof(float) * (size_t)Dh);
  for (int i = 0; i < T; ++i)
    for (int h = 0; h < Hq; ++h) {
      const int kvh = h / group;
      const float* qrow = q + ((size_t)i * Hq + h) * Dh;
      float m = -1e30f, l = 0.0f;
      for (int d = 0; d < Dh; ++d) acc[d] = 0.0f;
      const int jmax = causal ? i : (T - 1);
      for (int j = 0; j <= jmax; ++j) {
        const float* krow = k + ((size_t)j * Hkv + kvh) * Dh;
        const float* vrow = v + ((size_t)j * Hkv + kvh) * Dh;
        float dot = 0.0f;
        for (int d = 0; d < Dh; ++d) dot += qrow[d] * krow[d];
        const float score = dot * scale;
        const float nm = fmaxf(m, score);
        const float corr = expf(m - nm);
        const float p = expf(score - nm);
        l = l * corr + p;
        for (int d = 0; d < Dh; ++d) acc[d] = acc[d] * corr + p * vrow[d];
        m = nm;
      }
      const float invl = (l > 0.0f) ? 1.0f / l : 0.0f;
      float* orow = out + ((size_t)i * Hq + h) * Dh;
      for (int d = 0; d < Dh; ++d) orow[d] = acc[d] * invl;
    }
  free(acc);
}

void orc_attention_f64(const float* q, const float* k, const float* v, double* out, int T, int S,
                       int Hq, int Hkv, int Dh, int kv_off, double scale, int causal) {
  const int group = Hq / Hkv;
  double* sc = (double*)malloc(sizeof(double) * (size_t)(S > 0 ? S : 1));
  for (int t = 0; t < T; ++t)
    for (int h = 0; h < Hq; ++h) {
      const int kvh = h / group;
      const float* qrow = q + ((size_t)t * Hq + h) * Dh;
      int n = causal ? kv_off + t + 1 : S;
      if (n > S) n = S;
      double m = -INFINITY;
      for (int j = 0; j < n; ++j) {
        const float* krow = k + ((size_t)j * Hkv + kvh) * Dh;
        double dot = 0.0;
        for (int d = 0; d < Dh; ++d) dot += (double)qrow[d] * (double)krow[d];
        sc[j] = dot * scale;
        if (sc[j] > m) m = sc[j];
      }
      double sum = 0.0;
      for (int j = 0; j < n; ++j) {
        sc[j] = exp(sc[j] - m);
        sum += sc[j];
      }
      double* orow = out + ((size_t)t * Hq + h) * Dh;
      for (int d = 0; d < Dh; ++d) {
        double acc = 0.0;
        for (int j = 0; j < n; ++j) acc += sc[j] * (double)v[((size_t)j * Hkv + kvh) * Dh + d];
        orow[d] = n > 0 ? acc / sum : 0.0;
      }
    }
  free(sc);
}

/* ------------------------------------------------------------------------- */
/* a12 BuildPosEmb -- src/model/conformer_layer.cu:314-329                    */
/* Float arithmetic throughout, as the C++ float overloads of std::exp/log/   */
/* sin/cos evaluate it.                                                       */
/* ------------------------------------------------------------------------- */
void orc_build_pos_emb(int T, int d_model, float* pe) {
  const int P = 2 * T - 1;
  for (int idx = 0; idx < P; ++idx) {
    const float pos = (float)(T - 1 - idx);
    for (int i = 0; i < d_model; i += 2) {
      const float div = expf(-(logf(10000.0f)) * (float)i / (float)d_model);
      pe[(size_t)idx * d_model + i] = sinf(pos * div);
      if (i + 1 < d_model) pe[(size_t)idx * d_model + i + 1] = cosf(pos * div);
    }
  }
}

/* ------------------------------------------------------------------------- */
/* a11 rel-pos MHSA -- src/model/conformer_layer.cu:86-205, 387-448           */
/* ------------------------------------------------------------------------- */

/* RelShiftScoresKernel index map (src/model/conformer_layer.cu:144-153). */
int orc_relshift_column(int T, int i, int j, int* row_out) {
  const int P = 2 * T - 1;
  const long idx = (long)T + (long)i * P + j;
  const int ip = (int)(idx / (2 * T));
  const int c2 = (int)(idx % (2 * T));
  if (row_out) *row_out = ip;
  return c2 != 0 ? c2 - 1 : -1;
}

void orc_relpos_attention(const float* q, const float* k, const float* v, const float* p,
                          const float* u, const float* vb, float* out, int T, int H, int Dk,
                          int valid, float scale) {
  const int P = 2 * T - 1;
  float* qu = (float*)malloc(sizeof(float) * (size_t)Dk);
  float* qv = (float*)malloc(sizeof(float) * (size_t)Dk);
  float* bd = (float*)malloc(sizeof(float) * (size_t)T * P);
  float* row = (float*)malloc(sizeof(float) * (size_t)T);
  for (int h = 0; h < H; ++h) {
    /* BD[h,i,m] = (q_i + v_h) . p_m for every m (the batched SGEMM at :433). */
    for (int i = 0; i < T; ++i) {
      for (int d = 0; d < Dk; ++d) qv[d] = q[((size_t)i * H + h) * Dk + d] + vb[h * Dk + d];
      for (int m = 0; m < P; ++m) {
        float acc = 0.0f;
        for (int d = 0; d < Dk; ++d) acc += qv[d] * p[((size_t)m * H + h) * Dk + d];
        bd[(size_t)i * P + m] = acc;
      }
    }
    for (int i = 0; i < T; ++i) {
      for (int d = 0; d < Dk; ++d) qu[d] = q[((size_t)i * H + h) * Dk + d] + u[h * Dk + d];
      /* scores: (AC + rel_shift(BD)) * scale, keys j >= valid -> -1e30 (:130-155) */
      for (int j = 0; j < T; ++j) {
        if (j >= valid) {
          row[j] = -1e30f;
          continue;
        }
        float ac = 0.0f;
        for (int d = 0; d < Dk; ++d) ac += qu[d] * k[((size_t)j * H + h) * Dk + d];
        int ip;
        const int m = orc_relshift_column(T, i, j, &ip);
        const float bdv = m >= 0 ? bd[(size_t)ip * P + m] : 0.0f;
        row[j] = (ac + bdv) * scale;
      }
      /* row softmax (:158-192) */
      float mx = -1e30f;
      for (int j = 0; j < T; ++j) mx = fmaxf(mx, row[j]);
      float sum = 0.0f;
      for (int j = 0; j < T; ++j) {
        row[j] = expf(row[j] - mx);
        sum += row[j];
      }
      const float inv = 1.0f / sum;
      for (int j = 0; j < T; ++j) row[j] *= inv;
      /* ctx = P.V (:440-442), scattered back to [T,H,Dk] (:195-205) */
      for (int d = 0; d < Dk; ++d) {
        float acc = 0.0f;
        for (int j = 0; j < T; ++j) acc += row[j] * v[((size_t)j * H + h) * Dk + d];
        out[((size_t)i * H + h) * Dk + d] = acc;
      }
    }
  }
  free(qu);
  free(qv);
  free(bd);
  free(row);
}

void orc_relpos_attention_f64(const float* q, const float* k, const float* v, const float* p,
                              const float* u, const float* vb, double* out, int T, int H, int Dk,
                              int valid, double scale) {
  double* row = (double*)malloc(sizeof(double) * (size_t)T);
  for (int h = 0; h < H; ++h)
    for (int i = 0; i < T; ++i) {
      double mx = -INFINITY;
      for (int j = 0; j < T; ++j) {
        if (j >= valid) {
          row[j] = -INFINITY;
          continue;
        }
        const float* pm = p + ((size_t)(T - 1 - i + j) * H + h) * Dk;
        double s = 0.0;
        for (int d = 0; d < Dk; ++d) {
          const double qd = q[((size_t)i * H + h) * Dk + d];
          s += (qd + u[h * Dk + d]) * (double)k[((size_t)j * H + h) * Dk + d] +
               (qd + vb[h * Dk + d]) * (double)pm[d];
        }
        row[j] = s * scale;
        if (row[j] > mx) mx = row[j];
      }
      double sum = 0.0;
      for (int j = 0; j < T; ++j) {
        row[j] = j < valid ? exp(row[j] - mx) : 0.0;
        sum += row[j];
      }
      for (int d = 0; d < Dk; ++d) {
        double acc = 0.0;
        for (int j = 0; j < T; ++j) acc += row[j] * (double)v[((size_t)j * H + h) * Dk + d];
        out[((size_t)i * H + h) * Dk + d] = acc / sum;
      }
    }
  free(row);
}

/* ------------------------------------------------------------------------- */
/* a13 SGEMM -- include/model/gemm.cuh:40-45 (ApplyAct), 47-158, 181-268       */
/* out[m,n] = act(sum_k in[m,k]*W[n,k] (+ bias[n])), fp32 k-sequential.        */
/* ------------------------------------------------------------------------- */
static float apply_act(float v, int act) {
  if (act == 1) return v / (1.0f + expf(-v));
  if (act == 2) return fmaxf(v, 0.0f);
  if (act == 3) return 1.0f / (1.0f + expf(-v));
  return v;
}

void orc_sgemm(const float* in, const float* W, const float* bias, float* out, int M, int K,
               int N, int act) {
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n) {
      float acc = 0.0f;
      for (int kk = 0; kk < K; ++kk) acc += in[(size_t)m * K + kk] * W[(size_t)n * K + kk];
      if (bias) acc += bias[n];
      out[(size_t)m * N + n] = apply_act(acc, act);
    }
}

void orc_sgemm_batched(const float* in, const float* W, float* out, int M, int K, int N, int act,
                       int batch, long stride_in, long stride_w, long stride_out) {
  for (int b = 0; b < batch; ++b)
    orc_sgemm(in + b * stride_in, W + b * stride_w, NULL, out + b * stride_out, M, K, N, act);
}

/* WindowAttnKernel (src/model/asr_audio_tower.cu:204-258): per (query i, head h) an online
 * softmax over keys j in [seg_start[i], seg_end[i]): m starts at -1e30, score = (q.k) * scale
 * with the dot in dimension order, corr = exp(m - nm), p = exp(score - nm), l = l corr + p,
 * acc = acc corr + p v; out = acc / l, or 0 when l == 0. */
void orc_window_attention(const float* q, const float* k, const float* v, float* out,
                          const int* seg_start, const int* seg_end, int N, int H, int Dh,
                          float scale) {
  float* acc = (float*)malloc(sizeof(float) * (size_t)Dh);
  for (int i = 0; i < N; ++i)
    for (int h = 0; h < H; ++h) {
      const float* qr = q + ((size_t)i * H + h) * Dh;
      float m = -1e30f, l = 0.0f;
      for (int d = 0; d < Dh; ++d) acc[d] = 0.0f;
      for (int j = seg_start[i]; j < seg_end[i]; ++j) {
        const float* kr = k + ((size_t)j * H + h) * Dh;
        const float* vr = v + ((size_t)j * H + h) * Dh;
        float dot = 0.0f;
        for (int d = 0; d < Dh; ++d) dot += qr[d] * kr[d];
        const float score = dot * scale;
        const float nm = score > m ? score : m;
        const float corr = expf(m - nm);
        const float p = expf(score - nm);
        l = l * corr + p;
        for (int d = 0; d < Dh; ++d) acc[d] = acc[d] * corr + p * vr[d];
        m = nm;
      }
      const float invl = l > 0.0f ? 1.0f / l : 0.0f;
      float* o = out + ((size_t)i * H + h) * Dh;
      for (int d = 0; d < Dh; ++d) o[d] = acc[d] * invl;
    }
  free(acc);
}

/* Sortformer decoder MHA as the reference decomposes it (src/model/sortformer_decoder.cu:
 * 280-298): raw[h,i,j] = sum_d q.k in d order (the batched SGEMM), s = j >= valid ? -1e30 :
 * raw * scale (:114-123), row max, e = exp(s - max), sum in j order, p = e * (1 / sum)
 * (:126-160), ctx[i,h,d] = sum_j p v in j order (the PV SGEMM).  The reference's __expf is
 * the fast exponential; this restatement uses expf. */
void orc_masked_mha(const float* q, const float* k, const float* v, float* out, int T, int H,
                    int Dk, int valid, float scale) {
  float* s = (float*)malloc(sizeof(float) * (size_t)T);
  for (int h = 0; h < H; ++h)
    for (int i = 0; i < T; ++i) {
      const float* qr = q + ((size_t)i * H + h) * Dk;
      float mx = -1e30f;
      for (int j = 0; j < T; ++j) {
        const float* kr = k + ((size_t)j * H + h) * Dk;
        float raw = 0.0f;
        for (int d = 0; d < Dk; ++d) raw += qr[d] * kr[d];
        s[j] = j >= valid ? -1e30f : raw * scale;
        if (s[j] > mx) mx = s[j];
      }
      float sum = 0.0f;
      for (int j = 0; j < T; ++j) {
        s[j] = expf(s[j] - mx);
        sum += s[j];
      }
      const float inv = 1.0f / sum;
      for (int j = 0; j < T; ++j) s[j] *= inv;
      float* o = out + ((size_t)i * H + h) * Dk;
      for (int d = 0; d < Dk; ++d) {
        float acc = 0.0f;
        for (int j = 0; j < T; ++j) acc += s[j] * v[((size_t)j * H + h) * Dk + d];
        o[d] = acc;
      }
    }
  free(s);
}

/* LayerNormKernel (src/model/conformer_layer.cu:28-66): mean, mean square deviation,
 * inv = 1 / sqrt(var + eps), y = (x - mean) inv g + b, per row of C. */
void orc_layer_norm(const float* x, const float* g, const float* b, float* y, int T, int C,
                    float eps) {
  for (int t = 0; t < T; ++t) {
    const float* xr = x + (size_t)t * C;
    float* yr = y + (size_t)t * C;
    float s = 0.0f;
    for (int c = 0; c < C; ++c) s += xr[c];
    const float mean = s / (float)C;
    float sq = 0.0f;
    for (int c = 0; c < C; ++c) sq += (xr[c] - mean) * (xr[c] - mean);
    const float inv = 1.0f / sqrtf(sq / (float)C + eps);
    for (int c = 0; c < C; ++c) yr[c] = (xr[c] - mean) * inv * g[c] + b[c];
  }
}

/* GluKernel (:207-215) + MaskRowsKernel (:78-83): out[t,c] = a sigmoid(b) for t < valid,
 * else 0; in [T, 2C] = a | b. */
void orc_glu_mask(const float* in, float* out, int T, int C, int valid) {
  for (int t = 0; t < T; ++t)
    for (int c = 0; c < C; ++c) {
      const float a = in[(size_t)t * 2 * C + c], b = in[(size_t)t * 2 * C + C + c];
      out[(size_t)t * C + c] = t < valid ? a * (1.0f / (1.0f + expf(-b))) : 0.0f;
    }
}

/* DepthwiseConvKernel (:218-233) + BatchNormSiluKernel (:236-246). */
void orc_dwconv_bn_silu(const float* in, const float* w, const float* bias, const float* mean,
                        const float* var, const float* gamma, const float* beta, float* out,
                        int T, int C, int K, float eps) {
  const int pad = (K - 1) / 2;
  for (int t = 0; t < T; ++t)
    for (int c = 0; c < C; ++c) {
      float acc = bias ? bias[c] : 0.0f;
      for (int k = 0; k < K; ++k) {
        const int ti = t + k - pad;
        if (ti >= 0 && ti < T) acc += in[(size_t)ti * C + c] * w[(size_t)c * K + k];
      }
      const float y = (acc - mean[c]) * (1.0f / sqrtf(var[c] + eps)) * gamma[c] + beta[c];
      out[(size_t)t * C + c] = y / (1.0f + expf(-y));
    }
}

/* asr_gemm::LinearPre (src/model/asr_gemm.cu:175-208; kernels :62-155): out[m,n] =
 * act(sum_k bf16(in[m,k]) bf16(W[n,k]) + bias[n]), fp32 accumulation in k order; act 0 none,
 * 1 exact-erf GELU 0.5 v (1 + erf(v / sqrt 2)) (:93-94), 2 ReLU (:95-96). */
static float linear_act(float v, int act) {
  if (act == 1) return 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f));
  if (act == 2) return v > 0.0f ? v : 0.0f;
  return v;
}

/* Blocked over independent outputs only (LM rows x LN columns share each k step); every
 * output is still one fp32 chain, acc += x[k] * w[k] for k = 0, 1, ..., K-1 with no
 * contraction, so the bits equal the plain triple loop (tests/test_oracle.py checks). */
enum { LM = 4, LN = 4, LN1 = 16 };
/* M = 1 (decode GEMV): LN1 columns per k step, same per-output chain. */
static void linear_bf16_row(const uint16_t* in, const uint16_t* W, const float* bias, float* out,
                            int K, int N, int act) {
  float* xs = (float*)malloc(sizeof(float) * (size_t)K);
  float* ws = (float*)malloc(sizeof(float) * (size_t)K * LN1);
  for (int kk = 0; kk < K; ++kk) xs[kk] = orc_bf16_to_f32(in[kk]);
  for (int n0 = 0; n0 < N; n0 += LN1) {
    const int nb = N - n0 < LN1 ? N - n0 : LN1;
    for (int j = 0; j < LN1; ++j) {
      const uint16_t* wr = W + (size_t)(n0 + (j < nb ? j : nb - 1)) * K;
      for (int kk = 0; kk < K; ++kk) ws[(size_t)kk * LN1 + j] = orc_bf16_to_f32(wr[kk]);
    }
    float acc[LN1];
    for (int j = 0; j < LN1; ++j) acc[j] = 0.0f;
    for (int kk = 0; kk < K; ++kk) {
      const float x = xs[kk];
      const float* w = ws + (size_t)kk * LN1;
      for (int j = 0; j < LN1; ++j) acc[j] += x * w[j];
    }
    for (int j = 0; j < nb; ++j) {
      float v = acc[j];
      if (bias) v += bias[n0 + j];
      out[n0 + j] = linear_act(v, act);
    }
  }
  free(xs);
  free(ws);
}

void orc_linear_bf16(const uint16_t* in, const uint16_t* W, const float* bias, float* out, int M,
                     int K, int N, int act) {
  if (M == 1) {
    linear_bf16_row(in, W, bias, out, K, N, act);
    return;
  }
  const int mblocks = (M + LM - 1) / LM;
  /* xs[mb][k][i] = row LM*mb+i widened (rows past M repeat the last row; never stored) */
  float* xs = (float*)malloc(sizeof(float) * (size_t)mblocks * K * LM);
  float* ws = (float*)malloc(sizeof(float) * (size_t)K * LN);
  for (int mb = 0; mb < mblocks; ++mb)
    for (int kk = 0; kk < K; ++kk)
      for (int i = 0; i < LM; ++i) {
        int m = LM * mb + i;
        if (m >= M) m = M - 1;
        xs[((size_t)mb * K + kk) * LM + i] = orc_bf16_to_f32(in[(size_t)m * K + kk]);
      }
  for (int n0 = 0; n0 < N; n0 += LN) {
    const int nb = N - n0 < LN ? N - n0 : LN;
    for (int kk = 0; kk < K; ++kk)
      for (int j = 0; j < LN; ++j)
        ws[(size_t)kk * LN + j] = orc_bf16_to_f32(W[(size_t)(n0 + (j < nb ? j : nb - 1)) * K + kk]);
    for (int mb = 0; mb < mblocks; ++mb) {
      float acc[LM][LN];
      for (int i = 0; i < LM; ++i)
        for (int j = 0; j < LN; ++j) acc[i][j] = 0.0f;
      const float* xb = xs + (size_t)mb * K * LM;
      for (int kk = 0; kk < K; ++kk) {
        const float* x = xb + (size_t)kk * LM;
        const float* w = ws + (size_t)kk * LN;
        for (int i = 0; i < LM; ++i)
          for (int j = 0; j < LN; ++j) acc[i][j] += x[i] * w[j];
      }
      const int m0 = LM * mb, rows = M - m0 < LM ? M - m0 : LM;
      for (int i = 0; i < rows; ++i)
        for (int j = 0; j < nb; ++j) {
          float v = acc[i][j];
          if (bias) v += bias[n0 + j];
          out[(size_t)(m0 + i) * N + n0 + j] = linear_act(v, act);
        }
    }
  }
  free(xs);
  free(ws);
}

/* ------------------------------------------------------------------------- */
/* a14 ArgmaxBanned -- src/model/asr_ops.cu:300-325                           */
/* 256 thread-strided scans with strict '>', then a halving tree that takes   */
/* the right candidate only when strictly greater: ties keep the lower thread.*/
/* ------------------------------------------------------------------------- */
int orc_argmax_banned(const float* x, int n, int ban0, int ban1) {
  enum { kThreads = 256 };
  float sval[kThreads];
  int sidx[kThreads];
  for (int t = 0; t < kThreads; ++t) {
    float best = -1e30f;
    int bi = 0;
    for (int i = t; i < n; i += kThreads) {
      if (i == ban0 || i == ban1) continue;
      if (x[i] > best) {
        best = x[i];
        bi = i;
      }
    }
    sval[t] = best;
    sidx[t] = bi;
  }
  for (int s = kThreads / 2; s > 0; s >>= 1)
    for (int t = 0; t < s; ++t)
      if (sval[t + s] > sval[t]) {
        sval[t] = sval[t + s];
        sidx[t] = sidx[t + s];
      }
  return sidx[0];
}
