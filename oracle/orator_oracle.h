/*
 * orator_oracle.h -- CPU restatement of Orator's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP kernels
 * in orator_amd/csrc.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product path never calls it and has no
 * CPU fallback.
 *
 * Every function restates one reference routine (file:line relative to the
 * thomas-hiddenpeak/Orator tree).  "Reference semantics" means the same fp32
 * operation sequence where it changes results: fp32 RoPE angle, bf16
 * round-to-nearest-even for the KV cache, online softmax starting at -1e30,
 * multiply by 1/sum.  The *_f64 functions are fp64 "truth" used to bound the
 * fp32 error of both the oracle and the GPU.
 *
 * Layouts (row-major, as in the reference):
 *   q, out           [T, Hq, Dh]   fp32
 *   k, v (fp32)      [T, Hkv, Dh]
 *   contiguous cache [S_cap, Hkv, Dh] bf16 bits (uint16)
 *   paged pool       [n_pages, page_size, Hkv, Dh] bf16 bits; page_table[b*max_pages + i]
 *   rel-pos p        [2T-1, H, Dk]; u, vb [H, Dk]
 *
 * Pinning status of each function is listed in the header of orator_oracle.c.
 */
#ifndef ORATOR_ORACLE_H_
#define ORATOR_ORACLE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bf16 (test/unit/model/test_asr_gemm.cc:21-33; src/model/asr_text_decoder.cu:75-81) ---- */
uint16_t orc_f32_to_bf16(float x);
float orc_bf16_to_f32(uint16_t b);
void orc_f32_to_bf16_n(const float* in, uint16_t* out, long n);
void orc_bf16_to_f32_n(const uint16_t* in, float* out, long n);

/* ---- a1 RMSNorm (src/model/asr_ops.cu:21-51) ---- */
void orc_rms_norm(const float* x, const float* w, float* out, int rows, int dim, float eps);

/* ---- a2/a3 RoPE (src/model/asr_ops.cu:57-75, 92-111) ---- */
float orc_rope_inv_freq(float base, int j, int head_dim);
void orc_rope_half(float* x, const int* pos, int n_tokens, int n_heads, int head_dim, float base);
void orc_rope_interleaved(float* x, const int* pos, int n_tokens, int n_heads, int head_dim,
                          float base);

/* ---- SwiGLU (src/model/asr_ops.cu:80-87) ---- */
void orc_swiglu(const float* gate, const float* up, float* out, int n);

/* ---- a4 KV write (src/model/asr_text_decoder.cu:62-77) ---- */
void orc_kv_write(const float* k, const float* v, uint16_t* kc, uint16_t* vc, int Tq, int Hkv,
                  int Dh, int pos0);
void orc_kv_write_paged(const float* k, const float* v, uint16_t* kpool, uint16_t* vpool,
                        const int* page_table, int page_size, int Tq, int Hkv, int Dh, int pos0);

/* ---- a5 prefill attention over the bf16 cache (src/model/asr_text_decoder.cu:88-142) ---- */
void orc_gqa_prefill(const float* q, const uint16_t* kc, const uint16_t* vc, float* out, int Tq,
                     int Hq, int Hkv, int Dh, int pos0, float scale);
void orc_gqa_prefill_paged(const float* q, const uint16_t* kpool, const uint16_t* vpool,
                           const int* page_table, int page_size, float* out, int Tq, int Hq,
                           int Hkv, int Dh, int pos0, float scale);

/* ---- a6 decode attention (src/model/asr_text_decoder.cu:149-213) ---- */
void orc_gqa_decode(const float* q, const uint16_t* kc, const uint16_t* vc, float* out, int Hq,
                    int Hkv, int Dh, int pos, float scale);
/* Batched paged decode: stream b attends pos[b]+1 keys through its page-table row. */
void orc_gqa_decode_paged(const float* q, const uint16_t* kpool, const uint16_t* vpool,
                          const int* page_table, int max_pages, int page_size, const int* pos,
                          float* out, int B, int Hq, int Hkv, int Dh, float scale);
/* Same as orc_gqa_decode_paged with the (stream, q-head) pairs spread over n_threads pthreads. */
void orc_gqa_decode_paged_mt(const float* q, const uint16_t* kpool, const uint16_t* vpool,
                             const int* page_table, int max_pages, int page_size, const int* pos,
                             float* out, int B, int Hq, int Hkv, int Dh, float scale,
                             int n_threads);
/* Prefill with (q-head, query-row) work spread over n_threads pthreads. */
void orc_gqa_prefill_mt(const float* q, const uint16_t* kc, const uint16_t* vc, float* out,
                        int Tq, int Hq, int Hkv, int Dh, int pos0, float scale, int n_threads);

/* ---- a7 fp32 GQA self-attention (src/model/asr_ops.cu:130-195, 252-295) ---- */
void orc_gqa_attention(const float* q, const float* k, const float* v, float* out, int T, int Hq,
                       int Hkv, int Dh, float scale, int causal);

/* fp64 truth: general GQA attention over fp32 K/V given as float arrays, query row t
 * attends keys [0, kv_off + t] when causal, else [0, S).  K/V: [S, Hkv, Dh]. */
void orc_attention_f64(const float* q, const float* k, const float* v, double* out, int T, int S,
                       int Hq, int Hkv, int Dh, int kv_off, double scale, int causal);

/* ---- a11/a12 Conformer rel-pos MHSA (src/model/conformer_layer.cu:86-205, 314-329, 387-448) ---- */
void orc_build_pos_emb(int T, int d_model, float* pe);
/* Reference decomposition: AC, full BD [H,T,2T-1], RelShiftScores index formula, softmax, PV. */
void orc_relpos_attention(const float* q, const float* k, const float* v, const float* p,
                          const float* u, const float* vb, float* out, int T, int H, int Dk,
                          int valid, float scale);
/* fp64 truth using the closed form BD[h,i,T-1-i+j] (no full BD). */
void orc_relpos_attention_f64(const float* q, const float* k, const float* v, const float* p,
                              const float* u, const float* vb, double* out, int T, int H, int Dk,
                              int valid, double scale);
/* The rel_shift index map of RelShiftScoresKernel: returns the BD column m used for
 * score (i, j), or -1 when the reference substitutes 0. */
int orc_relshift_column(int T, int i, int j, int* row_out);

/* ---- a13 SGEMM (include/model/gemm.cuh:40-45, 47-158, 181-268) ---- */
void orc_sgemm(const float* in, const float* W, const float* bias, float* out, int M, int K,
               int N, int act);
void orc_sgemm_batched(const float* in, const float* W, float* out, int M, int K, int N, int act,
                       int batch, long stride_in, long stride_w, long stride_out);

/* ---- Conformer non-attention passes (src/model/conformer_layer.cu:28-83,207-246) ---- */
void orc_layer_norm(const float* x, const float* g, const float* b, float* y, int T, int C,
                    float eps);
void orc_glu_mask(const float* in, float* out, int T, int C, int valid);
void orc_dwconv_bn_silu(const float* in, const float* w, const float* bias, const float* mean,
                        const float* var, const float* gamma, const float* beta, float* out,
                        int T, int C, int K, float eps);

/* ---- Sortformer decoder MHA (src/model/sortformer_decoder.cu:280-298) ---- */
void orc_masked_mha(const float* q, const float* k, const float* v, float* out, int T, int H,
                    int Dk, int valid, float scale);

/* ---- WindowAttnKernel (src/model/asr_audio_tower.cu:204-258) ---- */
void orc_window_attention(const float* q, const float* k, const float* v, float* out,
                          const int* seg_start, const int* seg_end, int N, int H, int Dh,
                          float scale);

/* ---- asr_gemm::LinearPre (src/model/asr_gemm.cu:175-208): bf16 in/W, fp32 accumulate ---- */
void orc_linear_bf16(const uint16_t* in, const uint16_t* W, const float* bias, float* out, int M,
                     int K, int N, int act);

/* ---- a14 ArgmaxBanned (src/model/asr_ops.cu:300-333) ---- */
int orc_argmax_banned(const float* x, int n, int ban0, int ban1);

#ifdef __cplusplus
}
#endif
#endif /* ORATOR_ORACLE_H_ */
