/*
 * orator_attn.h -- C ABI of the MI355X (gfx950) attention hot path.
 *
 * Every entry point takes plain device pointers and sizes, a HIP stream passed as
 * `void*` (NULL = the default stream) and returns an int status (ORATOR_OK = 0).
 * On failure orator_last_error() returns a message for the calling thread.
 *
 * Conventions carried over from the reference launchers:
 *   - non-positive sizes are a silent no-op returning ORATOR_OK
 *     (src/model/asr_ops.cu:201,208,220,227,254,330);
 *   - launches are asynchronous on the given stream; RopeInterleaved and
 *     GqaAttention use the default stream, as the reference's do
 *     (src/model/asr_ops.cu:213,246-247);
 *   - positions are device-resident ints so a captured graph can replay at any
 *     position (src/model/asr_text_decoder.cu:60-61,159);
 *   - the caller owns every buffer; in-place use is allowed where the reference
 *     allows it (include/model/asr_ops.cuh:23,37).
 * New here: shapes the kernels do not support, and capacity overruns the host can
 * see, are rejected before launch with ORATOR_ERR_UNSUPPORTED / _CAPACITY.
 *
 * Layouts: q/out [T, Hq, Dh] fp32; k/v [T, Hkv, Dh]; a KV cache is bf16 bits
 * (uint16_t) [rows, Hkv, Dh].  A paged pool is [n_pages, page_size, Hkv, Dh] with
 * page_table[b * max_pages + i] naming the page that holds positions
 * [i*page_size, (i+1)*page_size) of stream b; contiguous pages in order are
 * exactly the reference layout [max_seq_len, Hkv, Dh]
 * (src/model/asr_text_decoder.cu:60-77,309-318).
 */
#ifndef ORATOR_ATTN_H_
#define ORATOR_ATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORATOR_OK 0
#define ORATOR_ERR_INVALID (-1)     /* bad argument (null pointer, inconsistent sizes)   */
#define ORATOR_ERR_UNSUPPORTED (-2) /* shape outside what the kernels are built for      */
#define ORATOR_ERR_CAPACITY (-3)    /* request exceeds a cache / workspace capacity      */
#define ORATOR_ERR_HIP (-4)         /* HIP runtime error                                  */

/* ---------------------------------------------------------------- runtime ---- */
/* Message for the last failing call on this thread ("" if none). */
const char* orator_last_error(void);
int orator_version(void);
/* Device plumbing for hosts without their own HIP code (tests, bench).  Mirrors the
 * reference's gpu runtime (include/gpu/memory.h:26-168, src/gpu/memory.cc:139-147). */
int orator_device_count(int* count);
int orator_set_device(int device);
int orator_device_name(char* buf, int len);
int orator_malloc(void** ptr, size_t bytes);
int orator_free(void* ptr);
int orator_memcpy_htod(void* dst, const void* src, size_t bytes);
int orator_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int orator_memcpy_dtod(void* dst, const void* src, size_t bytes, void* stream);
int orator_memset(void* ptr, int value, size_t bytes, void* stream);
int orator_stream_create(void** stream);
int orator_stream_destroy(void* stream);
int orator_stream_synchronize(void* stream);
int orator_device_synchronize(void);
/* Event timing: creates/records/reads hipEvents on a stream. */
int orator_event_create(void** event);
int orator_event_destroy(void* event);
int orator_event_record(void* event, void* stream);
int orator_event_elapsed_ms(float* ms, void* start, void* stop);
/* Pre-sizes the library workspace of `stream` (split-K decode partials, rel-pos fp32
 * intermediates) so that later calls do not allocate, e.g. before hipGraph capture. */
int orator_workspace_reserve(size_t bytes, void* stream);
/* Diagnostics (no reference counterpart): the library workspace blocks currently held (current
 * and retired, every device, stream and thread) and their bytes, after freeing the retired
 * blocks whose stream work has completed.  Either pointer may be NULL. */
int orator_workspace_stats(size_t* blocks, size_t* bytes);
/* Measurement hook (this thread; no reference counterpart): the next decode call records the
 * HIP events `start` before its split kernel, `split_end` after it and `stop` after the split
 * merge, on the launch stream, so the operation and its split kernel can be timed without
 * host gaps.  Any event may be NULL. */
int orator_time_next_decode(void* start, void* split_end, void* stop);

/* ------------------------------------------------------- asr_ops family ---- */
/* asr_ops::RmsNorm (include/model/asr_ops.cuh:21-25; src/model/asr_ops.cu:21-51,199-204).
 * out[r,d] = x[r,d] * rsqrt(mean_d(x[r,:]^2) + eps) * weight[d]; in-place allowed. */
int orator_rms_norm(const float* x, const float* weight, float* out, int rows, int dim,
                    float eps, void* stream);
/* asr_ops::RopeInterleaved (include/model/asr_ops.cuh:27-34; src/model/asr_ops.cu:57-75,206-216).
 * Default stream, in place. */
int orator_rope_interleaved(float* x, const int* positions, int n_tokens, int n_heads,
                            int head_dim, float theta_base);
/* asr_ops::SwiGLU (include/model/asr_ops.cuh:36-39; src/model/asr_ops.cu:80-87,218-223). */
int orator_swiglu(const float* gate, const float* up, float* out, int n, void* stream);
/* asr_ops::RopeHalf (include/model/asr_ops.cuh:41-48; src/model/asr_ops.cu:92-111,225-235).
 * rotate_half RoPE in place. */
int orator_rope_half(float* x, const int* positions, int n_tokens, int n_heads, int head_dim,
                     float theta_base, void* stream);
/* asr_ops::ArgmaxBanned (include/model/asr_ops.cuh:58-62; src/model/asr_ops.cu:300-333).
 * Same tie rule: ties keep the candidate of the lower scan slot. */
int orator_argmax_banned(const float* logits, int n, int ban0, int ban1, int* out_idx,
                         void* stream);
/* asr_ops::GqaAttention (include/model/asr_ops.cuh:50-56; src/model/asr_ops.cu:130-195,252-295).
 * fp32 q [T,Hq,Dh], k/v [T,Hkv,Dh]; row i attends keys [0,i] (causal) or [0,T).  Default
 * stream.  As the reference: any power-of-two Dh <= 1024 and any Hq that is a multiple of Hkv
 * (Dh 64 / 128 with Hq/Hkv in {1,2,4} run on the split-K kernel, the rest on a generic one). */
int orator_gqa_attention(const float* q, const float* k, const float* v, float* out, int T, int Hq,
                         int Hkv, int Dh, float scale, int causal);
/* asr_gemm::F32ToBf16 / Bf16ToF32 (include/model/asr_gemm.h:23-25; src/model/asr_gemm.cu:45-57).
 * Any n; operands at their natural alignment (16-byte fp32 and 8-byte bf16 addresses take the
 * 4-wide accesses). */
int orator_f32_to_bf16(const float* in, uint16_t* out, long n, void* stream);
int orator_bf16_to_f32(const uint16_t* in, float* out, long n, void* stream);

/* ------------------------------------------------- decoder KV + attention ---- */
/* WriteKvCacheKernel (src/model/asr_text_decoder.cu:62-77): cache[pos0 + t] = bf16(k/v[t]),
 * pos0 read from *d_pos0 on the device.  New: rows at or past `capacity` are not written. */
int orator_kv_write(const float* k, const float* v, uint16_t* kc, uint16_t* vc, int Tq, int Hkv,
                    int Dh, const int* d_pos0, int capacity, void* stream);
/* Paged form: stream b's Tq rows go to positions d_pos0[b] + t through its page-table row.
 * k/v are [B, Tq, Hkv, Dh]; page indices at or past n_pages are not written. */
int orator_kv_write_paged(const float* k, const float* v, uint16_t* kpool, uint16_t* vpool,
                          const int* page_table, int max_pages, int page_size, int n_pages,
                          int B, int Tq, int Hkv, int Dh, const int* d_pos0, void* stream);

/* Fused QK-RMSNorm + RoPE + KV write: the decoder's per-layer sequence
 *   RmsNorm(q, q_norm) ; RmsNorm(k, k_norm) ; RopeHalf(q) ; RopeHalf(k) ; WriteKvCache(k, v)
 * (src/model/asr_text_decoder.cu:408-413 decode, :530-536 prefill) in one launch.  Token t
 * of q/k/v (rows q + t*q_stride, k/v + t*kv_stride, heads contiguous, Dh = 128) is
 * normalised and rotated at positions[t] in place; k and v go to the cache row of
 * positions[t] as bf16.  Cache: contiguous (page_table NULL, `capacity` rows) or paged
 * (stream = t / tokens_per_stream selects the page-table row; `capacity` = pages in the
 * pool).  Rows outside the cache are not written. */
int orator_qk_norm_rope_kv_write(float* q, float* k, const float* v, long q_stride, long kv_stride,
                                 const float* q_norm, const float* k_norm, float eps,
                                 const int* positions, float theta, int n_tokens,
                                 int tokens_per_stream, int Hq, int Hkv, int Dh, uint16_t* kpool,
                                 uint16_t* vpool, const int* page_table, int max_pages,
                                 int page_size, int capacity, void* stream);
/* The RoPE (cos, sin) of every rotate-half pair j < 64 (Dh = 128, base theta) for positions
 * [0, n_pos): out[(p * 64 + j) * 2 + {0, 1}], the values RopeHalf forms
 * (src/model/asr_ops.cu:102-109: angle = (float)p * powf(theta, -2j/128), rounded once from
 * fp64 cos/sin).  Built once per model; the decoder keeps one for its context. */
int orator_rope_table(float* out, int n_pos, float theta, void* stream);
/* orator_qk_norm_rope_kv_write reading (cos, sin) from a table of orator_rope_table holding
 * positions [0, rope_rows) instead of forming them per call (same values); positions past
 * the table form them per call. */
int orator_qk_norm_rope_kv_write_table(float* q, float* k, const float* v, long q_stride,
                                       long kv_stride, const float* q_norm, const float* k_norm,
                                       float eps, const int* positions, float theta,
                                       const float* rope, int rope_rows, int n_tokens,
                                       int tokens_per_stream, int Hq, int Hkv, int Dh,
                                       uint16_t* kpool, uint16_t* vpool, const int* page_table,
                                       int max_pages, int page_size, int capacity, void* stream);

/* GqaDecodeAttnKernel (src/model/asr_text_decoder.cu:149-213, launch :416-418):
 * q [Hq, Dh] fp32 attends the S = *d_pos + 1 keys of the bf16 cache kc/vc.
 * `capacity` (the cache's max_seq_len) sizes the split-K grid; S is clamped to it.
 * Any S is supported (the reference stops at 2048).  Any Dh in [1, 1024] and any Hq multiple
 * of Hkv (as the reference): Dh 64 / 128 with Hq/Hkv in {1,2,4} run on the split-K kernels,
 * other shapes on a generic kernel; the same holds for every decode entry point below except
 * the QK-norm folding ones (Dh 128, Hq/Hkv in {1,2,4}). */
int orator_gqa_decode(const float* q, const uint16_t* kc, const uint16_t* vc, float* out, int Hq,
                      int Hkv, int Dh, const int* d_pos, int capacity, float scale, void* stream);
/* Batched paged decode: stream b's q [Hq, Dh] attends d_pos[b] + 1 keys through page-table
 * row b.  q/out [B, Hq, Dh]. */
int orator_gqa_decode_paged(const float* q, const uint16_t* kpool, const uint16_t* vpool,
                            const int* page_table, int max_pages, int page_size,
                            const int* d_pos, float* out, int B, int Hq, int Hkv, int Dh,
                            float scale, void* stream);
/* Measurement hook (no reference counterpart): reads the K/V bytes of a paged decode over S keys
 * per stream (head_dim 128, bf16, the first ceil(S / page_size) entries of each table row
 * mapped) with the decode kernels' access pattern and nothing else, so its time is that
 * pattern's streaming ceiling.  `sink`: a 4-byte device word the kernel may write. */
int orator_decode_read_probe(const uint16_t* kpool, const uint16_t* vpool, const int* page_table,
                             int max_pages, int page_size, int S, int B, int Hkv,
                             unsigned* sink, void* stream);
/* No counterpart in the reference: orator_gqa_decode_paged for callers that cannot allocate
 * (code under HIP graph capture, serving loops that forbid hipMalloc).  Same arguments and
 * results; the split partials (and the arrival counters of the in-launch split merge, its
 * last 512 KiB) live in a static 16 MiB device array per GPU instead of the library workspace,
 * so the call allocates nothing.  Limit: B * Hq * ceil(max_pages * page_size / 128) * (Dh +
 * 2) * 4 bytes <= 16 MiB - 512 KiB (B = 16, Hq = 16, Dh = 128: 15616 keys), else
 * ORATOR_ERR_CAPACITY.  Calls that overlap on one GPU share the array and race. */
int orator_gqa_decode_paged_noalloc(const float* q, const uint16_t* kpool, const uint16_t* vpool,
                                    const int* page_table, int max_pages, int page_size,
                                    const int* d_pos, float* out, int B, int Hq, int Hkv, int Dh,
                                    float scale, void* stream);
/* The attention half of one decode step (src/model/asr_text_decoder.cu:408-418: RmsNorm of q
 * and k per head, RopeHalf of q and k, WriteKvCacheKernel, GqaDecodeAttnKernel) in one launch:
 * q [Hq, Dh] and k_new/v_new [Hkv, Dh] are the raw projections (16-byte aligned, Dh = 128);
 * q and k are normalised (q_norm / k_norm gains, eps) and rotated at position *d_pos with
 * (cos, sin) from `rope` (orator_rope_table, rope_rows >= capacity), k and v stored as bf16
 * at *d_pos, and q attends the *d_pos + 1 keys.  Same results as orator_qk_norm_rope_kv_write
 * then orator_gqa_decode. */
int orator_gqa_decode_append_qknorm(const float* q, const float* k_new, const float* v_new,
                                    uint16_t* kc, uint16_t* vc, float* out, int Hq, int Hkv,
                                    int Dh, const int* d_pos, int capacity, float scale,
                                    const float* q_norm, const float* k_norm, float eps,
                                    const float* rope, int rope_rows, void* stream);
/* Batched paged form (B streams, page-table row b, capacity max_pages * page_size; rows of
 * unmapped pages or pages >= n_pages are not written). */
int orator_gqa_decode_append_qknorm_paged(const float* q, const float* k_new, const float* v_new,
                                          uint16_t* kpool, uint16_t* vpool, const int* page_table,
                                          int max_pages, int page_size, int n_pages,
                                          const int* d_pos, float* out, int B, int Hq, int Hkv,
                                          int Dh, float scale, const float* q_norm,
                                          const float* k_norm, float eps, const float* rope,
                                          int rope_rows, void* stream);
/* WriteKvCacheKernel + GqaDecodeAttnKernel of one decode step (src/model/asr_text_decoder.cu:
 * 412-418) in one launch: the new token's K/V rows k_new/v_new [Hkv, Dh] fp32 are stored (bf16,
 * round to nearest even) at position *d_pos, and q attends the *d_pos + 1 keys including them.
 * Same result as orator_kv_write then orator_gqa_decode; k_new/v_new 16-byte aligned. */
int orator_gqa_decode_append(const float* q, const float* k_new, const float* v_new,
                             uint16_t* kc, uint16_t* vc, float* out, int Hq, int Hkv, int Dh,
                             const int* d_pos, int capacity, float scale, void* stream);
/* Batched paged form: stream b appends k_new/v_new [B, Hkv, Dh] at d_pos[b] through page-table
 * row b and attends d_pos[b] + 1 keys.  A new row whose page-table entry is unmapped (< 0) or
 * >= n_pages is not written (as orator_kv_write_paged), but is still attended; every earlier
 * position's page must be mapped. */
int orator_gqa_decode_append_paged(const float* q, const float* k_new, const float* v_new,
                                   uint16_t* kpool, uint16_t* vpool, const int* page_table,
                                   int max_pages, int page_size, int n_pages, const int* d_pos,
                                   float* out, int B, int Hq, int Hkv, int Dh, float scale,
                                   void* stream);

/* WindowAttnKernel (src/model/asr_audio_tower.cu:204-258, launch :573-575): the audio tower's
 * self-attention, q/k/v fp32 [N, H, Dh] (Dh in [1, 1024]; 64 and 128 on the fast kernels);
 * query i attends keys [seg_start[i], seg_end[i]) (device int arrays, clamped into [0, N));
 * online softmax, zeros for an empty window.  The kernel has no reference launcher: the parameters mirror its
 * arguments. */
int orator_window_attention(const float* q, const float* k, const float* v, float* out,
                            const int* d_seg_start, const int* d_seg_end, int N, int H, int Dh,
                            float scale, void* stream);

/* The Sortformer decoder's self-attention (src/model/sortformer_decoder.cu:280-298: head-major
 * gathers, QK^T batched SGEMM, ScaleMaskScoresKernel :114-123, AttnSoftmaxKernel :126-160, PV
 * batched SGEMM, scatter :163-174) in one launch: q/k/v/out fp32 [T, H, Dk], Dk in
 * {24, 32, 64}; scores (q.k) * scale, keys >= valid_len scored -1e30, row softmax, out the
 * context fed to the out projection.  The sequence has no reference launcher: the parameters
 * mirror the decomposition's. */
int orator_masked_mha(const float* q, const float* k, const float* v, float* out, int T, int H,
                      int Dk, int valid_len, float scale, void* stream);

/* ----------------------------------------------------- bf16-weight linear ---- */
/* asr_gemm::LinearPre (include/model/asr_gemm.h:33-38, src/model/asr_gemm.cu:175-208):
 * out[M,N] fp32 = act(in[M,K] W[N,K]^T + bias), in and W bf16, fp32 accumulation; act 0 none,
 * 1 exact-erf GELU, 2 ReLU; bias may be NULL.  M == 1 runs a streaming GEMV, M > 1 an MFMA
 * GEMM.  Any K >= 1 and any 2-byte aligned in / W, as the reference (asr_gemm.cu:188-214,
 * gemm.cuh:461-501): K % 8 == 0 with 16-byte aligned in and W takes the 16-byte-load kernels,
 * anything else the GEMM with element loads (M == 1 included). */
int orator_linear_pre(const uint16_t* in_bf16, const uint16_t* W_bf16, const float* bias,
                      float* out, int M, int K, int N, int act, void* stream);
/* The decoder MLP's gate|up projection with SwiGLU and the bf16 cast folded into the GEMM's
 * epilogue: asr_gemm::LinearPre on the fused [gate; up] weight (2I rows), asr_ops::SwiGLU and
 * F32ToBf16 (src/model/asr_text_decoder.cu:547-552, :424-428) in one launch.  out_bf16[M,I] =
 * bf16_rne(silu(g) * u), g = in . W[0:I]^T, u = in . W[I:2I]^T, the same values as the three
 * separate calls.  I % 4 == 0; any K (K % 8 != 0 or unaligned operands run the plain GEMM
 * into workspace, then the SwiGLU pass).  No reference counterpart as one entry. */
int orator_linear_pre_swiglu(const uint16_t* in_bf16, const uint16_t* W_gateup,
                             uint16_t* out_bf16, int M, int K, int I, void* stream);
/* asr_gemm::Linear (asr_gemm.h:27-31, asr_gemm.cu:160-167): the same with fp32 `in`, cast to
 * bf16 (round to nearest even) into library workspace first. */
int orator_linear(const float* in_f32, const uint16_t* W_bf16, const float* bias, float* out,
                  int M, int K, int N, int act, void* stream);
/* gemm::LaunchBf16Gemm (include/model/gemm.cuh:484-501): the MFMA GEMM for any M >= 1, any
 * K >= 1, 2-byte aligned operands (as orator_linear_pre). */
int orator_bf16_gemm(const uint16_t* in_bf16, const uint16_t* W_bf16, const float* bias,
                     float* out, int M, int K, int N, int act, void* stream);

/* ------------------------------------------------------- decode-step glue ---- */
/* EmbedGatherKernel (src/model/asr_text_decoder.cu:38-45): out[i] = table[*d_token][i]
 * (bf16 table [vocab, hidden] widened); hidden % 8 == 0, 16-byte aligned. */
int orator_embed_gather(const uint16_t* table, const int* d_token, float* out, int hidden,
                        void* stream);
/* AddResidualKernel (asr_text_decoder.cu:30-34): a[i] += b[i]; 16-byte aligned. */
int orator_add_residual(float* a, const float* b, long n, void* stream);
/* RecordTokenKernel (asr_text_decoder.cu:50-55): out[*d_count] = *d_token (dropped at or past
 * `capacity`), ++*d_count.  IncPosKernel (:58): ++*d_pos. */
int orator_record_token(int* out, int* d_count, const int* d_token, int capacity, void* stream);
int orator_inc_pos(int* d_pos, void* stream);

/* ----------------------------------------------------------------- decoder ---- */
/* AsrTextConfig (include/model/asr_text_decoder.h:30-42).  profile != 0 times, as the
 * reference does (src/model/asr_text_decoder.cu:369-377, 504-583, 762-889), with events and
 * host clocks and prints to stderr: eager decode steps on the default stream (per-token GPU
 * average every 16 steps), single-row prefills (layer loop vs final norm + LM head), and each
 * DecodeGreedy call (seed, loop, tokens emitted, host syncs). */
typedef struct OratorDecoderConfig {
  int num_layers, hidden_size, num_q_heads, num_kv_heads, head_dim, intermediate_size,
      vocab_size, max_seq_len;
  float rms_norm_eps, rope_theta;
  int profile;
} OratorDecoderConfig;
/* One layer's device weights, in the reference's fused layout
 * (src/model/asr_text_decoder.cu:288-307): qkv_w = q | k | v rows [(Hq + 2 Hkv) Dh, hidden],
 * gateup_w = gate | up rows [2 I, hidden], o_w [hidden, Hq Dh], down_w [hidden, I], bf16;
 * norms fp32 ([hidden], [Dh], [Dh], [hidden]).  The caller keeps them alive. */
typedef struct OratorDecoderLayer {
  const float* in_ln;
  const float* q_norm;
  const float* k_norm;
  const float* post_ln;
  const uint16_t* qkv_w;
  const uint16_t* o_w;
  const uint16_t* gateup_w;
  const uint16_t* down_w;
} OratorDecoderLayer;
/* AsrTextDecoder (include/model/asr_text_decoder.h:45-112) over caller-owned device weights:
 * embed [vocab, hidden] bf16, final_norm [hidden] fp32, lm_head [vocab, hidden] bf16 (NULL:
 * tied to embed), layers[num_layers].  Owns the bf16 KV caches [max_seq_len][Hkv][Dh] per
 * layer and all scratch.  head_dim must be 128. */
int orator_decoder_create(const OratorDecoderConfig* cfg, const uint16_t* embed,
                          const float* final_norm, const uint16_t* lm_head,
                          const OratorDecoderLayer* layers, void** handle);
int orator_decoder_destroy(void* handle);
/* ResetCache (asr_text_decoder.h:51, .cu:338): cache length 0. */
int orator_decoder_reset(void* handle);
/* Embed (asr_text_decoder.h:53-54, .cu:340-346): the bf16 row of token_id widened into the
 * host array out[hidden]. */
int orator_decoder_embed(void* handle, int token_id, float* out);
/* PrefillAt (asr_text_decoder.h:62-69, .cu:589-617): T embeddings [T, hidden] (host or
 * device memory) at positions pos0 .. pos0+T-1; leaves the last row's logits; synchronises
 * the stream. */
int orator_decoder_prefill_at(void* handle, const float* embeds, int T, int pos0,
                              void* stream);
/* DecodeStep (asr_text_decoder.h:78, .cu:618-633): one embedding [hidden] (host or device)
 * at pos; synchronises the stream. */
int orator_decoder_decode_step(void* handle, const float* embed, int pos, void* stream);
/* DecodeStepDevice (asr_text_decoder.h:80-85, .cu:656-671): gathers the embedding of the
 * token id held in the device scalar d_token and runs the step at pos; no final sync. */
int orator_decoder_decode_step_device(void* handle, const int* d_token, int pos, void* stream);
/* Argmax (asr_text_decoder.h:89, .cu:635-641) over the current logits, two bans (-1 none). */
int orator_decoder_argmax(void* handle, int ban0, int ban1, int* token, void* stream);
/* ArgmaxToDevice (asr_text_decoder.h:91-93, .cu:643-647): the winning id into *d_out. */
int orator_decoder_argmax_to_device(void* handle, int* d_out, int ban0, int ban1, void* stream);
/* Device pointer to the current logits [vocab] (CopyLogits reads them). */
int orator_decoder_logits(void* handle, float** d_logits);
/* DecodeGreedy (asr_text_decoder.h:96-107, .cu:698-889): seeds from the current logits, emits
 * up to max_new tokens into `tokens`, stops at eos0/eos1 (not emitted) or 6 identical tokens;
 * EOS banned for the first ban_steps tokens; host sync every `batch` steps; use_graph replays
 * captured step graphs.  *n_tokens = tokens emitted; the cache length counts every step run. */
int orator_decoder_decode_greedy(void* handle, int start_pos, int max_new, int eos0, int eos1,
                                 int ban_steps, int batch, int use_graph, int* tokens,
                                 int* n_tokens, void* stream);
/* TruncateCache / cache_len (asr_text_decoder.h:73-76). */
int orator_decoder_truncate(void* handle, int len);
int orator_decoder_cache_len(void* handle, int* len);

/* -------------------------------------------------------- Conformer layer ---- */
/* ConformerLayer (include/model/conformer_layer.h:31-65) over caller-owned fp32 device
 * weights, in the checkpoint order of src/model/conformer_layer.cu:270-308. */
typedef struct OratorConformerWeights {
  const float *norm_ff1_w, *norm_ff1_b, *ff1_w1, *ff1_b1, *ff1_w2, *ff1_b2;
  const float *norm_att_w, *norm_att_b, *q_w, *q_b, *k_w, *k_b, *v_w, *v_b, *out_w, *out_b;
  const float *pos_w, *pos_bias_u, *pos_bias_v;
  const float *norm_conv_w, *norm_conv_b, *pw1_w, *pw1_b, *dw_w, *dw_b;
  const float *bn_w, *bn_b, *bn_mean, *bn_var, *pw2_w, *pw2_b;
  const float *norm_ff2_w, *norm_ff2_b, *ff2_w1, *ff2_b1, *ff2_w2, *ff2_b2;
  const float *norm_out_w, *norm_out_b;
} OratorConformerWeights;
/* ConformerLayer(d_model, n_heads, d_ff, conv_kernel) + LoadWeights (conformer_layer.h:33-37);
 * the weights stay owned by the caller. */
int orator_conformer_create(int d_model, int n_heads, int d_ff, int conv_kernel,
                            const OratorConformerWeights* weights, void** handle);
int orator_conformer_destroy(void* handle);
/* ConformerLayer::Forward (conformer_layer.h:39-43, .cu:364-488): x [T, d_model] in place,
 * pos_emb [2T-1, d_model] (BuildPosEmb), frames >= valid_len masked.  attn_mode 0 runs the
 * attention core in fp32 in the reference's decomposition, 1 the fused fp16 MFMA kernel
 * (d_model / n_heads = 64). */
int orator_conformer_forward(void* handle, float* x, int T, int valid_len, const float* pos_emb,
                             int attn_mode, void* stream);

/* ----------------------------------------------------------------- GEMM ---- */
/* gemm::LaunchSgemm (include/model/gemm.cuh:160-174): out[M,N] = act(in[M,K] W[N,K]^T + bias),
 * act 0 none, 1 SiLU, 2 ReLU, 3 sigmoid (gemm.cuh:38-45); bias may be NULL. */
int orator_sgemm(const float* in, const float* W, const float* bias, float* out, int M, int K,
                 int N, int act, void* stream);
/* gemm::LaunchSgemmBatched (include/model/gemm.cuh:251-268): per batch b,
 * out+b*stride_out = act(in+b*stride_in . (W+b*stride_w)^T); any M, N, K, alignment. */
int orator_sgemm_batched(const float* in, const float* W, float* out, int M, int K, int N, int act,
                         int batch, long stride_in, long stride_w, long stride_out, void* stream);

/* ----------------------------------------------------- Conformer rel-pos ---- */
/* Attention core of ConformerLayer::Forward (src/model/conformer_layer.cu:405-444): q/k/v
 * [T,H,Dk] (linear_q/k/v outputs), p [2T-1,H,Dk] (linear_pos of BuildPosEmb), u/v biases
 * [H,Dk]; out [T,H,Dk] = softmax((AC + rel_shift(BD)) * scale, keys >= valid_len masked) . v,
 * the context fed to linear_out.  fp32, reference decomposition (batched SGEMMs). */
int orator_relpos_attention(const float* q, const float* k, const float* v, const float* p,
                            const float* pos_bias_u, const float* pos_bias_v, float* out, int T,
                            int H, int Dk, int valid_len, float scale, void* stream);

/* Same attention core, fused on fp16 MFMA (one launch, no [H,T,2T-1] BD matrix): inputs
 * fp16 bits (in_f16 = 1), fp32 rounded to fp16 on load (in_f16 = 0), or q fp32 and k, v, p
 * fp16 bits (in_f16 = 2: the same result as in_f16 = 0 on the fp32 rows k, v, p round to);
 * biases and output fp32; Dk = 64.  Max abs error ~1e-3 on unit-scale outputs (fp16 operands, fp32 accumulate). */
int orator_relpos_attention_fast(const void* q, const void* k, const void* v, const void* p,
                                 const float* pos_bias_u, const float* pos_bias_v, float* out,
                                 int T, int H, int Dk, int valid_len, float scale, int in_f16,
                                 void* stream);

/* ConformerLayer::BuildPosEmb (src/model/conformer_layer.cu:314-329): HOST function filling
 * pe [2T-1, d_model] (host memory) with the relative positional encoding. */
int orator_build_pos_emb(float* pe, int T, int d_model);

/* Prefill precision modes.
 * FP32: q enters the MFMA products as three bf16 terms and the softmax weights as two, so
 *       results track the fp32 reference (GqaCacheAttnKernel) to fp32 rounding level.
 * BF16: q and the softmax weights rounded to bf16 (one MFMA per product). */
#define ORATOR_PREFILL_FP32 0
#define ORATOR_PREFILL_BF16 1

/* GqaCacheAttnKernel (src/model/asr_text_decoder.cu:88-142, launch :537-541): query row t
 * (absolute position *d_pos0 + t) of q [Tq, Hq, Dh] attends keys [0, pos0 + t] of the bf16
 * cache.  fp32 mode.  `capacity` = the cache's max_seq_len (keys past it are not read).
 * Any Dh in [1, 1024] and any Hq multiple of Hkv (the reference: Dh <= 256): Dh 128 with
 * Hq/Hkv in {1,2,4} runs on the MFMA kernels, other shapes on a generic fp32 kernel. */
int orator_gqa_prefill(const float* q, const uint16_t* kc, const uint16_t* vc, float* out, int Tq,
                       int Hq, int Hkv, int Dh, const int* d_pos0, int capacity, float scale,
                       void* stream);
/* General form: q as fp32 (`q`) or bf16 bits (`q_bf16`, used when q is NULL); contiguous
 * cache (page_table NULL) or one stream's page-table row; `mode` ORATOR_PREFILL_*. */
int orator_gqa_prefill_ex(const float* q, const uint16_t* q_bf16, const uint16_t* kpool,
                          const uint16_t* vpool, const int* page_table, int max_pages,
                          int page_size, float* out, int Tq, int Hq, int Hkv, int Dh,
                          const int* d_pos0, int capacity, float scale, int mode, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* ORATOR_ATTN_H_ */
