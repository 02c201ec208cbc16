// Host-side internals shared by the launchers and the C ABI: status codes, the
// per-thread error message, and the per-(device, stream) workspace used by the
// split-K decode combine.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

#include "../../include/orator_attn.h"

namespace orator_hip {

// Records `msg` as this thread's last error and returns `code`.
int fail(int code, const std::string& msg);
// Maps a HIP error to ORATOR_ERR_HIP (recording where it came from), or ORATOR_OK.
int check_hip(hipError_t e, const char* what);
// Checks hipGetLastError() after a launch.
int check_launch(const char* what);

// Device scratch owned by the library, one block per (device, stream, host thread, slot),
// grown geometrically on demand.  A grown block's old memory is freed once the work queued
// on the stream before the growth has finished (an event), or, if it was handed out during a
// graph capture, at workspace_release(stream).  Returns nullptr on failure (the error is
// recorded).
// Slots are independent blocks: kWsGemm holds the split-K partials of the GEMMs, which may run
// while a caller's slot-0 buffer (e.g. the bf16 cast of a Linear input) is being read.
constexpr int kWsGemm = 1;
constexpr int kWsArrive = 3;  // arrival counters of the decode's in-launch split merge
constexpr int kWsPrefill = 4;        // partials of the long-prompt prefill's cut blocks
constexpr int kWsPrefillArrive = 5;  // its arrival counters
// *fresh (optional): the block was allocated by this call, its contents undefined.
void* workspace(hipStream_t stream, size_t bytes, int slot = 0, bool* fresh = nullptr);
// Frees every workspace block of `stream` (all threads, current and retired) after the
// stream's queued work; for the owner of a stream about to be destroyed.
int workspace_release(hipStream_t stream);

inline int ilog2_exact(int v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int s = 0;
  while ((1 << s) < v) ++s;
  return s;
}

// Decode-step GEMV over an fp32 producer (linear.hip): mode selects how the bf16 input row is
// built (cast, RMSNorm with gain `aux`, SwiGLU with up = `aux`); accumulate adds into out;
// pair reads 2N weight rows (gate | up) and stores silu(gate) * up for N outputs.
enum { kGemvInF32 = 1, kGemvInRmsNorm = 2, kGemvInSwiglu = 3 };
constexpr int kFusedMaxK = 8192;
int launch_gemv_fused(int mode, const float* x, const float* aux, float eps, const uint16_t* W,
                      float* out, int K, int N, bool accumulate, hipStream_t s,
                      bool pair = false);

// ArgmaxBanned with caller-provided scratch of argmax_scratch_bytes(n) bytes (0: none
// needed, one workgroup does it).
size_t argmax_scratch_bytes(int n);
int launch_argmax_banned(const float* logits, int n, int ban0, int ban1, int* out_idx,
                         void* scratch, hipStream_t s);

// Compute units of the current device (cached per device); 0 if it cannot be queried.
int device_cu_count();

// Optional measurement hook: when set, the next decode launch records `start` right before
// its split kernel, `split_end` right after it and `stop` after its split merge (on the
// launch stream), then clears the hook.  Any of them may be null.
void take_timing_events(hipEvent_t* start, hipEvent_t* split_end, hipEvent_t* stop);

// ---- launchers (defined in the .hip files) ----
struct DecodeProblem {
  const float* q;
  const void* kpool;      // bf16 bits, or fp32 when kv_f32
  const void* vpool;
  bool kv_f32;
  int pos_mode;           // 0: stream b attends pos[b]+1 keys; 1: b+1 keys; 2: capacity keys;
                          // 3: keys [seg_start[b], seg_end[b]) (windowed self-attention)
  const int* seg_start;   // pos_mode 3
  const int* seg_end;
  const int* page_table;  // nullptr => contiguous caches
  int max_pages;          // page-table row length (paged)
  int page_size;          // paged only (power of two >= 16)
  long stream_stride;     // elements between streams' contiguous caches
  const int* pos;         // [B] device: stream b attends pos[b]+1 keys
  float* out;
  int B, Hq, Hkv, Dh;
  int capacity;           // max keys any stream can attend (grid sizing)
  float scale;
  // Append (bf16 caches, pos_mode 0): K/V rows [B][Hkv][Dh] fp32 written at pos[b] and
  // attended as the last key in the same launch; pool_rows bounds the write.
  const float* k_new;
  const float* v_new;
  long pool_rows;
  // Optional (append, Dh 128, bf16 caches): q and k_new are raw projections; the launch
  // applies the per-head RmsNorm (weights q_norm / k_norm, eps) and the rotate-half RoPE of
  // position pos[b], with (cos, sin) of pair j at rope[(pos * 64 + j) * 2 ..] (the values
  // rope_cs forms; the table holds `capacity` positions, and a position past it -- whose KV
  // write is dropped -- uses the last row), before attending: the step's QK-norm/RoPE kernel
  // folded in.
  const float* q_norm = nullptr;
  const float* k_norm = nullptr;
  const float* rope = nullptr;
  float eps = 0.0f;
  // Split-partial scratch supplied by the caller (scratch_bytes long) instead of the library
  // workspace; a launch needing more fails with ORATOR_ERR_CAPACITY.
  void* scratch = nullptr;
  size_t scratch_bytes = 0;
  // With scratch: kArriveCounters arrival counters (kCounterStride apart), zero between
  // launches, for the split
  // merge inside the split launch (small grids); nullptr runs the separate merge kernel.
  unsigned* arrive = nullptr;
};
constexpr int kArriveCounters = 4096;
// Counters are kCounterStride u32 apart, each on its own 128-byte line: agent-scope atomics on
// one line are serialised where they are performed (the 264 adds of a B = 1 decode on one
// line took ~2.5 us).
constexpr int kCounterStride = 32;
// A block of kArriveCounters counters (kCounterStride apart) in workspace slot `slot` of the
// stream, zeroed by a fill kernel when the block is allocated; the kernels using it return
// every counter to zero.
int zeroed_counters(hipStream_t stream, int slot, unsigned** out);
// Long-prompt bf16 prefill over a contiguous cache, one wave per SIMD with stream-K balance
// (prefill_sk.hip); Dh 128, Hq / Hkv in {1, 2, 4}, Hkv * ceil(Tq / (128 / G)) <= kArriveCounters.
int launch_prefill_sk(const float* q, const uint16_t* q_bf16, const uint16_t* kc,
                      const uint16_t* vc, float* out, int Tq, int Hq, int Hkv,
                      const int* d_pos0, int capacity, float scale, hipStream_t stream);
int launch_gqa_decode(const DecodeProblem& p, hipStream_t stream);
// Self-attention of fp32 [N, H, Dk] rows, Dk in {24, 32, 64}, on fp32 MFMA (range_attn.hip):
// query i attends keys [seg_start[i], seg_end[i]) clamped into [0, N) (device arrays), or
// without them keys [0, valid) (valid <= 0: a uniform softmax over all N keys); zeros for an
// empty range.  q, k, v 16-byte aligned.
int launch_range_attention(const float* q, const float* k, const float* v, float* out,
                           const int* seg_start, const int* seg_end, int N, int H, int Dk,
                           int valid, float scale, hipStream_t s);
// The generic attention kernel (attention_generic.hip) for the shapes the fast kernels are not
// built for: any Dh in [1, 1024], any Hq multiple of Hkv.
// asr_ops::GqaAttention: fp32 self-attention over T rows.
int launch_gqa_attention_generic(const float* q, const float* k, const float* v, float* out,
                                 int T, int Hq, int Hkv, int Dh, float scale, bool causal,
                                 hipStream_t s);
// Prefill over a bf16 cache (contiguous, or paged through one page-table row with 2^page_shift
// keys per page): row t attends keys [0, min(*d_pos0 + t + 1, capacity)); q fp32, or bf16
// when q is null.
int launch_prefill_generic(const float* q, const uint16_t* q_bf16, const uint16_t* kpool,
                           const uint16_t* vpool, const int* page_table, int max_pages,
                           int page_shift, float* out, int Tq, int Hq, int Hkv, int Dh,
                           const int* d_pos0, int capacity, float scale, hipStream_t s);
// Decode of a DecodeProblem (no QK-norm folding; the appended key, if any, is attended from
// k_new / v_new -- the caller writes it to the cache).
int launch_decode_generic(const DecodeProblem& p, int page_shift, hipStream_t s);
// (cos, sin) of RoPE pair j (head_dim 128, base theta) for positions [0, n_pos): out[(p * 64 +
// j) * 2 + {0, 1}], the values the fused QK-norm/RoPE kernels form.
int launch_rope_table(float* out, int n_pos, float theta, hipStream_t s);
// orator_qk_norm_rope_kv_write with an optional (cos, sin) table of launch_rope_table holding
// positions [0, rope_rows) (the same values, without the per-call fp64 pow/sincos); other
// positions, or rope == nullptr, form them per call.
int launch_qk_norm_rope_kv(float* q, float* k, const float* v, long q_stride, long kv_stride,
                           const float* q_norm, const float* k_norm, float eps,
                           const int* positions, float theta, const float* rope,
                           int rope_rows, int n_tokens, int tokens_per_stream, int Hq, int Hkv,
                           int Dh, uint16_t* kpool, uint16_t* vpool, const int* page_table,
                           int max_pages, int page_size, int capacity, hipStream_t stream);
// Workspace bytes a decode launch over B streams of `capacity` keys needs (split partials).
size_t decode_workspace_bytes(int B, int Hq, int Dh, int capacity);
// Sizes the stream's decode workspace (partials and arrival counters) for such launches ahead
// of a graph capture.
int decode_workspace_reserve(int B, int Hq, int Dh, int capacity, hipStream_t stream);

// out[M][N] += in[M][K] W[N][K]^T: the residual add folded into the GEMM's store (M > 1); the
// M = 1 GEMV writes tmp [N] and an add follows.
int launch_linear_pre_acc(const uint16_t* in, const uint16_t* W, float* out, int M, int K, int N,
                          float* tmp, hipStream_t stream);
// RmsNorm with the bf16 cast of its output folded in; SwiGLU of a fused gate|up block
// [T][2I] with the bf16 cast folded in.
int launch_rms_norm_bf16(const float* x, const float* w, uint16_t* out, int rows, int dim,
                         float eps, hipStream_t s);
int launch_swiglu_bf16(const float* gu, uint16_t* out, int T, int I, hipStream_t s);

// This library's bf16 GEMM (gemm_bf16.hip): out[M][N] (= or +=) act(in[M][K] W[N][K]^T +
// bias), fp32 accumulation and output.  K a multiple of 8 and 16-byte aligned operands, or
// `generic`: any K, operands at any 2-byte alignment (element loads).
int launch_gemm_bf16_nt(const uint16_t* in, const uint16_t* W, const float* bias, float* out,
                        int M, int K, int N, int act, bool accumulate, hipStream_t s,
                        bool generic = false);
// The gate|up projection with SwiGLU and the bf16 cast in the GEMM epilogue (gemm_bf16.hip):
// out[M][I] = bf16(silu(in W[0:I]^T) * (in W[I:2I]^T)); `tmp` ([M][2I] fp32, or null for the
// stream's workspace) is used only when the grid is too short for the fused kernel.
int launch_gemm_bf16_swiglu(const uint16_t* in, const uint16_t* W, uint16_t* out, float* tmp,
                            int M, int K, int I, hipStream_t s);

int launch_sgemm(const float* in, const float* W, const float* bias, float* out, int M, int K,
                 int N, int act, int batch, long stride_in, long stride_w, long stride_out,
                 hipStream_t stream);

// out[M][N] += res_scale * (in W^T + bias): a linear followed by the reference's AddScaledKernel
// (src/model/conformer_layer.cu:70-76, used at :385, :448, :467, :475), folded into one launch.
int launch_sgemm_residual(const float* in, const float* W, const float* bias, float* out, int M,
                          int K, int N, float res_scale, hipStream_t stream);

// launch_sgemm_residual, then ln_out = LayerNorm(out rows; ln_g, ln_b, eps) (conformer_layer.cu:
// 28-66, the next block's norm), fused into the split-K reduce when K is split and N <= 1024
// (else a LayerNorm pass); ln_out may be out.  Same bits as the two operations.
int launch_sgemm_residual_ln(const float* in, const float* W, const float* bias, float* out,
                             int M, int K, int N, float res_scale, const float* ln_g,
                             const float* ln_b, float* ln_out, float eps, hipStream_t stream);

// LayerNorm of T rows of C (conformer_ops.hip); out may be in.
int launch_layer_norm(const float* in, const float* g, const float* b, float* out, int T, int C,
                      float eps, hipStream_t s);

// The Conformer conv module's pointwise_conv1 + GLU + padding-row mask in one launch
// (src/model/conformer_layer.cu:455-458): W [2C][K] (value rows, then gate rows), out [M][C] =
// a * (1 / (1 + __expf(-b))) of the biased value / gate outputs, 0 for rows >= valid.
// ORATOR_ERR_UNSUPPORTED (nothing launched) unless K % 32 == 0 and in, W are 16-byte aligned.
int launch_sgemm_glu(const float* in, const float* W, const float* bias, float* out, int M, int K,
                     int C, int valid, hipStream_t stream);

// out[g] = in W[g]^T + bias[g] for g = 0..2: three products of one shape sharing `in`, one launch.
// out[g] is fp32, or fp16 (each fp32 result rounded to nearest even) where bit g of h16_mask is set.
int launch_sgemm_group3(const float* in, const float* const W[3], const float* const bias[3],
                        void* const out[3], int M, int K, int N, int h16_mask,
                        hipStream_t stream);

// out[M][N] = fp16(in W^T), the fp32 product rounded to nearest even once per element (never
// split over K): the values an fp16 consumer would round from launch_sgemm's fp32 output.
int launch_sgemm_f16_out(const float* in, const float* W, void* out, int M, int K, int N,
                         hipStream_t stream);

}  // namespace orator_hip
