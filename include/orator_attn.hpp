// orator_attn.hpp -- C++20 drop-in for the reference's operator API on the attention path.
//
// Re-exposes the launchers of include/model/asr_ops.cuh, include/model/asr_gemm.h and
// include/model/gemm.cuh (thomas-hiddenpeak/Orator) with the same namespaces, names,
// argument order and meaning, over the C ABI in orator_attn.h.  cudaStream_t becomes
// hipStream_t.  As in the reference, launches are asynchronous, non-positive sizes are a
// no-op, and a failure throws orator::gpu::GpuMemoryException (a std::runtime_error), which
// is what the reference's CheckCudaError throws (src/gpu/memory.cc:14-21).  Entry points
// the reference keeps file-static (the decoder's KV write and attention kernels, the
// Conformer attention block) are exposed under orator::model::decoder_attn and
// orator::model::conformer_attn.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "orator_attn.h"

namespace orator {
namespace gpu {

class GpuMemoryException : public std::runtime_error {
 public:
  GpuMemoryException(int code, const std::string& msg)
      : std::runtime_error("[orator " + std::to_string(code) + "] " + msg), code_(code) {}
  int code() const { return code_; }

 private:
  int code_;
};

inline void Check(int rc) {
  if (rc != ORATOR_OK) throw GpuMemoryException(rc, orator_last_error());
}

}  // namespace gpu

namespace model {
namespace asr_ops {  // include/model/asr_ops.cuh:21-62

inline void RmsNorm(const float* x, const float* weight, float* out, int rows, int dim, float eps,
                    hipStream_t stream = 0) {
  gpu::Check(orator_rms_norm(x, weight, out, rows, dim, eps, stream));
}
inline void RopeInterleaved(float* x, const int* positions, int n_tokens, int n_heads,
                            int head_dim, float theta_base) {
  gpu::Check(orator_rope_interleaved(x, positions, n_tokens, n_heads, head_dim, theta_base));
}
inline void SwiGLU(const float* gate, const float* up, float* out, int n, hipStream_t stream = 0) {
  gpu::Check(orator_swiglu(gate, up, out, n, stream));
}
inline void RopeHalf(float* x, const int* positions, int n_tokens, int n_heads, int head_dim,
                     float theta_base, hipStream_t stream = 0) {
  gpu::Check(orator_rope_half(x, positions, n_tokens, n_heads, head_dim, theta_base, stream));
}
inline void GqaAttention(const float* q, const float* k, const float* v, float* out, int T, int Hq,
                         int Hkv, int Dh, float scale, bool causal) {
  gpu::Check(orator_gqa_attention(q, k, v, out, T, Hq, Hkv, Dh, scale, causal ? 1 : 0));
}
inline void ArgmaxBanned(const float* logits, int n, int ban0, int ban1, int* out_idx,
                         hipStream_t stream = 0) {
  gpu::Check(orator_argmax_banned(logits, n, ban0, ban1, out_idx, stream));
}

}  // namespace asr_ops

namespace asr_gemm {  // include/model/asr_gemm.h:23-25 (the cast half of the interface)

inline void F32ToBf16(const float* in, uint16_t* out, long n, hipStream_t stream = 0) {
  gpu::Check(orator_f32_to_bf16(in, out, n, stream));
}
inline void Bf16ToF32(const uint16_t* in, float* out, long n, hipStream_t stream = 0) {
  gpu::Check(orator_bf16_to_f32(in, out, n, stream));
}

}  // namespace asr_gemm

// The decoder's file-static kernels (src/model/asr_text_decoder.cu:62-213) as callable
// operators; `capacity` is the cache's max_seq_len (AsrTextConfig::max_seq_len).
namespace decoder_attn {

inline void WriteKvCache(const float* k, const float* v, uint16_t* kc, uint16_t* vc, int Tq,
                         int Hkv, int Dh, const int* d_pos0, int capacity, hipStream_t stream = 0) {
  gpu::Check(orator_kv_write(k, v, kc, vc, Tq, Hkv, Dh, d_pos0, capacity, stream));
}
inline void GqaCacheAttn(const float* q, const uint16_t* kc, const uint16_t* vc, float* out, int Tq,
                         int Hq, int Hkv, int Dh, const int* d_pos0, int capacity, float scale,
                         hipStream_t stream = 0) {
  gpu::Check(orator_gqa_prefill(q, kc, vc, out, Tq, Hq, Hkv, Dh, d_pos0, capacity, scale, stream));
}
inline void GqaDecodeAttn(const float* q, const uint16_t* kc, const uint16_t* vc, float* out, int Hq,
                          int Hkv, int Dh, const int* d_pos, int capacity, float scale,
                          hipStream_t stream = 0) {
  gpu::Check(orator_gqa_decode(q, kc, vc, out, Hq, Hkv, Dh, d_pos, capacity, scale, stream));
}
// WriteKvCache + GqaDecodeAttn in one launch (asr_text_decoder.cu:412-418).
inline void GqaDecodeAttnAppend(const float* q, const float* k_new, const float* v_new,
                                uint16_t* kc, uint16_t* vc, float* out, int Hq, int Hkv, int Dh,
                                const int* d_pos, int capacity, float scale,
                                hipStream_t stream = 0) {
  gpu::Check(orator_gqa_decode_append(q, k_new, v_new, kc, vc, out, Hq, Hkv, Dh, d_pos, capacity,
                                      scale, stream));
}
// RmsNorm(q,k) + RopeHalf(q,k) + WriteKvCache in one launch (asr_text_decoder.cu:408-413).
inline void QkNormRopeKvWrite(float* q, float* k, const float* v, long q_stride, long kv_stride,
                              const float* q_norm, const float* k_norm, float eps,
                              const int* positions, float theta, int n_tokens, int Hq, int Hkv,
                              int Dh, uint16_t* kc, uint16_t* vc, int capacity,
                              hipStream_t stream = 0) {
  gpu::Check(orator_qk_norm_rope_kv_write(q, k, v, q_stride, kv_stride, q_norm, k_norm, eps,
                                          positions, theta, n_tokens, n_tokens, Hq, Hkv, Dh, kc,
                                          vc, nullptr, 0, 0, capacity, stream));
}

}  // namespace decoder_attn

// The rel-pos attention block of ConformerLayer::Forward (src/model/conformer_layer.cu:405-444).
namespace conformer_attn {

inline void RelPosAttention(const float* q, const float* k, const float* v, const float* p,
                            const float* pos_bias_u, const float* pos_bias_v, float* out, int T,
                            int H, int Dk, int valid_len, float scale, hipStream_t stream = 0) {
  gpu::Check(orator_relpos_attention(q, k, v, p, pos_bias_u, pos_bias_v, out, T, H, Dk, valid_len,
                                     scale, stream));
}

}  // namespace conformer_attn
}  // namespace model

namespace gemm {  // include/model/gemm.cuh:160-174, 251-268

inline void LaunchSgemm(const float* in, const float* W, const float* bias, float* out, int M,
                        int K, int N, int act) {
  gpu::Check(orator_sgemm(in, W, bias, out, M, K, N, act, nullptr));
}
inline void LaunchSgemm(const float* in, const float* W, const float* bias, float* out, int M,
                        int K, int N, int act, hipStream_t stream) {
  gpu::Check(orator_sgemm(in, W, bias, out, M, K, N, act, stream));
}
inline void LaunchSgemmBatched(const float* in, const float* W, float* out, int M, int K, int N,
                               int act, int batch, long strideIn, long strideW, long strideOut) {
  gpu::Check(orator_sgemm_batched(in, W, out, M, K, N, act, batch, strideIn, strideW, strideOut,
                                  nullptr));
}
inline void LaunchSgemmBatched(const float* in, const float* W, float* out, int M, int K, int N,
                               int act, int batch, long strideIn, long strideW, long strideOut,
                               hipStream_t stream) {
  gpu::Check(orator_sgemm_batched(in, W, out, M, K, N, act, batch, strideIn, strideW, strideOut,
                                  stream));
}

}  // namespace gemm
}  // namespace orator
