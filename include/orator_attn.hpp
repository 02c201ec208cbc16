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
#include <vector>

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

namespace asr_gemm {  // include/model/asr_gemm.h:23-41

inline void Linear(const float* in_f32, const uint16_t* W_bf16, const float* bias_f32,
                   float* out_f32, int M, int K, int N, int act, hipStream_t stream = 0) {
  gpu::Check(orator_linear(in_f32, W_bf16, bias_f32, out_f32, M, K, N, act, stream));
}
inline void LinearPre(const uint16_t* in_bf16, const uint16_t* W_bf16, const float* bias_f32,
                      float* out_f32, int M, int K, int N, int act, hipStream_t stream = 0) {
  gpu::Check(orator_linear_pre(in_bf16, W_bf16, bias_f32, out_f32, M, K, N, act, stream));
}
// The library's workspace lives until the process ends; nothing to release early.
inline void Shutdown() {}
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

// ConformerLayer (include/model/conformer_layer.h:31-65) over caller-owned fp32 device
// weights (LoadWeights' tensors, as an OratorConformerWeights of device pointers).
class ConformerLayer {
 public:
  ConformerLayer(const OratorConformerWeights& weights, int d_model = 512, int n_heads = 8,
                 int d_ff = 2048, int conv_kernel = 9) {
    gpu::Check(orator_conformer_create(d_model, n_heads, d_ff, conv_kernel, &weights, &h_));
  }
  ~ConformerLayer() { orator_conformer_destroy(h_); }
  ConformerLayer(const ConformerLayer&) = delete;
  ConformerLayer& operator=(const ConformerLayer&) = delete;
  // attn_mode 0: fp32 attention core (the reference's semantics); 1: fused fp16 MFMA core.
  void Forward(float* x, int T, int valid_len, const float* pos_emb, hipStream_t stream = nullptr,
               int attn_mode = 0) {
    gpu::Check(orator_conformer_forward(h_, x, T, valid_len, pos_emb, attn_mode, stream));
  }
  // ConformerLayer::BuildPosEmb (include/model/conformer_layer.h:45-46): the relative
  // positional encoding [2T-1, d_model] built on the host.
  static std::vector<float> BuildPosEmb(int T, int d_model) {
    std::vector<float> pe(T > 0 && d_model > 0 ? static_cast<size_t>(2 * T - 1) * d_model : 0);
    gpu::Check(orator_build_pos_emb(pe.data(), T, d_model));
    return pe;
  }

 private:
  void* h_ = nullptr;
};

}  // namespace conformer_attn

// The audio tower's WindowAttnKernel (src/model/asr_audio_tower.cu:204-258) and the Sortformer
// decoder's masked MHA (src/model/sortformer_decoder.cu:280-298), both file-static in the
// reference.
namespace aux_attn {

inline void WindowAttention(const float* q, const float* k, const float* v, float* out,
                            const int* seg_start, const int* seg_end, int N, int H, int Dh,
                            float scale, hipStream_t stream = 0) {
  gpu::Check(orator_window_attention(q, k, v, out, seg_start, seg_end, N, H, Dh, scale, stream));
}
inline void MaskedSelfAttention(const float* q, const float* k, const float* v, float* out, int T,
                                int H, int Dk, int valid_len, float scale,
                                hipStream_t stream = 0) {
  gpu::Check(orator_masked_mha(q, k, v, out, T, H, Dk, valid_len, scale, stream));
}

}  // namespace aux_attn

// AsrTextDecoder (include/model/asr_text_decoder.h:45-112) over caller-owned device weights.
struct AsrTextConfig {  // include/model/asr_text_decoder.h:30-42
  int hidden_size = 2048;
  int num_layers = 28;
  int num_q_heads = 16;
  int num_kv_heads = 8;
  int head_dim = 128;
  int intermediate_size = 6144;
  int vocab_size = 151936;
  float rms_norm_eps = 1e-6f;
  float rope_theta = 1000000.0f;
  int max_seq_len = 2048;
  bool profile = false;            // event timing to stderr (decode steps, prefill, greedy)
  bool cuda_graph_enabled = true;  // graph replay in DecodeGreedy
};

class AsrTextDecoder {
 public:
  // embed / lm_head bf16 [vocab, hidden] (lm_head nullptr: tied), final_norm fp32 [hidden],
  // layers[num_layers] in the fused qkv / gate|up layout.
  AsrTextDecoder(const AsrTextConfig& c, const uint16_t* embed, const float* final_norm,
                 const uint16_t* lm_head, const OratorDecoderLayer* layers)
      : config_(c) {
    const OratorDecoderConfig oc{c.num_layers,  c.hidden_size,       c.num_q_heads,
                                 c.num_kv_heads, c.head_dim,         c.intermediate_size,
                                 c.vocab_size,  c.max_seq_len,       c.rms_norm_eps,
                                 c.rope_theta,  c.profile ? 1 : 0};
    gpu::Check(orator_decoder_create(&oc, embed, final_norm, lm_head, layers, &h_));
  }
  ~AsrTextDecoder() { orator_decoder_destroy(h_); }
  AsrTextDecoder(const AsrTextDecoder&) = delete;
  AsrTextDecoder& operator=(const AsrTextDecoder&) = delete;

  void ResetCache() { gpu::Check(orator_decoder_reset(h_)); }
  void Embed(int token_id, float* out) const { gpu::Check(orator_decoder_embed(h_, token_id, out)); }
  int hidden_size() const { return config_.hidden_size; }
  int vocab_size() const { return config_.vocab_size; }
  void Prefill(const float* embeds, int T, hipStream_t stream = 0) {
    PrefillAt(embeds, T, 0, stream);
  }
  void PrefillAt(const float* embeds, int T, int pos0, hipStream_t stream = 0) {
    gpu::Check(orator_decoder_prefill_at(h_, embeds, T, pos0, stream));
  }
  void TruncateCache(int len) { gpu::Check(orator_decoder_truncate(h_, len)); }
  int cache_len() const {
    int n = 0;
    gpu::Check(orator_decoder_cache_len(h_, &n));
    return n;
  }
  void DecodeStep(const float* embed, int pos, hipStream_t stream = 0) {
    gpu::Check(orator_decoder_decode_step(h_, embed, pos, stream));
  }
  void DecodeStepDevice(const int* d_token, int pos, hipStream_t stream = 0) {
    gpu::Check(orator_decoder_decode_step_device(h_, d_token, pos, stream));
  }
  int Argmax(int ban0 = -1, int ban1 = -1, hipStream_t stream = 0) {
    int t = 0;
    gpu::Check(orator_decoder_argmax(h_, ban0, ban1, &t, stream));
    return t;
  }
  void ArgmaxToDevice(int* d_out, int ban0 = -1, int ban1 = -1, hipStream_t stream = 0) {
    gpu::Check(orator_decoder_argmax_to_device(h_, d_out, ban0, ban1, stream));
  }
  int ReadTokenId(const int* d_token, hipStream_t stream = 0) const {
    int t = 0;
    gpu::Check(orator_stream_synchronize(stream));
    gpu::Check(orator_memcpy_dtoh(&t, d_token, sizeof(int)));
    return t;
  }
  std::vector<int> DecodeGreedy(int start_pos, int max_new, int eos0, int eos1,
                                int ban_steps = 3, int batch = 32, hipStream_t stream = 0) {
    std::vector<int> out(max_new > 0 ? max_new : 0);
    int n = 0;
    gpu::Check(orator_decoder_decode_greedy(h_, start_pos, max_new, eos0, eos1, ban_steps, batch,
                                            config_.cuda_graph_enabled ? 1 : 0, out.data(), &n,
                                            stream));
    out.resize(n);
    return out;
  }
  std::vector<float> CopyLogits() const {
    float* d = nullptr;
    gpu::Check(orator_decoder_logits(h_, &d));
    std::vector<float> out(config_.vocab_size);
    gpu::Check(orator_device_synchronize());
    gpu::Check(orator_memcpy_dtoh(out.data(), d, sizeof(float) * out.size()));
    return out;
  }

 private:
  AsrTextConfig config_;
  void* h_ = nullptr;
};

}  // namespace model

namespace gemm {  // include/model/gemm.cuh:160-174, 251-268, 483-501

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

inline void LaunchBf16Gemm(const uint16_t* in, const uint16_t* W, const float* bias, float* out,
                           int M, int K, int N, int act, hipStream_t stream) {
  gpu::Check(orator_bf16_gemm(in, W, bias, out, M, K, N, act, stream));
}

}  // namespace gemm
}  // namespace orator
