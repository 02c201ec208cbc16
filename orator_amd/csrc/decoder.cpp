// The ASR text decoder on the attention path: prefill, single-token decode and greedy
// decoding with the reference's stop rules, composed from this library's operators.
//
// Mirrors AsrTextDecoder (include/model/asr_text_decoder.h:45-186,
// src/model/asr_text_decoder.cu:360-889):
//  * Forward (prefill, :457-583): per layer RmsNorm -> bf16 -> q, k, v projections ->
//    QK-RMSNorm + RoPE + KV write (one fused launch here) -> causal attention over the cache
//    (fp32-mode MFMA kernel) -> o projection + residual -> RmsNorm -> gate, up -> SwiGLU ->
//    down + residual; then the last row's final norm and the LM head.
//  * DecodeForwardOnStream (:360-455): the same with M = 1 projections (one fused q|k|v and
//    one gate|up GEMV) and the split-K decode attention; everything on the stream, reading
//    the position from a device scalar, allocation-free -- so one step can be captured in a
//    graph and replayed at any position.
//  * DecodeGreedy (:698-889): seed argmax of the prefill logits (EOS banned while fewer than
//    ban_steps tokens exist), then step bodies (record token, embed gather, forward, banned
//    argmax, position + 1) in batches with one host sync per batch; the host harvests the
//    recorded tokens and stops at EOS (not emitted) or after 6 identical tokens in a row (the
//    6th is emitted).  Steps past the stop in the same batch still advance the cache length,
//    as in the reference.  Two graphs (EOS banned / not) are captured once and replayed;
//    without graphs the same bodies run eagerly.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <new>
#include <vector>

#include "internal.hpp"

namespace orator_hip {
namespace {

// Longest context a decoder accepts: the decode split merge covers 1024 splits of 128 keys.
constexpr int kDecoderMaxSeq = 131072;

template <typename T>
int dalloc(T** p, size_t n) {
  *p = nullptr;
  if (n == 0) return ORATOR_OK;
  return check_hip(hipMalloc(reinterpret_cast<void**>(p), n * sizeof(T)), "decoder hipMalloc");
}

// Three events on a stream: start, mark, finish -> (start..mark, mark..finish) in ms.
struct Timer {
  hipEvent_t e[3] = {nullptr, nullptr, nullptr};
  ~Timer() {
    for (hipEvent_t x : e)
      if (x) (void)hipEventDestroy(x);
  }
  void start(hipStream_t s) {
    for (hipEvent_t& x : e)
      if (hipEventCreate(&x) != hipSuccess) x = nullptr;
    if (e[0]) (void)hipEventRecord(e[0], s);
  }
  void mark(hipStream_t s) {
    if (e[1]) (void)hipEventRecord(e[1], s);
  }
  bool finish(hipStream_t s, float* a, float* b) {
    if (!e[0] || !e[1] || !e[2]) return false;
    if (hipEventRecord(e[2], s) != hipSuccess || hipEventSynchronize(e[2]) != hipSuccess)
      return false;
    return hipEventElapsedTime(a, e[0], e[1]) == hipSuccess &&
           hipEventElapsedTime(b, e[1], e[2]) == hipSuccess;
  }
};

struct Decoder {
  OratorDecoderConfig c{};
  const uint16_t* embed = nullptr;
  const float* final_norm = nullptr;
  const uint16_t* lm_head = nullptr;
  std::vector<OratorDecoderLayer> layers;
  std::vector<uint16_t*> kc, vc;  // per layer [max_seq_len][Hkv][Dh] bf16
  int cache_len = 0;

  // prefill scratch (grown to the prefill length)
  int cap_t = 0;
  float *x = nullptr, *q = nullptr, *kv = nullptr, *attn = nullptr, *proj = nullptr,
        *gu = nullptr;
  uint16_t *norm_bf16 = nullptr, *act_bf16 = nullptr;
  int* pos_dev = nullptr;  // [cap_t + 1]: positions, then pos0
  int* pos_host = nullptr; // pinned staging
  // decode-step scratch (fixed addresses: captured graphs bake them in)
  float *sx = nullptr, *sqkv = nullptr, *sattn = nullptr, *sgateup = nullptr, *logits = nullptr;
  float* rope = nullptr;  // [max_seq_len][64][cos, sin]: the step's RoPE without fp64 trig
  void* argmax_scratch = nullptr;
  int *spos = nullptr, *stok = nullptr, *scount = nullptr, *sout = nullptr;
  int sout_cap = 0;
  int* host_int = nullptr;  // pinned staging for scalars
  hipStream_t capture_stream = nullptr;
  // profile (c.profile): per-token GPU time of eager default-stream decode steps
  double prof_sum_ms = 0.0;
  int prof_count = 0;
  bool prof_prefill_printed = false;
  hipGraphExec_t graph = nullptr, graph_banned = nullptr;
  bool graph_ready = false;
  int graph_ban0 = -1, graph_ban1 = -1;

  int Qd() const { return c.num_q_heads * c.head_dim; }
  int KVd() const { return c.num_kv_heads * c.head_dim; }
  float scale() const { return 1.0f / std::sqrt(static_cast<float>(c.head_dim)); }

  ~Decoder() {
    if (graph) (void)hipGraphExecDestroy(graph);
    if (graph_banned) (void)hipGraphExecDestroy(graph_banned);
    if (capture_stream) {
      // the graphs are gone: the capture stream's workspace (decode partials) goes too
      (void)workspace_release(capture_stream);
      (void)hipStreamDestroy(capture_stream);
    }
    for (auto* p : kc) (void)hipFree(p);
    for (auto* p : vc) (void)hipFree(p);
    free_prefill();
    for (void* p : {(void*)sx, (void*)sqkv, (void*)sattn, (void*)sgateup, (void*)logits,
                    argmax_scratch, (void*)spos, (void*)stok, (void*)scount, (void*)sout,
                    (void*)rope})
      if (p) (void)hipFree(p);
    if (host_int) (void)hipHostFree(host_int);
  }

  void free_prefill() {
    for (void* p : {(void*)x, (void*)q, (void*)kv, (void*)attn, (void*)proj, (void*)gu,
                    (void*)norm_bf16, (void*)act_bf16, (void*)pos_dev})
      if (p) (void)hipFree(p);
    if (pos_host) (void)hipHostFree(pos_host);
    x = q = kv = attn = proj = gu = nullptr;
    norm_bf16 = act_bf16 = nullptr;
    pos_dev = pos_host = nullptr;
    cap_t = 0;
  }

  int init() {
    const size_t cache = static_cast<size_t>(c.max_seq_len) * KVd();
    kc.assign(c.num_layers, nullptr);
    vc.assign(c.num_layers, nullptr);
    for (int l = 0; l < c.num_layers; ++l) {
      if (int rc = dalloc(&kc[l], cache)) return rc;
      if (int rc = dalloc(&vc[l], cache)) return rc;
      if (int rc = check_hip(hipMemset(kc[l], 0, cache * 2), "decoder cache clear")) return rc;
      if (int rc = check_hip(hipMemset(vc[l], 0, cache * 2), "decoder cache clear")) return rc;
    }
    const int H = c.hidden_size, I = c.intermediate_size;
    int rc = 0;
    if ((rc = dalloc(&sx, H)) || (rc = dalloc(&sqkv, Qd() + 2 * KVd())) ||
        (rc = dalloc(&sattn, Qd())) || (rc = dalloc(&sgateup, 2 * I)) ||
        (rc = dalloc(&logits, c.vocab_size)) || (rc = dalloc(&spos, 1)) ||
        (rc = dalloc(&stok, 1)) || (rc = dalloc(&scount, 1)) ||
        (rc = dalloc(&rope, static_cast<size_t>(c.max_seq_len) * 128)) ||
        (rc = launch_rope_table(rope, c.max_seq_len, c.rope_theta, nullptr)) ||
        (rc = check_hip(hipDeviceSynchronize(), "decoder rope table")))
      return rc;
    if (const size_t n = argmax_scratch_bytes(c.vocab_size))
      if ((rc = dalloc(reinterpret_cast<char**>(&argmax_scratch), n))) return rc;
    if ((rc = check_hip(hipHostMalloc(reinterpret_cast<void**>(&host_int), 4 * sizeof(int)),
                        "decoder pinned scalars")))
      return rc;
    return check_hip(hipStreamCreate(&capture_stream), "decoder capture stream");
  }

  int grow_prefill(int T) {
    if (T <= cap_t) return ORATOR_OK;
    free_prefill();
    const size_t H = c.hidden_size, I = c.intermediate_size, t = T;
    int rc = 0;
    const size_t act = std::max<size_t>(Qd(), I);
    if ((rc = dalloc(&x, t * H)) || (rc = dalloc(&q, t * Qd())) ||
        (rc = dalloc(&kv, t * 2 * KVd())) || (rc = dalloc(&attn, t * Qd())) ||
        (rc = dalloc(&proj, t * H)) || (rc = dalloc(&gu, t * 2 * I)) ||
        (rc = dalloc(&norm_bf16, t * H)) || (rc = dalloc(&act_bf16, t * act)) ||
        (rc = dalloc(&pos_dev, t + 1)))
      return rc;
    if ((rc = check_hip(hipHostMalloc(reinterpret_cast<void**>(&pos_host), (t + 1) * sizeof(int)),
                        "decoder pinned positions")))
      return rc;
    cap_t = T;
    return ORATOR_OK;
  }

  // act_bf16 = bf16(SwiGLU(norm_bf16 . gateup_w^T)) for T rows: one GEMM with the SwiGLU in
  // its epilogue; a single row runs the GEMV and the standalone SwiGLU pass (same values).
  int gate_up_swiglu(const uint16_t* gateup_w, int T, hipStream_t s) {
    const int H = c.hidden_size, I = c.intermediate_size;
    if (T > 1) return launch_gemm_bf16_swiglu(norm_bf16, gateup_w, act_bf16, gu, T, H, I, s);
    if (int rc = orator_linear_pre(norm_bf16, gateup_w, nullptr, gu, T, H, 2 * I, 0, s))
      return rc;
    return launch_swiglu_bf16(gu, act_bf16, T, I, s);
  }

  // Forward of T rows of residual stream x at positions pos0.. (asr_text_decoder.cu:457-583).
  int forward(int T, int pos0, hipStream_t s) {
    const int H = c.hidden_size, I = c.intermediate_size, Hq = c.num_q_heads,
              Hkv = c.num_kv_heads, Dh = c.head_dim;
    const float eps = c.rms_norm_eps;
    // profile: a single-row forward times its layer loop and its final norm + LM head
    // (asr_text_decoder.cu:504-583), printed once per decoder
    Timer prof;
    const bool timed = c.profile && T == 1 && !prof_prefill_printed;
    if (timed) prof.start(s);
    for (int t = 0; t < T; ++t) pos_host[t] = pos0 + t;
    pos_host[T] = pos0;
    int rc = check_hip(hipMemcpyAsync(pos_dev, pos_host, sizeof(int) * (T + 1),
                                      hipMemcpyHostToDevice, s),
                       "decoder positions");
    const int* d_pos0 = pos_dev + T;
    // Per layer, the reference's passes with the casts and residual adds folded in (same
    // fp32 values rounded once each): RmsNorm -> bf16, q and k|v projections (row slices of
    // the fused qkv weight), QK-norm/RoPE/KV write, attention, bf16 cast, o projection += x,
    // RmsNorm -> bf16, the fused gate|up projection with SwiGLU -> bf16 in its epilogue, down
    // projection += x.
    const long TQ = static_cast<long>(T) * Qd();
    for (int li = 0; li < c.num_layers && !rc; ++li) {
      const OratorDecoderLayer& L = layers[li];
      (rc = launch_rms_norm_bf16(x, L.in_ln, norm_bf16, T, H, eps, s)) ||
          (rc = orator_linear_pre(norm_bf16, L.qkv_w, nullptr, q, T, H, Qd(), 0, s)) ||
          (rc = orator_linear_pre(norm_bf16, L.qkv_w + static_cast<size_t>(Qd()) * H, nullptr,
                                  kv, T, H, 2 * KVd(), 0, s)) ||
          (rc = launch_qk_norm_rope_kv(q, kv, kv + KVd(), Qd(), 2 * KVd(), L.q_norm, L.k_norm,
                                       eps, pos_dev, c.rope_theta, rope, c.max_seq_len, T, T,
                                       Hq, Hkv, Dh, kc[li], vc[li], nullptr, 0, 0, c.max_seq_len,
                                       s)) ||
          (rc = orator_gqa_prefill(q, kc[li], vc[li], attn, T, Hq, Hkv, Dh, d_pos0,
                                   c.max_seq_len, scale(), s)) ||
          (rc = orator_f32_to_bf16(attn, act_bf16, TQ, s)) ||
          (rc = launch_linear_pre_acc(act_bf16, L.o_w, x, T, Qd(), H, proj, s)) ||
          (rc = launch_rms_norm_bf16(x, L.post_ln, norm_bf16, T, H, eps, s)) ||
          (rc = gate_up_swiglu(L.gateup_w, T, s)) ||
          (rc = launch_linear_pre_acc(act_bf16, L.down_w, x, T, I, H, proj, s));
    }
    if (rc) return rc;
    cache_len = pos0 + T;
    if (timed) prof.mark(s);
    const float* last = x + static_cast<size_t>(T - 1) * H;
    rc = launch_gemv_fused(kGemvInRmsNorm, last, final_norm, eps, lm_head, logits, H,
                           c.vocab_size, false, s);
    if (timed && !rc) {
      float layers_ms = 0.0f, head_ms = 0.0f;
      if (prof.finish(s, &layers_ms, &head_ms)) {
        std::fprintf(stderr, "[dec2] %d-layer loop=%.2fms lm_head+norm=%.2fms\n", c.num_layers,
                     layers_ms, head_ms);
        prof_prefill_printed = true;
      }
    }
    return rc;
  }

  // profile: GPU time of one eager decode step on the default stream
  // (asr_text_decoder.cu:369-377, 439-454); the running average is printed every 16 steps.
  int decode_forward_profiled(hipStream_t s) {
    if (!(c.profile && s == nullptr)) return decode_forward(s);
    Timer prof;
    prof.start(s);
    const int rc = decode_forward(s);
    float ms = 0.0f, unused = 0.0f;
    prof.mark(s);
    if (!rc && prof.finish(s, &ms, &unused)) {
      prof_sum_ms += ms;
      if (++prof_count % 16 == 0)
        std::fprintf(stderr, "[dec2] per-token GPU compute avg = %.3f ms (n=%d)\n",
                     prof_sum_ms / prof_count, prof_count);
    }
    return rc;
  }

  // One-token forward of sx at the device position spos (asr_text_decoder.cu:360-455).
  // Each projection is one fused GEMV that builds its bf16 input row from the fp32 producer
  // (RmsNorm -> cast, or cast); gate|up stores silu(gate) * up directly, and the o / down
  // projections add into the residual stream in their store: per layer 6 launches instead
  // of the reference's 16.
  int decode_forward(hipStream_t s) {
    const int H = c.hidden_size, I = c.intermediate_size, Hq = c.num_q_heads,
              Hkv = c.num_kv_heads, Dh = c.head_dim;
    const float eps = c.rms_norm_eps;
    float* dq = sqkv;
    float* dk = sqkv + Qd();
    float* dv = sqkv + Qd() + KVd();
    int rc = 0;
    for (int li = 0; li < c.num_layers && !rc; ++li) {
      const OratorDecoderLayer& L = layers[li];
      // attention of the step: QK-norm, RoPE (the position's table row), the KV write of the
      // new row and the split-K attention in one launch, plus the split merge
      DecodeProblem p{};
      p.q = dq;
      p.kpool = kc[li];
      p.vpool = vc[li];
      p.pos = spos;
      p.out = sattn;
      p.B = 1;
      p.Hq = Hq;
      p.Hkv = Hkv;
      p.Dh = Dh;
      p.capacity = c.max_seq_len;
      p.scale = scale();
      p.k_new = dk;
      p.v_new = dv;
      p.pool_rows = c.max_seq_len;
      p.q_norm = L.q_norm;
      p.k_norm = L.k_norm;
      p.rope = rope;
      p.eps = eps;
      (rc = launch_gemv_fused(kGemvInRmsNorm, sx, L.in_ln, eps, L.qkv_w, sqkv, H,
                              Qd() + 2 * KVd(), false, s)) ||
          (rc = launch_gqa_decode(p, s)) ||
          (rc = launch_gemv_fused(kGemvInF32, sattn, nullptr, 0.0f, L.o_w, sx, Qd(), H, true, s)) ||
          (rc = launch_gemv_fused(kGemvInRmsNorm, sx, L.post_ln, eps, L.gateup_w, sgateup, H, I,
                                  false, s, /*pair=*/true)) ||
          (rc = launch_gemv_fused(kGemvInF32, sgateup, nullptr, 0.0f, L.down_w, sx, I, H, true,
                                  s));
    }
    if (rc) return rc;
    return launch_gemv_fused(kGemvInRmsNorm, sx, final_norm, eps, lm_head, logits, H,
                             c.vocab_size, false, s);
  }

  int argmax(int ban0, int ban1, int* d_out, hipStream_t s) {
    return launch_argmax_banned(logits, c.vocab_size, ban0, ban1, d_out, argmax_scratch, s);
  }

  // Greedy step body (asr_text_decoder.cu:677-691): record, gather, forward, argmax, pos + 1.
  int body(hipStream_t s, int ban0, int ban1) {
    int rc = 0;
    (rc = orator_record_token(sout, scount, stok, sout_cap, s)) ||
        (rc = orator_embed_gather(embed, stok, sx, c.hidden_size, s)) ||
        (rc = decode_forward(s)) ||
        (rc = argmax(ban0, ban1, stok, s)) ||
        (rc = orator_inc_pos(spos, s));
    return rc;
  }

  int set_int(int* dst, int v, hipStream_t s) {
    *host_int = v;
    int rc = check_hip(hipMemcpyAsync(dst, host_int, sizeof(int), hipMemcpyHostToDevice, s),
                       "decoder scalar");
    return rc ? rc : check_hip(hipStreamSynchronize(s), "decoder sync");
  }

  void drop_graphs() {
    if (graph) (void)hipGraphExecDestroy(graph);
    if (graph_banned) (void)hipGraphExecDestroy(graph_banned);
    graph = graph_banned = nullptr;
    graph_ready = false;
  }

  int capture(int b0, int b1, hipGraphExec_t* exec) {
    *exec = nullptr;
    if (int rc = check_hip(hipStreamBeginCapture(capture_stream, hipStreamCaptureModeThreadLocal),
                           "decoder begin capture"))
      return rc;
    const int rc_body = body(capture_stream, b0, b1);
    hipGraph_t g = nullptr;
    const hipError_t end = hipStreamEndCapture(capture_stream, &g);
    if (rc_body) {
      if (g) (void)hipGraphDestroy(g);
      return rc_body;
    }
    if (int rc = check_hip(end, "decoder end capture")) return rc;
    const hipError_t inst = hipGraphInstantiate(exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    return check_hip(inst, "decoder graph instantiate");
  }

  int decode_greedy(int start_pos, int max_new, int eos0, int eos1, int ban_steps, int batch,
                    bool use_graph, std::vector<int>& out, hipStream_t s) {
    out.clear();
    if (max_new <= 0) return ORATOR_OK;
    if (batch <= 0) batch = 1;
    if (max_new > sout_cap) {
      if (sout) (void)hipFree(sout);
      sout = nullptr;
      sout_cap = 0;
      if (int rc = dalloc(&sout, max_new)) return rc;
      sout_cap = max_new;
      drop_graphs();  // the graphs baked the old token buffer
    }
    if (graph_ready && (graph_ban0 != eos0 || graph_ban1 != eos1)) drop_graphs();
    int rc = check_hip(hipStreamSynchronize(s), "decoder sync");
    if (rc || (rc = set_int(spos, start_pos, s)) || (rc = set_int(scount, 0, s))) return rc;
    std::vector<int> h_out(max_new);
    bool stop = false;
    auto harvest = [&](int upto) -> int {
      if (int e = check_hip(hipMemcpy(h_out.data(), sout, sizeof(int) * upto,
                                      hipMemcpyDeviceToHost),
                            "decoder harvest"))
        return e;
      for (int i = static_cast<int>(out.size()); i < upto; ++i) {
        const int t = h_out[i];
        if (t == eos0 || t == eos1) {
          stop = true;
          return ORATOR_OK;
        }
        out.push_back(t);
        if (out.size() >= 6) {
          bool same = true;
          for (size_t kk = out.size() - 6; kk + 1 < out.size(); ++kk)
            if (out[kk] != out.back()) {
              same = false;
              break;
            }
          if (same) {
            stop = true;
            return ORATOR_OK;
          }
        }
      }
      return ORATOR_OK;
    };
    // profile: host-clock split of the call (asr_text_decoder.cu:762-889)
    using clk = std::chrono::steady_clock;
    const auto t_seed0 = clk::now();
    auto t_seed1 = t_seed0, t_loop0 = t_seed0;
    int batches = 0;
    double first_sync_ms = 0.0;
    auto report = [&]() {
      if (!c.profile) return;
      const auto ms = [](clk::time_point a, clk::time_point b) {
        return std::chrono::duration<double, std::milli>(b - a).count();
      };
      std::fprintf(stderr,
                   "[decprof] seed+drain=%.1fms loop=%.1fms (emitted=%d batches=%d"
                   " first_batch_sync=%.1fms)\n",
                   ms(t_seed0, t_seed1), ms(t_loop0, clk::now()), static_cast<int>(out.size()),
                   batches, first_sync_ms);
    };
    // seed: argmax of the prefill logits -> the first token
    const bool seed_ban = 0 < ban_steps;
    if ((rc = argmax(seed_ban ? eos0 : -1, seed_ban ? eos1 : -1, stok, s)) ||
        (rc = check_hip(hipStreamSynchronize(s), "decoder sync")))
      return rc;
    t_seed1 = t_loop0 = clk::now();
    int emitted = 0;
    if (use_graph && !graph_ready) {
      const bool ban_first = (0 + 1) < ban_steps;
      if ((rc = body(s, ban_first ? eos0 : -1, ban_first ? eos1 : -1)) ||
          (rc = check_hip(hipStreamSynchronize(s), "decoder sync")))
        return rc;
      ++emitted;
      // the decode attention's split partials and arrival counters live in the capture
      // stream's workspace
      if ((rc = decode_workspace_reserve(1, c.num_q_heads, c.head_dim, c.max_seq_len,
                                         capture_stream)))
        return rc;
      graph_ban0 = eos0;
      graph_ban1 = eos1;
      if (capture(eos0, eos1, &graph_banned) || capture(-1, -1, &graph)) {
        // as the reference (asr_text_decoder.cu:846-847): a failed capture leaves the
        // eager bodies in charge for this decoder
        drop_graphs();
        (void)hipGetLastError();
      }
      graph_ready = true;
      if (c.profile)
        std::fprintf(stderr, "[graph] ready (banned=%p normal=%p)\n",
                     static_cast<void*>(graph_banned), static_cast<void*>(graph));
      if ((rc = harvest(emitted))) return rc;
      if (stop) {
        cache_len = start_pos + emitted;
        report();
        return ORATOR_OK;
      }
    }
    if (!(use_graph && graph && graph_banned)) {
      while (emitted < max_new) {
        const bool next_ban = (emitted + 1) < ban_steps;
        const int this_batch = next_ban ? 1 : std::min(batch, max_new - emitted);
        const auto tb = clk::now();
        for (int b = 0; b < this_batch && !rc; ++b)
          rc = body(s, next_ban ? eos0 : -1, next_ban ? eos1 : -1);
        if (rc || (rc = check_hip(hipStreamSynchronize(s), "decoder sync"))) return rc;
        if (batches++ == 0)
          first_sync_ms = std::chrono::duration<double, std::milli>(clk::now() - tb).count();
        emitted += this_batch;
        if ((rc = harvest(emitted))) return rc;
        if (stop) break;
      }
      cache_len = start_pos + emitted;
      report();
      return ORATOR_OK;
    }
    while (emitted < max_new) {
      const bool in_ban = (emitted + 1) < ban_steps;
      hipGraphExec_t g = in_ban ? graph_banned : graph;
      const int limit = in_ban ? std::min(ban_steps - 1, max_new) : max_new;
      const int this_batch = std::max(1, std::min(batch, limit - emitted));
      const auto tb = clk::now();
      for (int b = 0; b < this_batch && !rc; ++b) rc = check_hip(hipGraphLaunch(g, s), "graph launch");
      if (rc || (rc = check_hip(hipStreamSynchronize(s), "decoder sync"))) return rc;
      if (batches++ == 0)
        first_sync_ms = std::chrono::duration<double, std::milli>(clk::now() - tb).count();
      emitted += this_batch;
      if ((rc = harvest(emitted))) return rc;
      if (stop) break;
    }
    cache_len = start_pos + emitted;
    report();
    return ORATOR_OK;
  }
};

Decoder* as_dec(void* h) { return static_cast<Decoder*>(h); }

}  // namespace
}  // namespace orator_hip

using namespace orator_hip;

extern "C" {

int orator_decoder_create(const OratorDecoderConfig* cfg, const uint16_t* embed,
                          const float* final_norm, const uint16_t* lm_head,
                          const OratorDecoderLayer* layers, void** handle) {
  if (!handle) return fail(ORATOR_ERR_INVALID, "decoder_create: null handle");
  *handle = nullptr;
  if (!cfg || !embed || !final_norm || !layers)
    return fail(ORATOR_ERR_INVALID, "decoder_create: null pointer");
  const OratorDecoderConfig& c = *cfg;
  if (c.num_layers <= 0 || c.hidden_size <= 0 || c.num_q_heads <= 0 || c.num_kv_heads <= 0 ||
      c.intermediate_size <= 0 || c.vocab_size <= 0 || c.max_seq_len <= 0)
    return fail(ORATOR_ERR_INVALID, "decoder_create: sizes must be positive");
  if (c.max_seq_len > kDecoderMaxSeq)
    return fail(ORATOR_ERR_UNSUPPORTED, "decoder_create: max_seq_len above 131072");
  if (c.head_dim != 128 || c.num_q_heads % c.num_kv_heads || c.hidden_size % 8 ||
      c.intermediate_size % 8 || c.hidden_size > kFusedMaxK || c.intermediate_size > kFusedMaxK ||
      c.num_q_heads * c.head_dim > kFusedMaxK)
    return fail(ORATOR_ERR_UNSUPPORTED,
                "decoder_create: head_dim 128, Hq multiple of Hkv, hidden and intermediate % 8, "
                "hidden, Hq * head_dim and intermediate <= 8192");
  for (int l = 0; l < c.num_layers; ++l) {
    const OratorDecoderLayer& L = layers[l];
    if (!L.in_ln || !L.q_norm || !L.k_norm || !L.post_ln || !L.qkv_w || !L.o_w || !L.gateup_w ||
        !L.down_w)
      return fail(ORATOR_ERR_INVALID, "decoder_create: null layer weight");
  }
  Decoder* d = new (std::nothrow) Decoder();
  if (!d) return fail(ORATOR_ERR_CAPACITY, "decoder_create: out of host memory");
  d->c = c;
  d->embed = embed;
  d->final_norm = final_norm;
  d->lm_head = lm_head ? lm_head : embed;  // tied (asr_text_decoder.cu:255-257)
  d->layers.assign(layers, layers + c.num_layers);
  if (int rc = d->init()) {
    delete d;
    return rc;
  }
  *handle = d;
  return ORATOR_OK;
}

int orator_decoder_destroy(void* handle) {
  delete as_dec(handle);
  return ORATOR_OK;
}

int orator_decoder_prefill_at(void* handle, const float* embeds, int T, int pos0, void* stream) {
  Decoder* d = as_dec(handle);
  if (!d || !embeds) return fail(ORATOR_ERR_INVALID, "decoder_prefill: null pointer");
  if (T <= 0) return ORATOR_OK;
  if (pos0 < 0 || pos0 + T > d->c.max_seq_len)
    return fail(ORATOR_ERR_CAPACITY, "decoder_prefill: positions past max_seq_len");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = d->grow_prefill(T);
  if (!rc)
    rc = check_hip(hipMemcpyAsync(d->x, embeds, sizeof(float) * T * d->c.hidden_size,
                                  hipMemcpyDefault, s),
                   "decoder embeds");
  if (!rc) rc = d->forward(T, pos0, s);
  return rc ? rc : check_hip(hipStreamSynchronize(s), "decoder sync");
}

int orator_decoder_decode_step(void* handle, const float* embed, int pos, void* stream) {
  Decoder* d = as_dec(handle);
  if (!d || !embed) return fail(ORATOR_ERR_INVALID, "decoder_decode_step: null pointer");
  if (pos < 0 || pos >= d->c.max_seq_len)
    return fail(ORATOR_ERR_CAPACITY, "decoder_decode_step: position past max_seq_len");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = check_hip(hipMemcpyAsync(d->sx, embed, sizeof(float) * d->c.hidden_size,
                                    hipMemcpyDefault, s),
                     "decoder embed");
  if (!rc) rc = d->set_int(d->spos, pos, s);
  d->cache_len = pos + 1;
  if (!rc) rc = d->decode_forward_profiled(s);
  return rc ? rc : check_hip(hipStreamSynchronize(s), "decoder sync");
}

int orator_decoder_decode_step_device(void* handle, const int* d_token, int pos, void* stream) {
  Decoder* d = as_dec(handle);
  if (!d || !d_token) return fail(ORATOR_ERR_INVALID, "decoder_decode_step_device: null pointer");
  if (pos < 0 || pos >= d->c.max_seq_len)
    return fail(ORATOR_ERR_CAPACITY, "decoder_decode_step_device: position past max_seq_len");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = d->set_int(d->spos, pos, s);
  d->cache_len = pos + 1;
  if (!rc) rc = orator_embed_gather(d->embed, d_token, d->sx, d->c.hidden_size, s);
  return rc ? rc : d->decode_forward_profiled(s);
}

int orator_decoder_argmax_to_device(void* handle, int* d_out, int ban0, int ban1, void* stream) {
  Decoder* d = as_dec(handle);
  if (!d || !d_out) return fail(ORATOR_ERR_INVALID, "decoder_argmax_to_device: null pointer");
  return d->argmax(ban0, ban1, d_out, static_cast<hipStream_t>(stream));
}

int orator_decoder_embed(void* handle, int token_id, float* out) {
  Decoder* d = as_dec(handle);
  if (!d || !out) return fail(ORATOR_ERR_INVALID, "decoder_embed: null pointer");
  if (token_id < 0 || token_id >= d->c.vocab_size)
    return fail(ORATOR_ERR_INVALID, "decoder_embed: token id out of range");
  const int H = d->c.hidden_size;
  std::vector<uint16_t> row(H);
  if (int rc = check_hip(hipMemcpy(row.data(), d->embed + static_cast<size_t>(token_id) * H,
                                   sizeof(uint16_t) * H, hipMemcpyDeviceToHost),
                         "decoder_embed copy"))
    return rc;
  for (int i = 0; i < H; ++i) {
    const uint32_t bits = static_cast<uint32_t>(row[i]) << 16;
    std::memcpy(out + i, &bits, sizeof(float));
  }
  return ORATOR_OK;
}

int orator_decoder_reset(void* handle) {
  Decoder* d = as_dec(handle);
  if (!d) return fail(ORATOR_ERR_INVALID, "decoder_reset: null handle");
  d->cache_len = 0;
  return ORATOR_OK;
}

int orator_decoder_argmax(void* handle, int ban0, int ban1, int* token, void* stream) {
  Decoder* d = as_dec(handle);
  if (!d || !token) return fail(ORATOR_ERR_INVALID, "decoder_argmax: null pointer");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = d->argmax(ban0, ban1, d->stok, s);
  if (!rc) rc = check_hip(hipMemcpyAsync(d->host_int, d->stok, sizeof(int), hipMemcpyDeviceToHost, s),
                          "decoder argmax copy");
  if (!rc) rc = check_hip(hipStreamSynchronize(s), "decoder sync");
  if (!rc) *token = *d->host_int;
  return rc;
}

int orator_decoder_logits(void* handle, float** d_logits) {
  Decoder* d = as_dec(handle);
  if (!d || !d_logits) return fail(ORATOR_ERR_INVALID, "decoder_logits: null pointer");
  *d_logits = d->logits;
  return ORATOR_OK;
}

int orator_decoder_decode_greedy(void* handle, int start_pos, int max_new, int eos0, int eos1,
                                 int ban_steps, int batch, int use_graph, int* tokens,
                                 int* n_tokens, void* stream) {
  Decoder* d = as_dec(handle);
  if (!d || !n_tokens || (max_new > 0 && !tokens))
    return fail(ORATOR_ERR_INVALID, "decoder_decode_greedy: null pointer");
  *n_tokens = 0;
  if (start_pos < 0 || start_pos + max_new > d->c.max_seq_len)
    return fail(ORATOR_ERR_CAPACITY, "decoder_decode_greedy: positions past max_seq_len");
  std::vector<int> out;
  const int rc = d->decode_greedy(start_pos, max_new, eos0, eos1, ban_steps, batch, use_graph != 0,
                                  out, static_cast<hipStream_t>(stream));
  if (rc) return rc;
  if (!out.empty()) std::memcpy(tokens, out.data(), sizeof(int) * out.size());
  *n_tokens = static_cast<int>(out.size());
  return ORATOR_OK;
}

int orator_decoder_truncate(void* handle, int len) {
  Decoder* d = as_dec(handle);
  if (!d) return fail(ORATOR_ERR_INVALID, "decoder_truncate: null handle");
  d->cache_len = len;
  return ORATOR_OK;
}

int orator_decoder_cache_len(void* handle, int* len) {
  Decoder* d = as_dec(handle);
  if (!d || !len) return fail(ORATOR_ERR_INVALID, "decoder_cache_len: null pointer");
  *len = d->cache_len;
  return ORATOR_OK;
}

}  // extern "C"
