// The reference's decoder test, run through the C++ drop-in header (orator_attn.hpp).
//
// Same structure and gates as test/unit/model/test_asr_decoder.cc after its oracle check
// (which needs the checkpoint and a PyTorch dump, absent here; the Python suite checks the
// logits against the CPU oracle instead): on a small random-weight decoder,
//   * Prefill, then PrefillAt in two parts (pos0 = split): cache_len == T, identical argmax,
//     logits max abs diff <= 0.5 (test_asr_decoder.cc:76-112);
//   * TruncateCache(split) + PrefillAt of the second part: identical argmax (:114-127);
// and, for the greedy loop: DecodeGreedy with graph replay == DecodeGreedy eager after the same
// single-call prefill, token for token, and cache_len == start + tokens run.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "orator_attn.hpp"

using orator::model::AsrTextConfig;
using orator::model::AsrTextDecoder;

namespace {

struct Rng {  // xorshift64*
  uint64_t s;
  explicit Rng(uint64_t seed) : s(seed * 2654435761u + 1) {}
  uint64_t next() {
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return s * 0x2545F4914F6CDD1DULL;
  }
  float uniform() { return static_cast<float>((next() >> 40) * (1.0 / 16777216.0)); }
};

uint16_t to_bf16(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

template <typename T>
T* upload(const std::vector<T>& h) {
  void* p = nullptr;
  orator::gpu::Check(orator_malloc(&p, h.size() * sizeof(T)));
  orator::gpu::Check(orator_memcpy_htod(p, h.data(), h.size() * sizeof(T)));
  return static_cast<T*>(p);
}

std::vector<uint16_t> bf16_matrix(Rng& r, size_t n, float scale) {
  std::vector<uint16_t> w(n);
  for (auto& x : w) x = to_bf16((2.0f * r.uniform() - 1.0f) * scale);
  return w;
}

std::vector<float> gains(Rng& r, size_t n) {
  std::vector<float> g(n);
  for (auto& x : g) x = 1.0f + 0.2f * (r.uniform() - 0.5f);
  return g;
}

}  // namespace

int main() {
  std::printf("Testing the ASR text decoder through the C++ drop-in...\n");
  AsrTextConfig c;
  c.num_layers = 2;
  c.hidden_size = 512;
  c.num_q_heads = 4;
  c.num_kv_heads = 2;
  c.head_dim = 128;
  c.intermediate_size = 1024;
  c.vocab_size = 4096;
  c.max_seq_len = 256;
  const int H = c.hidden_size, I = c.intermediate_size, V = c.vocab_size;
  const int Qd = c.num_q_heads * c.head_dim, KVd = c.num_kv_heads * c.head_dim;
  Rng r(2024);
  std::vector<void*> owned;
  auto keep = [&](auto* p) {
    owned.push_back(p);
    return p;
  };
  const uint16_t* embed = keep(upload(bf16_matrix(r, static_cast<size_t>(V) * H, 0.03f)));
  const uint16_t* lm_head = keep(upload(bf16_matrix(r, static_cast<size_t>(V) * H, 0.03f)));
  const float* final_norm = keep(upload(gains(r, H)));
  std::vector<OratorDecoderLayer> layers(c.num_layers);
  for (auto& L : layers) {
    L.in_ln = keep(upload(gains(r, H)));
    L.q_norm = keep(upload(gains(r, c.head_dim)));
    L.k_norm = keep(upload(gains(r, c.head_dim)));
    L.post_ln = keep(upload(gains(r, H)));
    L.qkv_w = keep(upload(bf16_matrix(r, static_cast<size_t>(Qd + 2 * KVd) * H, 0.03f)));
    L.o_w = keep(upload(bf16_matrix(r, static_cast<size_t>(H) * Qd, 0.03f)));
    L.gateup_w = keep(upload(bf16_matrix(r, static_cast<size_t>(2 * I) * H, 0.03f)));
    L.down_w = keep(upload(bf16_matrix(r, static_cast<size_t>(H) * I, 0.03f)));
  }
  const int T = 60, split = T / 2;
  std::vector<float> embeds(static_cast<size_t>(T) * H);
  for (auto& x : embeds) x = 0.04f * (r.uniform() - 0.5f);

  int failures = 0;
  {
    AsrTextDecoder dec(c, embed, final_norm, lm_head, layers.data());
    dec.ResetCache();
    dec.Prefill(embeds.data(), T);
    const std::vector<float> logits = dec.CopyLogits();
    const int our_am = dec.Argmax();
    std::printf("  prompt T=%d hidden=%d vocab=%d argmax=%d\n", T, H, V, our_am);

    std::printf("\nT010: incremental PrefillAt append equivalence...\n");
    dec.ResetCache();
    dec.PrefillAt(embeds.data(), split, 0);
    dec.PrefillAt(embeds.data() + static_cast<size_t>(split) * H, T - split, split);
    if (dec.cache_len() != T) {
      std::printf("FAIL: cache_len=%d expected %d\n", dec.cache_len(), T);
      ++failures;
    }
    const std::vector<float> inc = dec.CopyLogits();
    const int inc_am = dec.Argmax();
    double diff = 0.0;
    for (int i = 0; i < V; ++i) diff = std::max(diff, std::fabs(double(inc[i]) - logits[i]));
    std::printf("  split=%d argmax inc=%d single=%d ; logits max abs diff = %.3e\n", split, inc_am,
                our_am, diff);
    if (inc_am != our_am || diff > 0.5) {
      std::printf("FAIL: incremental prefill\n");
      ++failures;
    }
    dec.TruncateCache(split);
    if (dec.cache_len() != split) {
      std::printf("FAIL: TruncateCache did not set cache_len\n");
      ++failures;
    }
    dec.PrefillAt(embeds.data() + static_cast<size_t>(split) * H, T - split, split);
    const int retry_am = dec.Argmax();
    if (retry_am != our_am) {
      std::printf("FAIL: re-prefill after truncate argmax mismatch (%d vs %d)\n", retry_am,
                  our_am);
      ++failures;
    }
    // Graph replay against eager launches from the same history: both decoders prefill the
    // whole prompt in one call (a split prefill may round the cache differently, since the
    // projection GEMM of a 60-row prompt and of two 30-row parts need not sum in one order).
    dec.Prefill(embeds.data(), T);
    const std::vector<int> graph = dec.DecodeGreedy(T, 24, 151645, 151643, 3, 4);
    const int graph_len = dec.cache_len();
    std::printf("  greedy (graph): %zu tokens, cache_len %d\n", graph.size(), graph_len);

    AsrTextConfig ce = c;
    ce.cuda_graph_enabled = false;
    AsrTextDecoder eager(ce, embed, final_norm, lm_head, layers.data());
    eager.Prefill(embeds.data(), T);
    const std::vector<int> eag = eager.DecodeGreedy(T, 24, 151645, 151643, 3, 4);
    if (eag != graph || eager.cache_len() != graph_len || graph.empty()) {
      std::printf("FAIL: eager greedy differs from the replayed graphs (%zu vs %zu tokens)\n",
                  eag.size(), graph.size());
      ++failures;
    }
  }
  for (void* p : owned) (void)orator_free(p);
  if (failures) return 1;
  std::printf("ASR text decoder drop-in test PASSED\n");
  return 0;
}
