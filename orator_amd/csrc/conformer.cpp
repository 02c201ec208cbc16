// One FastConformer layer, the Sortformer encoder's (ConformerLayer::Forward,
// src/model/conformer_layer.cu:364-488), composed from this library's operators:
//   x += 0.5 FFN1(LN(x))                                   FFN: Linear+SiLU, Linear
//   x += MHSA(LN(x))        linear_q/k/v, linear_pos(pos_emb), rel-pos attention, linear_out
//   x += Conv(LN(x))        pointwise 2C + GLU (+ padding-row mask) in one launch, depthwise K,
//                           BatchNorm(eval)+SiLU, pointwise C
//   x += 0.5 FFN2(LN(x));  x = LN_out(x)
// The projections run on the fp32 MFMA SGEMM; the attention core is either the reference
// decomposition in fp32 (attn_mode 0) or the fused fp16 MFMA kernel (attn_mode 1).  Each
// residual update x += s * (h W^T + b) is the last projection's epilogue or split-K reduce
// (the same fp32 value, then one fused multiply-add, exact for s = 0.5 and 1), and that reduce
// also writes the next block's LayerNorm of x (the closing one in place); q/k/v are one grouped
// launch sharing LN(x).
#include <hip/hip_runtime.h>

#include <cmath>
#include <new>
#include <vector>

#include "internal.hpp"

namespace orator_hip {

int launch_glu_mask(const float* in, float* out, int T, int C, int valid, hipStream_t s);
int launch_dwconv_bn_silu(const float* in, const float* w, const float* bias, const float* mean,
                          const float* var, const float* gamma, const float* beta, float* out,
                          int T, int C, int K, float eps, hipStream_t s);

namespace {

constexpr float kEps = 1e-5f;  // conformer_layer.cu:368

struct Conformer {
  int D = 0, H = 0, Dff = 0, K = 0;
  OratorConformerWeights w{};
  int cap_t = 0;
  float *ln = nullptr, *ff = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *p = nullptr,
        *ctx = nullptr, *pw1 = nullptr, *glu = nullptr, *dw = nullptr;

  ~Conformer() { release(); }

  void release() {
    for (float* b : {ln, ff, q, k, v, p, ctx, pw1, glu, dw})
      if (b) (void)hipFree(b);
    ln = ff = q = k = v = p = ctx = pw1 = glu = dw = nullptr;
    cap_t = 0;
  }

  int grow(int T) {
    if (T <= cap_t) return ORATOR_OK;
    release();
    const size_t t = T, P = 2 * t - 1;
    const std::pair<float**, size_t> bufs[] = {
        {&ln, t * D}, {&ff, t * Dff},     {&q, t * D},   {&k, t * D},  {&v, t * D},
        {&p, P * D},  {&ctx, t * D},      {&pw1, 2 * t * D}, {&glu, t * D}, {&dw, t * D}};
    for (const auto& [ptr, n] : bufs)
      if (int rc = check_hip(hipMalloc(reinterpret_cast<void**>(ptr), n * sizeof(float)),
                             "conformer scratch"))
        return rc;
    cap_t = T;
    return ORATOR_OK;
  }

  int linear(const float* in, const float* W, const float* b, float* out, int M, int Kd, int N,
             int act, hipStream_t s) {
    return orator_sgemm(in, W, b, out, M, Kd, N, act, s);
  }

  // pointwise_conv1 + GLU + padding-row mask: one launch when the product takes 16-byte
  // loads, else the product then the GLU pass (the same values either way)
  int pw1_glu(int T, int valid, hipStream_t s) {
    const int rc = launch_sgemm_glu(ln, w.pw1_w, w.pw1_b, glu, T, D, D, valid, s);
    if (rc != ORATOR_ERR_UNSUPPORTED) return rc;
    if (int r = linear(ln, w.pw1_w, w.pw1_b, pw1, T, D, 2 * D, 0, s)) return r;
    return launch_glu_mask(pw1, glu, T, D, valid, s);
  }

  // q, k, v projections in one launch; with the fused core (f16_kv) k and v are written as
  // the fp16 values that core would round them to on load, and q stays fp32 (q + u and q + v
  // are formed in fp32 before their one rounding)
  int qkv(int T, bool f16_kv, hipStream_t s) {
    const float* const W[3] = {w.q_w, w.k_w, w.v_w};
    const float* const b[3] = {w.q_b, w.k_b, w.v_b};
    void* const out[3] = {q, k, v};
    return launch_sgemm_group3(ln, W, b, out, T, D, D, f16_kv ? 6 : 0, s);
  }

  // x += 0.5 FFN(ln) (ln = this block's LayerNorm of x), then next_out = the next block's
  // LayerNorm of the updated x (ng, nb)
  int ffn(float* x, int T, const float* w1, const float* b1, const float* w2, const float* b2,
          const float* ng, const float* nb, float* next_out, hipStream_t s) {
    int rc = 0;
    (rc = linear(ln, w1, b1, ff, T, D, Dff, 1, s)) ||  // SiLU
        (rc = launch_sgemm_residual_ln(ff, w2, b2, x, T, Dff, D, 0.5f, ng, nb, next_out, kEps, s));
    return rc;
  }

  int forward(float* x, int T, int valid, const float* pos_emb, int attn_mode, hipStream_t s) {
    if (int rc = grow(T)) return rc;
    const int P = 2 * T - 1, Dk = D / H;
    const float scale = 1.0f / std::sqrt(static_cast<float>(Dk));
    int rc = 0;
    // FFN1.  Its LayerNorm is the only separate one: every residual update below also writes
    // the next block's LayerNorm of x (into `ln`, whose previous contents are consumed by then;
    // the last one, norm_out, into x itself).
    (rc = launch_layer_norm(x, w.norm_ff1_w, w.norm_ff1_b, ln, T, D, kEps, s)) ||
        (rc = ffn(x, T, w.ff1_w1, w.ff1_b1, w.ff1_w2, w.ff1_b2, w.norm_att_w, w.norm_att_b, ln, s));
    if (rc) return rc;
    // MHSA (the fused core reads k, v and p as fp16: half the bytes written and read)
    (rc = qkv(T, attn_mode == 1, s)) ||
        (rc = attn_mode == 1 ? launch_sgemm_f16_out(pos_emb, w.pos_w, p, P, D, D, s)
                             : linear(pos_emb, w.pos_w, nullptr, p, P, D, D, 0, s));
    if (rc) return rc;
    rc = attn_mode == 1
             ? orator_relpos_attention_fast(q, k, v, p, w.pos_bias_u, w.pos_bias_v, ctx, T, H, Dk,
                                            valid, scale, 2, s)
             : orator_relpos_attention(q, k, v, p, w.pos_bias_u, w.pos_bias_v, ctx, T, H, Dk,
                                       valid, scale, s);
    (rc) || (rc = launch_sgemm_residual_ln(ctx, w.out_w, w.out_b, x, T, D, D, 1.0f, w.norm_conv_w,
                                           w.norm_conv_b, ln, kEps, s));
    if (rc) return rc;
    // Conv module
    (rc = pw1_glu(T, valid, s)) ||
        (rc = launch_dwconv_bn_silu(glu, w.dw_w, w.dw_b, w.bn_mean, w.bn_var, w.bn_w, w.bn_b, dw,
                                    T, D, K, kEps, s)) ||
        (rc = launch_sgemm_residual_ln(dw, w.pw2_w, w.pw2_b, x, T, D, D, 1.0f, w.norm_ff2_w,
                                       w.norm_ff2_b, ln, kEps, s));
    if (rc) return rc;
    // FFN2, then norm_out in place
    return ffn(x, T, w.ff2_w1, w.ff2_b1, w.ff2_w2, w.ff2_b2, w.norm_out_w, w.norm_out_b, x, s);
  }
};

}  // namespace
}  // namespace orator_hip

using namespace orator_hip;

extern "C" {

int orator_conformer_create(int d_model, int n_heads, int d_ff, int conv_kernel,
                            const OratorConformerWeights* weights, void** handle) {
  if (!handle) return fail(ORATOR_ERR_INVALID, "conformer_create: null handle");
  *handle = nullptr;
  if (!weights) return fail(ORATOR_ERR_INVALID, "conformer_create: null weights");
  if (d_model <= 0 || n_heads <= 0 || d_ff <= 0 || conv_kernel <= 0 || d_model % n_heads)
    return fail(ORATOR_ERR_INVALID, "conformer_create: bad sizes");
  const float* const* wp = reinterpret_cast<const float* const*>(weights);
  for (size_t i = 0; i < sizeof(OratorConformerWeights) / sizeof(float*); ++i)
    if (!wp[i]) return fail(ORATOR_ERR_INVALID, "conformer_create: null weight");
  Conformer* c = new (std::nothrow) Conformer();
  if (!c) return fail(ORATOR_ERR_CAPACITY, "conformer_create: out of host memory");
  c->D = d_model;
  c->H = n_heads;
  c->Dff = d_ff;
  c->K = conv_kernel;
  c->w = *weights;
  *handle = c;
  return ORATOR_OK;
}

int orator_conformer_destroy(void* handle) {
  delete static_cast<Conformer*>(handle);
  return ORATOR_OK;
}

int orator_conformer_forward(void* handle, float* x, int T, int valid_len, const float* pos_emb,
                             int attn_mode, void* stream) {
  Conformer* c = static_cast<Conformer*>(handle);
  if (!c || !x || !pos_emb) return fail(ORATOR_ERR_INVALID, "conformer_forward: null pointer");
  if (T <= 0) return ORATOR_OK;
  if (attn_mode != 0 && attn_mode != 1)
    return fail(ORATOR_ERR_INVALID, "conformer_forward: attn_mode 0 (fp32) or 1 (fused fp16)");
  if (attn_mode == 1 && c->D / c->H != 64)
    return fail(ORATOR_ERR_UNSUPPORTED, "conformer_forward: the fused attention needs Dk = 64");
  return c->forward(x, T, valid_len, pos_emb, attn_mode, static_cast<hipStream_t>(stream));
}

}  // extern "C"
