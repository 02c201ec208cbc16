// The Conformer layer's non-attention passes (src/model/conformer_layer.cu:28-76,207-246):
// LayerNorm, GLU (fused with the padding-row mask that follows it), the depthwise time
// convolution fused with the BatchNorm (eval) + SiLU after it.  (The scaled residual add is the
// epilogue of the projection before it: launch_sgemm_residual.)
// Each keeps the reference's per-element arithmetic; the fusions only drop the HBM round trips
// between passes.  All tensors are [T, C] fp32, C the channel count (d_model).
#include "common.hpp"
#include "internal.hpp"

namespace orator_hip {
namespace {

// LayerNormKernel (conformer_layer.cu:28-66): mean, then the mean square deviation, both over
// the row, inv = rsqrt(var + eps), y = (x - mean) inv g + b.  One wave per row; lane l owns
// elements l, l + 64, ... and sums them in that order, then the wave sum.  PER > 0 (C <= 64 PER)
// holds the row in registers, so all of a lane's loads are in flight together; PER = 0 re-reads
// the row from cache, for any C.  Both give the same bits.  `out` may be `in` (each lane reads
// its own elements before writing them).
template <int PER>
__global__ __launch_bounds__(256) void layer_norm_kernel(const float* in,
                                                         const float* __restrict__ g,
                                                         const float* __restrict__ b, float* out,
                                                         int T, int C, float eps) {
#pragma clang fp contract(off)
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= T) return;
  const float* x = in + static_cast<long>(row) * C;
  float* y = out + static_cast<long>(row) * C;
  if constexpr (PER > 0) {
    float v[PER], gv[PER], bv[PER];  // the row, gamma and beta: one round of loads
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = min(lane + 64 * i, C - 1);
      v[i] = x[c];
      gv[i] = g[c];
      bv[i] = b[c];
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (lane + 64 * i < C) s += v[i];
    const float mean = wave_sum(s) / static_cast<float>(C);
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const float t = v[i] - mean;
      if (lane + 64 * i < C) sq += t * t;
    }
    const float inv = rsqrtf(wave_sum(sq) / static_cast<float>(C) + eps);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = lane + 64 * i;
      if (c < C) y[c] = (v[i] - mean) * inv * gv[i] + bv[i];
    }
  } else {
    float s = 0.0f;
    for (int c = lane; c < C; c += 64) s += x[c];
    const float mean = wave_sum(s) / static_cast<float>(C);
    float sq = 0.0f;
    for (int c = lane; c < C; c += 64) {
      const float t = x[c] - mean;
      sq += t * t;
    }
    const float inv = rsqrtf(wave_sum(sq) / static_cast<float>(C) + eps);
    for (int c = lane; c < C; c += 64) y[c] = (x[c] - mean) * inv * g[c] + b[c];
  }
}

// GluKernel (:207-215) then MaskRowsKernel (:78-83): out[t,c] = a * sigmoid(b) for rows
// t < valid, 0 for padded rows; in is [T, 2C] (a | b).
__global__ __launch_bounds__(256) void glu_mask_kernel(const float* __restrict__ in,
                                                       float* __restrict__ out, int T, int C,
                                                       int valid) {
  const long idx = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<long>(T) * C) return;
  const int c = static_cast<int>(idx % C);
  const int t = static_cast<int>(idx / C);
  if (t >= valid) {
    out[idx] = 0.0f;
    return;
  }
  const float a = in[static_cast<long>(t) * 2 * C + c];
  const float bb = in[static_cast<long>(t) * 2 * C + C + c];
  out[idx] = a * (1.0f / (1.0f + __expf(-bb)));
}

// DepthwiseConvKernel (:218-233) then BatchNormSiluKernel (:236-246): per channel c,
// acc = bias[c] + sum_k in[t + k - pad, c] w[c, k] over in-range taps (pad = (K - 1) / 2),
// y = (acc - mean) rsqrt(var + eps) gamma + beta, out = y / (1 + exp(-y)).
__global__ __launch_bounds__(256) void dwconv_bn_silu_kernel(
    const float* __restrict__ in, const float* __restrict__ w, const float* __restrict__ bias,
    const float* __restrict__ mean, const float* __restrict__ var,
    const float* __restrict__ gamma, const float* __restrict__ beta, float* __restrict__ out,
    int T, int C, int K, float eps) {
#pragma clang fp contract(off)
  const long idx = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<long>(T) * C) return;
  const int c = static_cast<int>(idx % C);
  const int t = static_cast<int>(idx / C);
  const int pad = (K - 1) / 2;
  float acc = bias ? bias[c] : 0.0f;
  const float* wc = w + static_cast<long>(c) * K;
  for (int k = 0; k < K; ++k) {
    const int ti = t + k - pad;
    if (ti >= 0 && ti < T) acc += in[static_cast<long>(ti) * C + c] * wc[k];
  }
  const float y = (acc - mean[c]) * rsqrtf(var[c] + eps) * gamma[c] + beta[c];
  out[idx] = y / (1.0f + __expf(-y));
}

// AddScaledKernel (:70-73): r += scale * x.
unsigned blocks256(long n) { return static_cast<unsigned>((n + 255) / 256); }

}  // namespace

int launch_layer_norm(const float* in, const float* g, const float* b, float* out, int T, int C,
                      float eps, hipStream_t s) {
  if (T <= 0 || C <= 0) return ORATOR_OK;
  const dim3 grid((T + 3) / 4), block(256);
  if (C <= 256)
    hipLaunchKernelGGL(layer_norm_kernel<4>, grid, block, 0, s, in, g, b, out, T, C, eps);
  else if (C <= 512)
    hipLaunchKernelGGL(layer_norm_kernel<8>, grid, block, 0, s, in, g, b, out, T, C, eps);
  else if (C <= 1024)
    hipLaunchKernelGGL(layer_norm_kernel<16>, grid, block, 0, s, in, g, b, out, T, C, eps);
  else
    hipLaunchKernelGGL(layer_norm_kernel<0>, grid, block, 0, s, in, g, b, out, T, C, eps);
  return check_launch("layer_norm_kernel");
}

int launch_glu_mask(const float* in, float* out, int T, int C, int valid, hipStream_t s) {
  if (T <= 0 || C <= 0) return ORATOR_OK;
  hipLaunchKernelGGL(glu_mask_kernel, dim3(blocks256(static_cast<long>(T) * C)), dim3(256), 0, s,
                     in, out, T, C, valid);
  return check_launch("glu_mask_kernel");
}

int launch_dwconv_bn_silu(const float* in, const float* w, const float* bias, const float* mean,
                          const float* var, const float* gamma, const float* beta, float* out,
                          int T, int C, int K, float eps, hipStream_t s) {
  if (T <= 0 || C <= 0) return ORATOR_OK;
  hipLaunchKernelGGL(dwconv_bn_silu_kernel, dim3(blocks256(static_cast<long>(T) * C)), dim3(256),
                     0, s, in, w, bias, mean, var, gamma, beta, out, T, C, K, eps);
  return check_launch("dwconv_bn_silu_kernel");
}

}  // namespace orator_hip
