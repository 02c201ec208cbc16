// Small kernels of the decoder's step body (src/model/asr_text_decoder.cu:30-58): embedding
// gather, residual add, and the device-side token record / position increment that let one
// decode step be replayed from a captured graph at any position.
#include "common.hpp"
#include "internal.hpp"

namespace orator_hip {
namespace {

// out[i] = bf16 table[token][i] widened (EmbedGatherKernel, asr_text_decoder.cu:38-45).
// Eight values per thread (16-byte table loads).
__global__ __launch_bounds__(256) void embed_gather_kernel(const uint16_t* __restrict__ table,
                                                           const int* __restrict__ token,
                                                           float* __restrict__ out, int hidden) {
  const int i = 8 * (blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= hidden) return;
  const uint4 w = *reinterpret_cast<const uint4*>(table + static_cast<long>(*token) * hidden + i);
  *reinterpret_cast<float4*>(out + i) = make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
  *reinterpret_cast<float4*>(out + i + 4) =
      make_float4(bf16_lo(w.z), bf16_hi(w.z), bf16_lo(w.w), bf16_hi(w.w));
}

// a += b (AddResidualKernel, asr_text_decoder.cu:30-34), four values per thread.
__global__ __launch_bounds__(256) void add_residual_kernel(float* __restrict__ a,
                                                           const float* __restrict__ b, long n) {
  const long i = 4 * (static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x);
  if (i + 3 < n) {
    float4 x = *reinterpret_cast<float4*>(a + i);
    const float4 y = *reinterpret_cast<const float4*>(b + i);
    x.x += y.x;
    x.y += y.y;
    x.z += y.z;
    x.w += y.w;
    *reinterpret_cast<float4*>(a + i) = x;
  } else {
    for (long j = i; j < n; ++j) a[j] += b[j];
  }
}

// out[*count] = *token; ++*count (RecordTokenKernel, asr_text_decoder.cu:50-55).
__global__ void record_token_kernel(int* out, int* count, const int* token, int capacity) {
  const int c = *count;
  if (c < capacity) out[c] = *token;
  *count = c + 1;
}

// ++*pos (IncPosKernel, asr_text_decoder.cu:58).
__global__ void inc_pos_kernel(int* pos) { *pos = *pos + 1; }

}  // namespace
}  // namespace orator_hip

using namespace orator_hip;

extern "C" {

int orator_embed_gather(const uint16_t* table, const int* d_token, float* out, int hidden,
                        void* stream) {
  if (hidden <= 0) return ORATOR_OK;
  if (!table || !d_token || !out) return fail(ORATOR_ERR_INVALID, "embed_gather: null pointer");
  if (hidden % 8 || (reinterpret_cast<uintptr_t>(table) & 15u) ||
      (reinterpret_cast<uintptr_t>(out) & 15u))
    return fail(ORATOR_ERR_INVALID, "embed_gather: hidden % 8 == 0 and 16-byte alignment needed");
  const int threads = hidden / 8;
  hipLaunchKernelGGL(embed_gather_kernel, dim3((threads + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), table, d_token, out, hidden);
  return check_launch("embed_gather");
}

int orator_add_residual(float* a, const float* b, long n, void* stream) {
  if (n <= 0) return ORATOR_OK;
  if (!a || !b) return fail(ORATOR_ERR_INVALID, "add_residual: null pointer");
  if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15u)
    return fail(ORATOR_ERR_INVALID, "add_residual: a and b must be 16-byte aligned");
  const long threads = (n + 3) / 4;
  hipLaunchKernelGGL(add_residual_kernel, dim3(static_cast<unsigned>((threads + 255) / 256)),
                     dim3(256), 0, static_cast<hipStream_t>(stream), a, b, n);
  return check_launch("add_residual");
}

int orator_record_token(int* out, int* d_count, const int* d_token, int capacity, void* stream) {
  if (!out || !d_count || !d_token) return fail(ORATOR_ERR_INVALID, "record_token: null pointer");
  hipLaunchKernelGGL(record_token_kernel, dim3(1), dim3(1), 0, static_cast<hipStream_t>(stream),
                     out, d_count, d_token, capacity);
  return check_launch("record_token");
}

int orator_inc_pos(int* d_pos, void* stream) {
  if (!d_pos) return fail(ORATOR_ERR_INVALID, "inc_pos: null pointer");
  hipLaunchKernelGGL(inc_pos_kernel, dim3(1), dim3(1), 0, static_cast<hipStream_t>(stream), d_pos);
  return check_launch("inc_pos");
}

}  // extern "C"
