// Plain GEMMs on hipBLASLt: the bf16 prompt projections (M > 1) and the fp32 nn.Linear
// products of the Conformer.
//
// LaunchBf16Gemm (include/model/gemm.cuh:384-501) computes out[M][N] = act(in[M][K] W[N][K]^T
// + bias) in fp32 from bf16 operands, LaunchSgemm[Batched] (:47-268) the same from fp32
// operands.  Where the product is a plain GEMM it runs on the library's tuned MFMA kernels:
// the row-major problem is the column-major D[N x M] = op_T(W: K x N, ld K) * op_N(in: K x M,
// ld K), fp32 compute (exact fp32 products for fp32 operands, not a reduced-precision mode)
// and fp32 output; strided batches map onto the layouts' batch strides.  beta = 1 with C = D
// folds a residual add into the product (one fp32 rounding, as the add).  Bias and
// activation, when asked for, follow in one elementwise pass of the caller, so the
// activations are this library's own (erf GELU / ReLU, SiLU / ReLU / sigmoid), not the GEMM
// library's epilogue.
//
// Plans (descriptors + the heuristic's first algorithm) are cached per device and shape.  Only
// algorithms that need no workspace are taken, so concurrent streams share nothing; a shape
// with none returns ORATOR_ERR_UNSUPPORTED and the caller runs its own MFMA kernel.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <cstdlib>
#include <map>
#include <mutex>
#include <tuple>

#include "internal.hpp"

namespace orator_hip {
namespace {

struct Plan {
  bool ok = false;
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};

struct DeviceLt {
  hipblasLtHandle_t handle = nullptr;
  bool failed = false;
  // (M, K, N, fp32 operands, batch, batch strides of in, W, out)
  std::map<std::tuple<int, int, int, bool, int, long, long, long>, Plan> plans;
};

std::mutex g_lt_mu;
std::map<int, DeviceLt> g_lt;

bool lt_ok(hipblasStatus_t st) { return st == HIPBLAS_STATUS_SUCCESS; }

bool set_batch(hipblasLtMatrixLayout_t l, int batch, long stride) {
  const int32_t n = batch;
  const int64_t st = stride;
  return batch == 1 ||
         (lt_ok(hipblasLtMatrixLayoutSetAttribute(l, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &n,
                                                  sizeof(n))) &&
          lt_ok(hipblasLtMatrixLayoutSetAttribute(l, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET,
                                                  &st, sizeof(st))));
}

// Builds (once) the plan of a (batched) M x K x N product; false when the library has none.
bool make_plan(DeviceLt& d, int M, int K, int N, bool f32, int batch, long s_in, long s_w,
               long s_out, Plan& p) {
  const int32_t op_t = HIPBLAS_OP_T, op_n = HIPBLAS_OP_N;
  const hipDataType ab = f32 ? HIP_R_32F : HIP_R_16BF;
  if (!lt_ok(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F)) ||
      !lt_ok(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op_t,
                                             sizeof(op_t))) ||
      !lt_ok(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op_n,
                                             sizeof(op_n))) ||
      !lt_ok(hipblasLtMatrixLayoutCreate(&p.la, ab, K, N, K)) ||
      !lt_ok(hipblasLtMatrixLayoutCreate(&p.lb, ab, K, M, K)) ||
      !lt_ok(hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_32F, N, M, N)) ||
      !set_batch(p.la, batch, s_w) || !set_batch(p.lb, batch, s_in) ||
      !set_batch(p.lc, batch, s_out))
    return false;
  hipblasLtMatmulPreference_t pref = nullptr;
  if (!lt_ok(hipblasLtMatmulPreferenceCreate(&pref))) return false;
  const uint64_t no_ws = 0;
  hipblasLtMatmulHeuristicResult_t res[4];
  int n = 0;
  const bool got =
      lt_ok(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                  &no_ws, sizeof(no_ws))) &&
      lt_ok(hipblasLtMatmulAlgoGetHeuristic(d.handle, p.desc, p.la, p.lb, p.lc, p.lc, pref, 4, res,
                                            &n));
  (void)hipblasLtMatmulPreferenceDestroy(pref);
  for (int i = 0; got && i < n; ++i)
    if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize == 0) {
      p.algo = res[i].algo;
      p.ok = true;
      return true;
    }
  return false;
}

}  // namespace

// Tuning override (read once): ORATOR_GEMM_LIB=0 keeps every M > 1 product on this library's
// own MFMA GEMM.
bool bf16_gemm_lib_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("ORATOR_GEMM_LIB");
    return !(e && std::atoi(e) == 0);
  }();
  return on;
}

namespace {

int gemm_lib(const void* in, const void* W, float* out, int M, int K, int N, bool f32, int batch,
             long s_in, long s_w, long s_out, float beta, hipStream_t stream) {
  int dev = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
  std::lock_guard<std::mutex> lock(g_lt_mu);
  DeviceLt& d = g_lt[dev];
  if (d.failed) return ORATOR_ERR_UNSUPPORTED;
  if (!d.handle && !lt_ok(hipblasLtCreate(&d.handle))) {
    d.failed = true;
    d.handle = nullptr;
    return ORATOR_ERR_UNSUPPORTED;
  }
  auto key = std::make_tuple(M, K, N, f32, batch, s_in, s_w, s_out);
  auto it = d.plans.find(key);
  if (it == d.plans.end()) {
    Plan p;
    make_plan(d, M, K, N, f32, batch, s_in, s_w, s_out, p);
    it = d.plans.emplace(key, p).first;
  }
  Plan& p = it->second;
  if (!p.ok) return ORATOR_ERR_UNSUPPORTED;
  const float alpha = 1.0f;  // D = alpha op(A) op(B) + beta C, C = D = out
  const hipblasStatus_t st = hipblasLtMatmul(d.handle, p.desc, &alpha, W, p.la, in, p.lb, &beta,
                                             out, p.lc, out, p.lc, &p.algo, nullptr, 0, stream);
  if (!lt_ok(st)) return fail(ORATOR_ERR_HIP, "gemm: hipblasLtMatmul failed");
  return ORATOR_OK;
}

}  // namespace

int launch_bf16_gemm_lib(const uint16_t* in, const uint16_t* W, float* out, int M, int K, int N,
                         float beta, hipStream_t stream) {
  return gemm_lib(in, W, out, M, K, N, false, 1, 0, 0, 0, beta, stream);
}

int launch_f32_gemm_lib(const float* in, const float* W, float* out, int M, int K, int N,
                        int batch, long stride_in, long stride_w, long stride_out,
                        hipStream_t stream) {
  return gemm_lib(in, W, out, M, K, N, true, batch, stride_in, stride_w, stride_out, 0.0f,
                  stream);
}

}  // namespace orator_hip
