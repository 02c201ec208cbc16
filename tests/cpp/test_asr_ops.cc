// The reference's operator tests, run through the C++ drop-in header (orator_attn.hpp).
//
// Same structure and gates as test/unit/model/test_asr_ops.cc (fixture files, max-abs
// tolerances RMSNorm 1e-4, RoPE 1e-4, SwiGLU 1e-5, GQA 5e-4, then a GqaAttention timing at
// T = 256) and test/unit/model/test_gemm_batched.cu (shapes (13,64,13,8), (14,64,14,8),
// index%17/17 and index%13/13 inputs, f64 brute force, 1e-4).  Usage:
//   test_asr_ops <fixture dir with rmsnorm_x.f32 ... gqa_out.f32>
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <fstream>
#include <string>
#include <vector>

#include "orator_attn.hpp"

namespace ops = orator::model::asr_ops;

namespace {

template <typename T>
std::vector<T> ReadRaw(const std::string& path) {
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f) throw std::runtime_error("missing fixture " + path);
  const std::streamsize n = f.tellg();
  f.seekg(0);
  std::vector<T> v(static_cast<size_t>(n) / sizeof(T));
  f.read(reinterpret_cast<char*>(v.data()), n);
  return v;
}

// RAII device buffer (the reference tests use UnifiedBuffer; plain device memory here).
template <typename T>
struct Dev {
  T* p = nullptr;
  size_t n = 0;
  explicit Dev(size_t count) : n(count) {
    if (hipMalloc(reinterpret_cast<void**>(&p), std::max<size_t>(1, n) * sizeof(T)) != hipSuccess)
      throw std::runtime_error("hipMalloc failed");
  }
  explicit Dev(const std::vector<T>& h) : Dev(h.size()) {
    if (hipMemcpy(p, h.data(), n * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
      throw std::runtime_error("H2D failed");
  }
  std::vector<T> Host() const {
    std::vector<T> h(n);
    if (hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(h.data(), p, n * sizeof(T), hipMemcpyDeviceToHost) != hipSuccess)
      throw std::runtime_error("D2H failed");
    return h;
  }
  ~Dev() { (void)hipFree(p); }
  Dev(const Dev&) = delete;
  Dev& operator=(const Dev&) = delete;
};

double MaxAbsErr(const std::vector<float>& ref, const std::vector<float>& got) {
  double e = 0.0;
  for (size_t i = 0; i < ref.size(); ++i)
    e = std::max(e, std::abs(static_cast<double>(ref[i]) - got[i]));
  return e;
}

int g_failures = 0;
void Gate(const char* what, double err, double tol) {
  std::printf("  %-10s max abs err = %.3e (gate %.0e) %s\n", what, err, tol,
              err < tol ? "ok" : "FAIL");
  if (!(err < tol)) ++g_failures;
}

bool BatchedShape(int rows, int inner, int columns, int batch) {
  const size_t ni = static_cast<size_t>(batch) * rows * inner;
  const size_t nw = static_cast<size_t>(batch) * columns * inner;
  std::vector<float> a(ni), w(nw);
  for (size_t i = 0; i < ni; ++i) a[i] = static_cast<float>(i % 17) / 17.0f;
  for (size_t i = 0; i < nw; ++i) w[i] = static_cast<float>(i % 13) / 13.0f;
  Dev<float> da(a), dw(w), dout(static_cast<size_t>(batch) * rows * columns);
  orator::gemm::LaunchSgemmBatched(da.p, dw.p, dout.p, rows, inner, columns, 0, batch,
                                   static_cast<long>(rows) * inner,
                                   static_cast<long>(columns) * inner,
                                   static_cast<long>(rows) * columns);
  const std::vector<float> out = dout.Host();
  double max_abs = 0.0;
  for (int b = 0; b < batch; ++b)
    for (int r = 0; r < rows; ++r)
      for (int c = 0; c < columns; ++c) {
        double e = 0.0;
        for (int k = 0; k < inner; ++k)
          e += static_cast<double>(a[(static_cast<size_t>(b) * rows + r) * inner + k]) *
               w[(static_cast<size_t>(b) * columns + c) * inner + k];
        max_abs = std::max(max_abs,
                           std::fabs(out[(static_cast<size_t>(b) * rows + r) * columns + c] - e));
      }
  std::printf("  batched SGEMM rows=%d inner=%d columns=%d batch=%d max_abs=%.6g\n", rows, inner,
              columns, batch, max_abs);
  return max_abs < 1e-4;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    std::printf("usage: %s <fixture dir>\n", argv[0]);
    return 2;
  }
  const std::string d = std::string(argv[1]) + "/";
  try {
    std::printf("Testing ASR core operators (C++ drop-in over the gfx950 library)...\n");
    {  // RMSNorm (test_asr_ops.cc:73-95)
      const int rows = 8, dim = 2048;
      auto hx = ReadRaw<float>(d + "rmsnorm_x.f32");
      auto hw = ReadRaw<float>(d + "rmsnorm_w.f32");
      auto hr = ReadRaw<float>(d + "rmsnorm_out.f32");
      Dev<float> x(hx), w(hw), y(hr.size());
      ops::RmsNorm(x.p, w.p, y.p, rows, dim, 1e-6f);
      Gate("RMSNorm", MaxAbsErr(hr, y.Host()), 1e-4);
    }
    {  // RoPE interleaved (:97-120)
      const int T = 12, H = 16, Dh = 128;
      auto hx = ReadRaw<float>(d + "rope_x.f32");
      auto hp = ReadRaw<int>(d + "rope_pos.i32");
      auto hr = ReadRaw<float>(d + "rope_out.f32");
      Dev<float> x(hx);
      Dev<int> pos(hp);
      ops::RopeInterleaved(x.p, pos.p, T, H, Dh, 1000000.0f);
      Gate("RoPE", MaxAbsErr(hr, x.Host()), 1e-4);
    }
    {  // SwiGLU (:122-143)
      auto hg = ReadRaw<float>(d + "swiglu_gate.f32");
      auto hu = ReadRaw<float>(d + "swiglu_up.f32");
      auto hr = ReadRaw<float>(d + "swiglu_out.f32");
      Dev<float> g(hg), u(hu), o(hr.size());
      ops::SwiGLU(g.p, u.p, o.p, static_cast<int>(hg.size()));
      Gate("SwiGLU", MaxAbsErr(hr, o.Host()), 1e-5);
    }
    {  // GQA attention, causal (:145-169)
      const int T = 24, Hq = 16, Hkv = 8, Dh = 128;
      auto hq = ReadRaw<float>(d + "gqa_q.f32");
      auto hk = ReadRaw<float>(d + "gqa_k.f32");
      auto hv = ReadRaw<float>(d + "gqa_v.f32");
      auto hr = ReadRaw<float>(d + "gqa_out.f32");
      Dev<float> q(hq), k(hk), v(hv), out(hr.size());
      ops::GqaAttention(q.p, k.p, v.p, out.p, T, Hq, Hkv, Dh, 1.0f / std::sqrt(128.0f), true);
      Gate("GQA attn", MaxAbsErr(hr, out.Host()), 5e-4);
    }
    {  // error behaviour: an unsupported shape throws, as a failed launch does in the reference
      bool threw = false;
      try {
        ops::GqaAttention(nullptr, nullptr, nullptr, nullptr, 4, 16, 8, 96, 0.1f, true);
      } catch (const orator::gpu::GpuMemoryException&) {
        threw = true;
      }
      std::printf("  errors     unsupported shape throws GpuMemoryException: %s\n",
                  threw ? "ok" : "FAIL");
      if (!threw) ++g_failures;
    }
    {  // ConformerLayer::BuildPosEmb is a static of the class (conformer_layer.h:45-46):
       // pe[m][2k] = sin((T-1-m) * 10000^(-2k/d)), pe[m][2k+1] = cos(...)
      const int T = 3, d = 8;
      const std::vector<float> pe = orator::model::conformer_attn::ConformerLayer::BuildPosEmb(T, d);
      double e = pe.size() == static_cast<size_t>((2 * T - 1) * d) ? 0.0 : 1.0;
      for (int m = 0; m < 2 * T - 1 && e == 0.0; ++m)
        for (int k = 0; k < d / 2; ++k) {
          const double a = (T - 1 - m) * std::exp(-std::log(10000.0) * 2 * k / d);
          e = std::max(e, std::fabs(pe[m * d + 2 * k] - std::sin(a)));
          e = std::max(e, std::fabs(pe[m * d + 2 * k + 1] - std::cos(a)));
        }
      std::printf("  pos_emb    static BuildPosEmb(3, 8) max abs err = %.3e %s\n", e,
                  e < 1e-6 ? "ok" : "FAIL");
      if (!(e < 1e-6)) ++g_failures;
    }
    {  // throughput print, representative decoder self-attention (:177-202)
      const int T = 256, Hq = 16, Hkv = 8, Dh = 128;
      std::vector<float> hq(static_cast<size_t>(T) * Hq * Dh, 0.1f), hk(static_cast<size_t>(T) * Hkv * Dh, 0.1f);
      Dev<float> q(hq), k(hk), v(hk), out(hq.size());
      const float scale = 1.0f / std::sqrt(static_cast<float>(Dh));
      ops::GqaAttention(q.p, k.p, v.p, out.p, T, Hq, Hkv, Dh, scale, true);
      (void)hipDeviceSynchronize();
      const int iters = 50;
      const auto t0 = std::chrono::high_resolution_clock::now();
      for (int it = 0; it < iters; ++it) ops::GqaAttention(q.p, k.p, v.p, out.p, T, Hq, Hkv, Dh, scale, true);
      (void)hipDeviceSynchronize();
      const auto t1 = std::chrono::high_resolution_clock::now();
      std::printf("  GQA attn   T=%d Hq=%d Dh=%d: %.3f ms/pass (causal self-attn)\n", T, Hq, Dh,
                  std::chrono::duration<double, std::milli>(t1 - t0).count() / iters);
    }
    if (!BatchedShape(13, 64, 13, 8) || !BatchedShape(14, 64, 14, 8)) ++g_failures;
  } catch (const std::exception& e) {
    std::printf("FAIL: %s\n", e.what());
    return 1;
  }
  std::printf(g_failures ? "ASR core operators test FAILED\n" : "ASR core operators test PASSED\n");
  return g_failures ? 1 : 0;
}
