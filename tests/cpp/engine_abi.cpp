// engine_abi.cpp -- the library called from C++ the way the reference engine calls libr4d: through the C ABI of
// include/r4d_mi355x.h (device pointers and streams as int64_t), with an illegal launch caught as the
// std::runtime_error the reference's contract promises (third_party/libr4d/r4d.h:30-31), and results checked
// against the CPU oracle (oracle/r4o.h, test infrastructure). The checks follow the reference's
// tests/kernels/test_trellis_gemm.cpp: bit-exact dequant, the transform, the GEMV's sums and epilogue, the split's
// tickets after a poisoned buffer, and the M = 256 / M = 64 row identity.
//
//   engine_abi cpu   checks that need no GPU (the _check rules, the thrown errors, the sizes)
//   engine_abi gpu   all of them, on device 0
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "r4d_mi355x.h"
#include "r4o.h"

namespace {

int g_fail = 0, g_pass = 0;
void expect(bool ok, const std::string& what) {
  if (ok) {
    ++g_pass;
  } else {
    ++g_fail;
    std::fprintf(stderr, "FAIL: %s\n", what.c_str());
  }
}

// A fake device address for calls that must be refused before any launch.
const int64_t kFake = 0x1000;

template <class F>
std::string thrown(F&& f) {
  try {
    f();
  } catch (const std::runtime_error& e) {
    return e.what();
  }
  return "";
}

void cpu_checks() {
  // r4d.h:364-375: M above 64 is illegal; the _check names it and the entry throws std::runtime_error
  const char* m = r4d_gemm_trellis_nt_m64_check(65, 512, 256, 256, 4, 1, 1, 1, 0);
  expect(m != nullptr, "m64_check refuses M = 65");
  const std::string e = thrown([] {
    r4d_gemm_trellis_nt_m64(kFake, 0, 256, kFake, kFake, kFake, 0, 0, 65, 512, 256, 4, 0, 0, 0, 0, 1, 0, 0, 1.f, 0);
  });
  expect(e.rfind("r4d gemm_trellis_nt_m64", 0) == 0, "m64 throws std::runtime_error on M = 65: '" + e + "'");
  // a split launch without ws
  const std::string e2 = thrown([] {
    r4d_gemm_trellis_nt_m64(kFake, 0, 256, kFake, kFake, kFake, 0, 0, 1, 512, 256, 4, 0, 0, 0, 0, 2, 0, 0, 1.f, 0);
  });
  expect(!e2.empty(), "m64 throws on SKG 2 without ws");
  // the M = 256 GEMM computes the one-wave-per-pair order only: SK 4 is refused
  expect(r4d_gemm_trellis_nt_m256_check(256, 512, 256, 256, 4, 4, 0, 1, 0, 0) != nullptr, "m256_check refuses SK 4");
  const std::string e3 = thrown([] {
    r4d_gemm_trellis_nt_m256(kFake, 0, 256, kFake, kFake, kFake, kFake, 0, 256, 512, 256, 4, 4, 0, 1, 0, 1.f, 0, 0);
  });
  expect(!e3.empty(), "m256 throws on SK 4");
  expect(r4d_gemm_trellis_nt_m256_check(256, 512, 256, 256, 4, 1, 0, 1, 0, 0) == nullptr, "m256_check accepts SK 1");
  expect(r4d_gemm_trellis_nt_m64_tickets_bytes(5120) == 40 * 128, "tickets_bytes: one 128-byte line per group");
  expect(r4d_gemm_trellis_nt_m64_ws_bytes(8, 5120, 4) == (size_t)4 * 8 * 5120 * 4, "ws_bytes = SKG M N fp32");
  expect(r4d_gemm_trellis_nt_m64_has_rate(4) && r4d_gemm_trellis_nt_m64_has_rate(5) &&
             !r4d_gemm_trellis_nt_m64_has_rate(6),
         "has_rate: KB 3-5");
}

// ---- GPU checks -----------------------------------------------------------------------------------------
#define HIPCHECK(x)                                                                   \
  do {                                                                                \
    hipError_t err_ = (x);                                                            \
    if (err_ != hipSuccess) {                                                         \
      std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(err_), __FILE__, __LINE__); \
      std::exit(2);                                                                   \
    }                                                                                 \
  } while (0)

struct Dev {
  void* p = nullptr;
  size_t n = 0;
  explicit Dev(size_t bytes) : n(bytes) { HIPCHECK(hipMalloc(&p, bytes ? bytes : 1)); }
  ~Dev() { (void)hipFree(p); }
  int64_t a() const { return (int64_t)(uintptr_t)p; }
  template <class T>
  void put(const std::vector<T>& v) { HIPCHECK(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice)); }
  template <class T>
  std::vector<T> get(size_t count) const {
    std::vector<T> v(count);
    HIPCHECK(hipMemcpy(v.data(), p, count * sizeof(T), hipMemcpyDeviceToHost));
    return v;
  }
};

uint64_t g_rng = 0x9E3779B97F4A7C15ull;
uint32_t rnd() {
  g_rng ^= g_rng << 13;
  g_rng ^= g_rng >> 7;
  g_rng ^= g_rng << 17;
  return (uint32_t)(g_rng >> 16);
}
float gauss() {   // Irwin-Hall approximation of N(0, 1)
  float s = 0.f;
  for (int i = 0; i < 12; ++i) s += (float)(rnd() & 0xFFFFFF) / 16777216.f;
  return s - 6.f;
}

void gpu_checks() {
  const int K = 512, N = 256, KB = 4;
  hipStream_t st;
  HIPCHECK(hipStreamCreate(&st));
  const int64_t s = (int64_t)(uintptr_t)st;

  // words: uniform random u32 in the pair grid (every word is a valid ring)
  std::vector<uint32_t> words((size_t)K * N * KB / 32);
  for (auto& w : words) w = rnd() ^ (rnd() << 16);
  Dev dw(words.size() * 4);
  dw.put(words);

  // 1. reconstruct: bit-exact dequant against the oracle's decode
  std::vector<uint16_t> qref((size_t)K * N);
  r4o_decode_pair_grid(words.data(), K, N, KB, qref.data(), 1);
  Dev dq((size_t)K * N * 2);
  r4d_trellis_reconstruct_f16(dw.a(), dq.a(), K, N, KB, s);
  HIPCHECK(hipStreamSynchronize(st));
  expect(dq.get<uint16_t>((size_t)K * N) == qref, "reconstruct == oracle decode, bit for bit");

  // 2. the input transform (bf16 x, one output)
  const int M = 4;
  std::vector<uint16_t> x((size_t)M * K);
  for (auto& v : x) v = r4o_f32_to_bf16(gauss());
  std::vector<float> suh(K), svh(N);
  for (auto& v : suh) v = (rnd() & 1) ? 1.f : -1.f;
  for (auto& v : svh) v = 0.01f * std::exp(0.3f * gauss());
  Dev dx(x.size() * 2), dsuh(K * 4), dsvh(N * 4), da((size_t)M * K * 2);
  dx.put(x);
  dsuh.put(suh);
  dsvh.put(svh);
  const int64_t suh_p[1] = {dsuh.a()}, out_p[1] = {da.a()};
  r4dx_trellis_input_bf16(dx.a(), M, K, 1, suh_p, out_p, 0, s);
  HIPCHECK(hipStreamSynchronize(st));
  std::vector<uint16_t> aref((size_t)M * K);
  r4o_transform_input(x.data(), 1, M, K, suh.data(), 0, aref.data());
  const std::vector<uint16_t> a = da.get<uint16_t>((size_t)M * K);
  expect(a == aref, "transform == oracle, bit for bit");

  // 3. the GEMV, split in two K slices (ws + tickets): fp32 sums against fp64, the bf16 epilogue bit for bit
  const int SKG = 2;
  Dev dws(r4d_gemm_trellis_nt_m64_ws_bytes(M, N, SKG)), dtk(r4d_gemm_trellis_nt_m64_tickets_bytes(N));
  HIPCHECK(hipMemset(dtk.p, 0, dtk.n));
  Dev draw((size_t)M * N * 4), dc((size_t)M * N * 2);
  const float out_scale = (float)(1.0 / std::sqrt(128.0));
  r4d_gemm_trellis_nt_m64_raw(da.a(), 0, N, dw.a(), draw.a(), dws.a(), dtk.a(), M, K, N, KB, 0, 0, 0, 0, SKG, 0, 0, 0,
                              s);
  r4d_gemm_trellis_nt_m64(da.a(), 0, N, dw.a(), dsvh.a(), dc.a(), dws.a(), dtk.a(), M, K, N, KB, 0, 0, 0, 0, SKG, 0,
                          0, out_scale, s);
  HIPCHECK(hipStreamSynchronize(st));
  const std::vector<float> raw = draw.get<float>((size_t)M * N);
  std::vector<double> sref((size_t)M * N);
  r4o_raw_sums_f64(aref.data(), nullptr, N, M, K, N, qref.data(), sref.data(), 1);
  double ms = 0;
  for (double v : sref) ms += v * v;
  const double rms = std::sqrt(ms / sref.size());
  double worst = 0;
  for (size_t i = 0; i < sref.size(); ++i)
    worst = std::fmax(worst, std::fabs(raw[i] - sref[i]) / (1e-3 * std::fabs(sref[i]) + 1e-4 * rms));
  expect(worst <= 1.0, "GEMV fp32 sums within 1e-3 |ref| + 1e-4 rms of fp64 (worst " + std::to_string(worst) + ")");
  std::vector<uint16_t> cref((size_t)M * N);
  r4o_epilogue_from_raw(raw.data(), M, N, svh.data(), out_scale, cref.data());
  expect(dc.get<uint16_t>((size_t)M * N) == cref, "GEMV bf16 == the oracle's epilogue of its sums, bit for bit");

  // 4. a poisoned ticket buffer, reset by zero_tickets: the next split launch is exact again
  std::vector<uint32_t> junk(dtk.n / 4, 7u);
  dtk.put(junk);
  r4d_gemm_trellis_nt_m64_zero_tickets(dtk.a(), dtk.n, s);
  r4d_gemm_trellis_nt_m64(da.a(), 0, N, dw.a(), dsvh.a(), dc.a(), dws.a(), dtk.a(), M, K, N, KB, 0, 0, 0, 0, SKG, 0,
                          0, out_scale, s);
  HIPCHECK(hipStreamSynchronize(st));
  expect(dc.get<uint16_t>((size_t)M * N) == cref, "after zero_tickets the split launch is exact again");
  expect(dtk.get<uint32_t>(dtk.n / 4) == std::vector<uint32_t>(dtk.n / 4, 0u), "tickets back at zero");

  // 5. M = 256 against M = 64 chunks at SK = 1 and the same SKG: every element bit for bit (r4d.h:395-412)
  const int MB = 256;
  std::vector<uint16_t> a256((size_t)MB * K);
  for (auto& v : a256) v = r4o_f32_to_f16(gauss());
  Dev da256(a256.size() * 2), dc256((size_t)MB * N * 2), dc64((size_t)64 * N * 2);
  da256.put(a256);
  Dev dws256(r4d_gemm_trellis_nt_m256_ws_bytes(MB, N, SKG)), dtk256(r4d_gemm_trellis_nt_m64_tickets_bytes(N));
  HIPCHECK(hipMemset(dtk256.p, 0, dtk256.n));
  r4d_gemm_trellis_nt_m256(da256.a(), 0, N, dw.a(), dsvh.a(), dc256.a(), dws256.a(), dtk256.a(), MB, K, N, KB, 1, 0,
                           SKG, 0, out_scale, s, 0);
  HIPCHECK(hipStreamSynchronize(st));
  const std::vector<uint16_t> c256 = dc256.get<uint16_t>((size_t)MB * N);
  bool same = true;
  Dev dws64(r4d_gemm_trellis_nt_m64_ws_bytes(64, N, SKG));
  for (int r0 = 0; r0 < MB; r0 += 64) {
    r4d_gemm_trellis_nt_m64(da256.a() + (int64_t)r0 * K * 2, 0, N, dw.a(), dsvh.a(), dc64.a(), dws64.a(), dtk.a(), 64,
                            K, N, KB, 0, 1, 0, 0, SKG, 0, 0, out_scale, s);
    HIPCHECK(hipStreamSynchronize(st));
    const std::vector<uint16_t> c64 = dc64.get<uint16_t>((size_t)64 * N);
    same = same && std::memcmp(c64.data(), c256.data() + (size_t)r0 * N, c64.size() * 2) == 0;
  }
  expect(same, "M = 256 rows == M = 64 rows at SK 1, SKG 2, bit for bit");
  HIPCHECK(hipStreamDestroy(st));
}

}  // namespace

int main(int argc, char** argv) {
  const bool gpu = argc > 1 && std::strcmp(argv[1], "gpu") == 0;
  std::printf("[engine_abi] %s checks\n", gpu ? "cpu + gpu" : "cpu");
  std::fflush(stdout);
  cpu_checks();
  if (gpu) gpu_checks();
  std::printf("engine_abi: %d passed, %d failed\n", g_pass, g_fail);
  return g_fail ? 1 : 0;
}
