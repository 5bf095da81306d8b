// engine_abi.cpp -- the library called from C++ the way the reference engine calls libr4d: through the C ABI of
// include/r4d_mi355x.h (device pointers and streams as int64_t), with an illegal launch caught as the
// std::runtime_error the reference's contract promises (third_party/libr4d/r4d.h:30-31), and results checked
// against the CPU oracle (oracle/r4o.h, test infrastructure). The checks follow the reference's
// tests/kernels/test_trellis_gemm.cpp: bit-exact dequant, the transform, the GEMV's sums and epilogue, the split's
// tickets after a poisoned buffer, and the M = 256 / M = 64 row identity; then the w4a16 GEMM (quant_int4.hpp's
// packers), the row argmax (argmax_ref.hpp's order), the int8 row quantizer and the dense int8 GEMM's exact sums.
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
  // the M = 256 GEMM reproduces the M = 64 row of SK 1 / 2 (one wave per pair) and SK 4 / 8 / 16 (4-wave split);
  // any other SK is refused
  expect(r4d_gemm_trellis_nt_m256_check(256, 512, 256, 256, 4, 3, 0, 1, 0, 0) != nullptr, "m256_check refuses SK 3");
  const std::string e3 = thrown([] {
    r4d_gemm_trellis_nt_m256(kFake, 0, 256, kFake, kFake, kFake, kFake, 0, 256, 512, 256, 4, 3, 0, 1, 0, 1.f, 0, 0);
  });
  expect(!e3.empty(), "m256 throws on SK 3");
  expect(r4d_gemm_trellis_nt_m256_check(256, 512, 256, 256, 4, 1, 0, 1, 0, 0) == nullptr, "m256_check accepts SK 1");
  expect(r4d_gemm_trellis_nt_m256_check(256, 512, 256, 256, 4, 4, 0, 1, 0, 0) == nullptr, "m256_check accepts SK 4");
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
  // the same at SK 4 (the 4-wave split order; ws and tickets given to both)
  r4d_gemm_trellis_nt_m256(da256.a(), 0, N, dw.a(), dsvh.a(), dc256.a(), dws256.a(), dtk256.a(), MB, K, N, KB, 4, 0,
                           SKG, 0, out_scale, s, 0);
  HIPCHECK(hipStreamSynchronize(st));
  const std::vector<uint16_t> c256s = dc256.get<uint16_t>((size_t)MB * N);
  same = true;
  for (int r0 = 0; r0 < MB; r0 += 64) {
    r4d_gemm_trellis_nt_m64(da256.a() + (int64_t)r0 * K * 2, 0, N, dw.a(), dsvh.a(), dc64.a(), dws64.a(), dtk.a(), 64,
                            K, N, KB, 0, 4, 0, 0, SKG, 0, 0, out_scale, s);
    HIPCHECK(hipStreamSynchronize(st));
    const std::vector<uint16_t> c64 = dc64.get<uint16_t>((size_t)64 * N);
    same = same && std::memcmp(c64.data(), c256s.data() + (size_t)r0 * N, c64.size() * 2) == 0;
  }
  expect(same, "M = 256 rows == M = 64 rows at SK 4, SKG 2, bit for bit");

  // 6. w4a16 at group 64 (quant_int4.hpp's quantizer and packers), then the argmax of its fp32 logits
  {
    const int WN = 512, WK = 512, G = 64, WM = 2;
    std::vector<float> wf((size_t)WN * WK), sc((size_t)WN * WK / G);
    for (auto& v : wf) v = 0.05f * gauss();
    std::vector<uint8_t> q4((size_t)WN * WK), z((size_t)WN * WK / G);
    r4o_w4_quantize(wf.data(), WN, WK, G, q4.data(), sc.data(), z.data());
    std::vector<uint32_t> wq((size_t)WN * WK / 8), wsz((size_t)WN / 16 * (WK / G) * 16);
    r4o_w4_pack(q4.data(), WN, WK, wq.data());
    r4o_w4_pack_scales(sc.data(), z.data(), WN, WK, G, wsz.data());
    std::vector<uint16_t> a4((size_t)WM * WK);
    for (auto& v : a4) v = r4o_f32_to_f16(gauss());
    Dev dwq(wq.size() * 4), dwsz(wsz.size() * 4), da4(a4.size() * 2), dc4((size_t)WM * WN * 2);
    dwq.put(wq);
    dwsz.put(wsz);
    da4.put(a4);
    expect(r4d_gemm_w4a16_nt_m64_check(G, WM, WK, WN) == nullptr, "w4a16 check accepts g64 M 2");
    r4d_gemm_w4a16_nt_m64_g(G, da4.a(), dwq.a(), dwsz.a(), dc4.a(), WM, WK, WN, 0, 0, 0, 0, 0, s);
    HIPCHECK(hipStreamSynchronize(st));
    const std::vector<uint16_t> c4 = dc4.get<uint16_t>((size_t)WM * WN);
    std::vector<double> y((size_t)WM * WN);
    r4o_w4_gemm_ref(a4.data(), wq.data(), wsz.data(), WM, WN, WK, G, y.data(), 1);
    double yms = 0, wst = 0;
    for (double v : y) yms += v * v;
    const double yrms = std::sqrt(yms / y.size());
    for (size_t i = 0; i < y.size(); ++i)
      wst = std::fmax(wst, std::fabs(r4o_bf16_to_f32(c4[i]) - y[i]) / (std::ldexp(std::fabs(y[i]), -8) + 1e-3 * yrms));
    expect(wst <= 1.0, "w4a16 bf16 within one bf16 rounding of the fp64 reference (worst " + std::to_string(wst) + ")");

    // argmax over fp32 rows (ties to the lowest index, NaN never wins), against the oracle's order
    const int R = 3, V = 100003;
    std::vector<float> lg((size_t)R * V);
    for (auto& v : lg) v = gauss();
    lg[5] = 40.f;
    lg[V + 77] = 40.f;
    lg[V + 99] = 40.f;                                   // a tie: the lower index wins
    lg[2 * (size_t)V + 11] = std::nanf("");
    Dev dl(lg.size() * 4), di(R * 4), dv(R * 4);
    dl.put(lg);
    r4dx_argmax_rows_f32(dl.a(), V, di.a(), dv.a(), 1, R, V, s);
    HIPCHECK(hipStreamSynchronize(st));
    const std::vector<int32_t> idx = di.get<int32_t>(R);
    bool am = true;
    for (int r = 0; r < R; ++r) {
      float bv = 0.f;
      am = am && idx[r] == r4o_argmax_f32(lg.data() + (size_t)r * V, V, &bv);
    }
    expect(am, "argmax rows == the oracle's order (ties, NaN)");
  }

  // 7. int8: the per-row activation quantizer byte for byte, and the dense GEMM's exact int32 sums
  {
    const int IM = 256, IK = 512, IN = 256;
    std::vector<uint16_t> xi((size_t)IM * IK);
    for (auto& v : xi) v = r4o_f32_to_f16(gauss());
    std::vector<float> sa_ref(IM);
    std::vector<int8_t> ap((size_t)IM * IK), a8_ref((size_t)IM * IK);
    r4o_i8_quant_act_row(xi.data(), IM, IK, sa_ref.data(), ap.data());
    r4o_pack_a8(ap.data(), IK, a8_ref.data());
    Dev dxi(xi.size() * 2), da8((size_t)IM * IK), dsa(IM * 4);
    dxi.put(xi);
    r4d_trellis_i8_quant_act_row(dxi.a(), da8.a(), dsa.a(), 1, 0, IK, s);
    HIPCHECK(hipStreamSynchronize(st));
    const std::vector<int8_t> a8 = da8.get<int8_t>((size_t)IM * IK);
    const std::vector<float> sa = dsa.get<float>(IM);
    expect(a8 == a8_ref && std::memcmp(sa.data(), sa_ref.data(), IM * 4) == 0,
           "int8 row quantizer == oracle (A8 bytes and scales)");
    std::vector<int8_t> wp((size_t)IN * IK);
    for (auto& v : wp) v = (int8_t)((int)(rnd() % 255) - 127);
    Dev dwp(wp.size()), dw8(wp.size()), dci((size_t)IM * IN * 4);
    dwp.put(wp);
    r4d_i8_pack_w(dwp.a(), dw8.a(), IN, IK, s);
    r4d_gemm_i8_dense_raw(da8.a(), dw8.a(), dci.a(), 0, 0, IM, IK, IN, 1, s);
    HIPCHECK(hipStreamSynchronize(st));
    std::vector<int32_t> acc((size_t)IM * IN);
    r4o_i8_gemm_i32(ap.data(), wp.data(), IM, IN, IK, acc.data(), 1);
    expect(dci.get<int32_t>((size_t)IM * IN) == acc, "dense int8 int32 sums exact");
  }
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
