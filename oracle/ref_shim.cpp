// ref_shim.cpp -- TEST INFRASTRUCTURE ONLY.  A C-ABI face over the reference's own header-only CPU
// references, compiled from their sources where they lie under the reference checkout (never
// copied).  Built by oracle/Makefile into oracle/_ref/libr4dref.so when the checkout is present;
// tests/test_oracle_vs_ref.py uses it to validate the C restatement in r4o.c.
//   tests/kernels/trellis_ref.hpp                        decode, transform, linear, epilogue
//   tests/kernels/int8_gemm_proto_ref.h                  int8 quantizers and reference GEMM
//   src/convert/include/r4dx_convert/quant_int4.hpp      w4a16 quantizer and packers
//   src/kernels/include/r4dx/kernels/argmax_ref.hpp      argmax order
//   src/model/fake_quant_w.h                             weight fake-quant table and rounding
#include <cstring>
#include <vector>

#include "trellis_ref.hpp"
#include "int8_gemm_proto_ref.h"
#include "r4dx_convert/quant_int4.hpp"
#include "r4dx/kernels/argmax_ref.hpp"
#include "fake_quant_w.h"

extern "C" {

void ref_codebook(uint16_t* out) {
  const auto& cb = trellis_ref::Mul1CodebookF16();
  std::memcpy(out, cb.data(), 65536 * 2);
}
uint32_t ref_trellis_state(const uint32_t* w, int KB, int p) { return trellis_ref::TrellisState(w, KB, p); }
int ref_tc_perm(int p) { return trellis_ref::TensorCorePerm(p); }
void ref_to_pair_grid(const uint32_t* words, int64_t K, int64_t N, int KB, uint32_t* grid) {
  std::vector<uint32_t> w(words, words + (size_t)(K * N * KB / 32));
  auto g = trellis_ref::ToPairGrid(w, K, N, KB);
  std::memcpy(grid, g.data(), g.size() * 4);
}
void ref_decode_pair_grid(const uint32_t* grid, int64_t K, int64_t N, int KB, uint16_t* q) {
  std::vector<uint32_t> g(grid, grid + (size_t)(K * N * KB / 32));
  auto out = trellis_ref::DecodePairGrid(g, K, N, KB);
  std::memcpy(q, out.data(), out.size() * 2);
}
void ref_fwht_lds_f32(float* v) { trellis_ref::FwhtLdsF32(v); }
void ref_transform_input_bf16(const uint16_t* x, int64_t M, int64_t K, const float* suh, int s,
                              uint16_t* a) {
  std::vector<uint16_t> xv(x, x + (size_t)(M * K));
  auto out = trellis_ref::TransformInput(xv, M, K, suh, s);
  std::memcpy(a, out.data(), out.size() * 2);
}
void ref_linear_from_a(const uint16_t* a0, const uint16_t* a1, int64_t n_split, int64_t M, int64_t K,
                       int64_t N, const uint16_t* q, const float* svh, int s, double* y) {
  std::vector<const uint16_t*> a{a0};
  if (a1) a.push_back(a1);
  std::vector<uint16_t> qv(q, q + (size_t)(K * N));
  auto out = trellis_ref::LinearFromA(a, M, K, N, n_split, qv, svh, s);
  std::memcpy(y, out.data(), out.size() * 8);
}
void ref_epilogue_from_raw(const float* s, int64_t M, int64_t N, const float* svh, float out_scale,
                           uint16_t* c) {
  std::vector<float> sv(s, s + (size_t)(M * N));
  auto out = trellis_ref::EpilogueFromRaw(sv, M, N, svh, out_scale);
  std::memcpy(c, out.data(), out.size() * 2);
}

// int8 (M is the layout's 256 for the activation quantizers)
void ref_i8_quant_w_blk(const uint16_t* q, int K, int N, float* sw, int8_t* wp) {
  std::vector<float> s; std::vector<int8_t> w;
  i8p::QuantizeWeightsRef(q, K, N, s, w);
  std::memcpy(sw, s.data(), s.size() * 4); std::memcpy(wp, w.data(), w.size());
}
void ref_i8_quant_w_col(const uint16_t* q, int K, int N, float* sw, int8_t* wp) {
  std::vector<float> s; std::vector<int8_t> w;
  i8p::QuantizeWeightsColRef(q, K, N, s, w);
  std::memcpy(sw, s.data(), s.size() * 4); std::memcpy(wp, w.data(), w.size());
}
void ref_i8_quant_act_blk(const float* x, int K, float* sa, int8_t* ap) {
  std::vector<float> s; std::vector<int8_t> a;
  i8p::QuantizeActRef(x, K, s, a);
  std::memcpy(sa, s.data(), s.size() * 4); std::memcpy(ap, a.data(), a.size());
}
void ref_i8_quant_act_row(const float* x, int K, float* sa, int8_t* ap) {
  std::vector<float> s; std::vector<int8_t> a;
  i8p::QuantizeActRowRef(x, K, s, a);
  std::memcpy(sa, s.data(), s.size() * 4); std::memcpy(ap, a.data(), a.size());
}
void ref_i8_gemm(const int8_t* A, const float* sa, const int8_t* W, const float* sw, int M, int N, int K,
                 int mask, double* C) {
  i8p::RefGemmInt8(A, sa, W, sw, M, N, K, mask, C);
}
size_t ref_a8_offset(int r, int k, int K) { return i8p::A8Offset(r, k, K); }
size_t ref_w8_offset(int n, int k, int K) { return i8p::W8Offset(n, k, K); }
int8_t ref_i8_quant_w(uint16_t w, uint16_t rs) { return i8p::QuantWTrick(w, rs); }
uint16_t ref_i8_rs_half(float s) { return i8p::RsHalf(s); }

// w4a16
void ref_w4_quantize_pack(const float* w, int N, int K, int group, uint32_t* wq, uint32_t* wsz) {
  std::vector<uint8_t> q, z; std::vector<float> sc;
  r4dx_convert::QuantizeInt4Asymmetric(w, N, K, group, 1, q, sc, z);
  auto a = r4dx_convert::PackW4Nibbles(q, N, K, 1);
  auto b = r4dx_convert::PackW4A16Scales(sc, z, N, K, group);
  std::memcpy(wq, a.data(), a.size() * 4);
  std::memcpy(wsz, b.data(), b.size() * 4);
}

int32_t ref_argmax(const float* x, int64_t n, float* v) {
  auto p = r4dx::kernels::ArgmaxDirectRef(x, n);
  if (v) *v = p.v;
  return p.i;
}

// weight fake-quant: Q f16 bits widened to fp32, as the reference's own test feeds it
void ref_wq_table(const uint16_t* q, int64_t K, int64_t N, int group, float* t) {
  std::vector<float> qf(static_cast<size_t>(K * N));
  for (size_t i = 0; i < qf.size(); ++i) qf[i] = r4dx::core::F16ToFloat(q[i]);
  auto v = r4dx::model::FakeQuantWTableRef(qf.data(), K, N, group);
  std::memcpy(t, v.data(), v.size() * 4);
}
void ref_wq_apply(const uint16_t* q, int64_t K, int64_t N, int group, const float* t, float* out) {
  std::vector<float> qf(static_cast<size_t>(K * N));
  for (size_t i = 0; i < qf.size(); ++i) qf[i] = r4dx::core::F16ToFloat(q[i]);
  std::vector<float> tab(t, t + static_cast<size_t>(K / group) * static_cast<size_t>(N));
  auto v = r4dx::model::FakeQuantWApplyRef(qf.data(), K, N, group, tab);
  std::memcpy(out, v.data(), v.size() * 4);
}

uint16_t ref_f32_to_f16(float f) { return r4dx::core::FloatToF16(f); }
uint16_t ref_f32_to_bf16(float f) { return r4dx::core::FloatToBf16(f); }

}  // extern "C"
