// trellis_input.hip -- the input side of a trellis linear on gfx950 (reference entry:
// src/kernels/include/r4dx/kernels/kernels.h:110-128, arithmetic src/kernels/src/trellis_transform.hip:
// 63-100 and tests/kernels/trellis_ref.hpp:150-169):
//   out[o][m, k] = f16( fp32( FWHT128( fp32(x[m, :]) * suh[o][:] )[k] * scale ) ),  scale = float(2^s / sqrt(128))
// per 128-block, fp32 butterflies in the reference's stage order, the product x * suh and the final
// product each rounded to fp32, then ONE rounding to f16. One wave64 per (128-block, row): lane l
// holds elements l and l + 64. Also r4dx_fwht128_f32 (kernels.h:192-197), and the fused producers
// (kernels.h:130-147; trellis_transform.hip:100-170): the transform of bf16(silu(gate) * up) or of
// bf16(attn_out * sigmoid(gate)) in one launch, each element the bf16 value the producer kernel
// (r4dx_silu_mul_wide_bf16, kernels.h:90-91; r4dx_model_attn_gate_mul_bf16, attn_kernels.h:30-31, also
// here) would have stored, so the result is byte-identical to the producer followed by the transform.
#include "r4d_dev.h"
#include "r4d_host.h"
#include "r4d_mi355x.h"

namespace {

constexpr int kMaxOut = 3;
struct OutPtrs {
  const float* suh[kMaxOut];
  unsigned short* out[kMaxOut];
};

template <int SRC, bool BF16>
__global__ __launch_bounds__(64) void tq_input_kernel(R4XSrc src, int64_t K, int nout, OutPtrs p, float scale) {
  const int lane = threadIdx.x;
  const int64_t k0 = (int64_t)blockIdx.x * 128;
  const int64_t row = blockIdx.y;
  const float x0 = r4_xsrc<SRC, BF16>(src, row, k0 + lane);
  const float x1 = r4_xsrc<SRC, BF16>(src, row, k0 + lane + 64);
  // every output's suh requested up front (an absent output reads the first one's): one memory round trip for the
  // wave instead of one per output
  float s0[kMaxOut], s1[kMaxOut];
#pragma unroll
  for (int o = 0; o < kMaxOut; ++o) {
    const float* sp = p.suh[o < nout ? o : 0];
    s0[o] = sp[k0 + lane];
    s1[o] = sp[k0 + lane + 64];
  }
  // every output computed (an absent one's work is discarded), so the loads above stay ahead of all of it
#pragma unroll
  for (int o = 0; o < kMaxOut; ++o) {
    float v0 = x0 * s0[o];
    float v1 = x1 * s1[o];
    r4_fwht128_wave(v0, v1, lane);
    if (o < nout) {
      unsigned short* dst = p.out[o] + row * K + k0;
      dst[lane] = r4_f16_rn(v0 * scale);
      dst[lane + 64] = r4_f16_rn(v1 * scale);
    }
  }
}

__global__ __launch_bounds__(64) void tq_fwht128_kernel(float* __restrict__ x) {
  const int lane = threadIdx.x;
  float* b = x + (int64_t)blockIdx.x * 128;
  float v0 = b[lane], v1 = b[lane + 64];
  r4_fwht128_wave(v0, v1, lane);
  b[lane] = v0;
  b[lane + 64] = v1;
}

void input_run(bool bf16, int64_t x, int64_t M, int64_t K, int nout, const int64_t* suh,
               const int64_t* out, int prescale_log2, int64_t stream, const char* entry) {
  if (nout < 1 || nout > kMaxOut) r4d::fail(entry, "nout must be 1..3");
  if (K <= 0 || K % 128) r4d::fail(entry, "K must be a positive multiple of 128");
  if (M < 0 || M > 65535) r4d::fail(entry, "M must be 0..65535");
  if (prescale_log2 < -24 || prescale_log2 > 24) r4d::fail(entry, "|prescale_log2| must be <= 24");
  if (!suh || !out) r4d::fail(entry, "null pointer array");
  if (M == 0) return;
  if (!x) r4d::fail(entry, "null x");
  OutPtrs p{};
  for (int o = 0; o < nout; ++o) {
    if (!suh[o] || !out[o]) r4d::fail(entry, "null suh or out");
    p.suh[o] = (const float*)suh[o];
    p.out[o] = (unsigned short*)out[o];
  }
  // float(2^s / sqrt(128)), rounded once from double (trellis_ref.hpp:146-148)
  const float scale = (float)(__builtin_ldexp(1.0, prescale_log2) / __builtin_sqrt(128.0));
  dim3 grid((unsigned)(K / 128), (unsigned)M), block(64);
  const R4XSrc src{(const unsigned short*)x, nullptr, (long long)K, 0};
  if (bf16)
    hipLaunchKernelGGL((tq_input_kernel<R4_SRC_X, true>), grid, block, 0, (hipStream_t)stream, src, K, nout, p, scale);
  else
    hipLaunchKernelGGL((tq_input_kernel<R4_SRC_X, false>), grid, block, 0, (hipStream_t)stream, src, K, nout, p, scale);
  r4d::launch_ok(entry);
}

// The producers' preconditions (trellis_transform.hip:508-519, 893-945): K a positive multiple of 128, rows
// 0..65535, |prescale_log2| <= 24, non-null suh and out; returns float(2^s / sqrt(128)).
float producer_scale(const char* entry, int64_t rows, int64_t K, int64_t suh, int64_t out, int prescale_log2) {
  if (K <= 0 || K % 128) r4d::fail(entry, "K must be a positive multiple of 128, got " + r4d::str(K));
  if (rows < 0 || rows > 65535) r4d::fail(entry, "rows must be 0..65535, got " + r4d::str(rows));
  if (prescale_log2 < -24 || prescale_log2 > 24) r4d::fail(entry, "|prescale_log2| must be <= 24");
  if (!suh || !out) r4d::fail(entry, "suh and out must be non-null");
  return (float)(__builtin_ldexp(1.0, prescale_log2) / __builtin_sqrt(128.0));
}

template <int SRC>
void producer_run(const R4XSrc& src, int64_t rows, int64_t K, int64_t suh, int64_t out, float scale,
                  int64_t stream, const char* entry) {
  if (rows == 0) return;
  OutPtrs p{};
  p.suh[0] = (const float*)suh;
  p.out[0] = (unsigned short*)out;
  hipLaunchKernelGGL((tq_input_kernel<SRC, true>), dim3((unsigned)(K / 128), (unsigned)rows), dim3(64), 0,
                     (hipStream_t)stream, src, K, 1, p, scale);
  r4d::launch_ok(entry);
}

// The producers alone (bf16 out): one thread per element.
template <int SRC>
__global__ __launch_bounds__(256) void producer_kernel(R4XSrc src, int64_t cols, int64_t total,
                                                       unsigned short* __restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t row = i / cols, k = i - row * cols;
    out[i] = r4_bf16_rn(r4_xsrc<SRC, true>(src, row, k));
  }
}
template <int SRC>
void producer_only(const R4XSrc& src, int64_t cols, int64_t total, int64_t out, int64_t stream, const char* entry) {
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL((producer_kernel<SRC>), dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0,
                     (hipStream_t)stream, src, cols, total, (unsigned short*)out);
  r4d::launch_ok(entry);
}

}  // namespace

extern "C" {

void r4dx_trellis_input_bf16(int64_t x, int64_t M, int64_t K, int nout, const int64_t* suh,
                             const int64_t* out, int prescale_log2, int64_t stream) {
  input_run(true, x, M, K, nout, suh, out, prescale_log2, stream, "trellis_input_bf16");
}

void r4dx_trellis_input_f16(int64_t x, int64_t M, int64_t K, int nout, const int64_t* suh,
                            const int64_t* out, int prescale_log2, int64_t stream) {
  input_run(false, x, M, K, nout, suh, out, prescale_log2, stream, "trellis_input_f16");
}

// kernels.h:130-145: the transform of bf16(g * sigmoid(g) * u) over gate_up rows [gate | up] (row stride
// in_row_stride >= 2 intermediate); out f16 [rows][intermediate] (mlp.down's A), suh fp32 [intermediate].
void r4dx_silu_mul_trellis_bf16(int64_t gate_up, int64_t rows, int64_t intermediate, int64_t in_row_stride,
                                int64_t suh, int64_t out, int prescale_log2, int64_t stream) {
  const char* e = "silu_mul_trellis_bf16";
  const float scale = producer_scale(e, rows, intermediate, suh, out, prescale_log2);
  if (!gate_up) r4d::fail(e, "gate_up is null");
  if (in_row_stride < 2 * intermediate) r4d::fail(e, "in_row_stride must be >= 2 * intermediate");
  const R4XSrc src{(const unsigned short*)gate_up, nullptr, (long long)in_row_stride, (long long)intermediate};
  producer_run<R4_SRC_SILU>(src, rows, intermediate, suh, out, scale, stream, e);
}

// kernels.h:146-147: the transform of bf16(attn_out * sigmoid(gate)), both bf16 [rows][K]; out f16 [rows][K].
void r4dx_attn_gate_mul_trellis_bf16(int64_t attn_out, int64_t gate, int64_t rows, int64_t K, int64_t suh,
                                     int64_t out, int prescale_log2, int64_t stream) {
  const char* e = "attn_gate_mul_trellis_bf16";
  const float scale = producer_scale(e, rows, K, suh, out, prescale_log2);
  if (!attn_out || !gate) r4d::fail(e, "attn_out and gate must be non-null");
  const R4XSrc src{(const unsigned short*)attn_out, (const unsigned short*)gate, (long long)K, 0};
  producer_run<R4_SRC_GATE>(src, rows, K, suh, out, scale, stream, e);
}

// kernels.h:90-91: out bf16 [rows][intermediate] = bf16(g * sigmoid(g) * u) (rows or intermediate <= 0: nothing).
void r4dx_silu_mul_wide_bf16(int64_t gate_up, int64_t out, int64_t rows, int64_t intermediate, int64_t in_row_stride,
                             int64_t stream) {
  if (rows <= 0 || intermediate <= 0) return;
  if (!gate_up || !out) r4d::fail("silu_mul_wide_bf16", "null pointer");
  if (in_row_stride < 2 * intermediate) r4d::fail("silu_mul_wide_bf16", "in_row_stride must be >= 2 * intermediate");
  const R4XSrc src{(const unsigned short*)gate_up, nullptr, (long long)in_row_stride, (long long)intermediate};
  producer_only<R4_SRC_SILU>(src, intermediate, rows * intermediate, out, stream, "silu_mul_wide_bf16");
}

// attn_kernels.h:26-31: out[i] = bf16(attn_out[i] * sigmoid(gate[i])) over n elements (n <= 0: nothing).
void r4dx_model_attn_gate_mul_bf16(int64_t attn_out, int64_t gate, int64_t out, int64_t n, int64_t stream) {
  if (n <= 0) return;
  if (!attn_out || !gate || !out) r4d::fail("model_attn_gate_mul_bf16", "null pointer");
  const R4XSrc src{(const unsigned short*)attn_out, (const unsigned short*)gate, 0, 0};
  producer_only<R4_SRC_GATE>(src, n, n, out, stream, "model_attn_gate_mul_bf16");
}

void r4dx_fwht128_f32(int64_t x, int64_t blocks, int use_lds, int64_t stream) {
  (void)use_lds;
  if (blocks < 0) r4d::fail("fwht128_f32", "blocks must be >= 0");
  if (blocks == 0) return;
  if (!x) r4d::fail("fwht128_f32", "null x");
  hipLaunchKernelGGL(tq_fwht128_kernel, dim3((unsigned)blocks), dim3(64), 0, (hipStream_t)stream, (float*)x);
  r4d::launch_ok("fwht128_f32");
}

}  // extern "C"
