// trellis_input.hip -- the input side of a trellis linear on gfx950 (reference entry:
// src/kernels/include/r4dx/kernels/kernels.h:110-128, arithmetic src/kernels/src/trellis_transform.hip:
// 63-100 and tests/kernels/trellis_ref.hpp:150-169):
//   out[o][m, k] = f16( fp32( FWHT128( fp32(x[m, :]) * suh[o][:] )[k] * scale ) ),  scale = float(2^s / sqrt(128))
// per 128-block, fp32 butterflies in the reference's stage order, the product x * suh and the final
// product each rounded to fp32, then ONE rounding to f16. One wave64 per (128-block, row): lane l
// holds elements l and l + 64. Also r4dx_fwht128_f32 (kernels.h:192-197).
#include "r4d_dev.h"
#include "r4d_host.h"
#include "r4d_mi355x.h"

namespace {

constexpr int kMaxOut = 3;
struct OutPtrs {
  const float* suh[kMaxOut];
  unsigned short* out[kMaxOut];
};

template <bool BF16>
__global__ __launch_bounds__(64) void tq_input_kernel(const unsigned short* __restrict__ x, int64_t K,
                                                      int nout, OutPtrs p, float scale) {
  const int lane = threadIdx.x;
  const int64_t k0 = (int64_t)blockIdx.x * 128;
  const int64_t row = blockIdx.y;
  const unsigned short* xr = x + row * K + k0;
  const float x0 = BF16 ? r4_bf16_to_f32(xr[lane]) : r4_f16_to_f32(xr[lane]);
  const float x1 = BF16 ? r4_bf16_to_f32(xr[lane + 64]) : r4_f16_to_f32(xr[lane + 64]);
#pragma unroll
  for (int o = 0; o < kMaxOut; ++o) {
    if (o >= nout) break;
    float v0 = x0 * p.suh[o][k0 + lane];
    float v1 = x1 * p.suh[o][k0 + lane + 64];
    r4_fwht128_wave(v0, v1, lane);
    unsigned short* dst = p.out[o] + row * K + k0;
    dst[lane] = r4_f16_rn(v0 * scale);
    dst[lane + 64] = r4_f16_rn(v1 * scale);
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
  if (bf16)
    hipLaunchKernelGGL(tq_input_kernel<true>, grid, block, 0, (hipStream_t)stream,
                       (const unsigned short*)x, K, nout, p, scale);
  else
    hipLaunchKernelGGL(tq_input_kernel<false>, grid, block, 0, (hipStream_t)stream,
                       (const unsigned short*)x, K, nout, p, scale);
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

void r4dx_fwht128_f32(int64_t x, int64_t blocks, int use_lds, int64_t stream) {
  (void)use_lds;
  if (blocks < 0) r4d::fail("fwht128_f32", "blocks must be >= 0");
  if (blocks == 0) return;
  if (!x) r4d::fail("fwht128_f32", "null x");
  hipLaunchKernelGGL(tq_fwht128_kernel, dim3((unsigned)blocks), dim3(64), 0, (hipStream_t)stream, (float*)x);
  r4d::launch_ok("fwht128_f32");
}

}  // extern "C"
