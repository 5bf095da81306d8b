/* r4o.c -- CPU oracle for r4dx's quantized-weight matrix-product path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker the HIP kernels are compared against (tests/, the smoke
 * check and bench.py's cpu_baseline leg).  Never linked into or called by the product.
 * Every function restates the arithmetic of the reference CPU code it cites (paths relative to
 * the reference repository root); see r4o.h for how each one is pinned.
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off -fopenmp).  -ffp-contract=off is load-bearing:
 * every product below is a separately rounded operation.
 */
#include "r4o.h"

#include <math.h>
#include <string.h>
#include <stdlib.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define NT(n) ((n) > 0 ? (n) : r4o_max_threads())

int r4o_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

double r4o_now_seconds(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* ---- scalar conversions ---------------------------------------------------------------------- */
/* src/core/include/r4dx/core/dtype.hpp:79-140 (F16ToFloat / FloatToF16), restated from IEEE 754. */
static uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float f32_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float r4o_f16_to_f32(uint16_t h) {
  const int sign = (h >> 15) & 1, e = (h >> 10) & 0x1F, m = h & 0x3FF;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);                 /* zero / subnormal: m * 2^-24 */
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(m + 1024), e - 25);            /* (1024 + m) * 2^(e - 15 - 10) */
  return sign ? -v : v;
}

/* One rounding from double to binary16, nearest-even; overflow -> inf; NaN -> quiet NaN. */
uint16_t r4o_f64_to_f16(double x) {
  if (isnan(x)) return 0x7E00;
  const uint16_t sign = signbit(x) ? 0x8000 : 0;
  double a = fabs(x);
  if (isinf(a)) return sign | 0x7C00;
  if (a == 0.0) return sign;
  int ex;
  frexp(a, &ex);                 /* a = f * 2^ex, f in [0.5, 1) -> a = 1.x * 2^(ex-1) */
  int e = ex - 1;
  if (e < -14) {                 /* subnormal range: units of 2^-24 */
    double r = nearbyint(ldexp(a, 24));
    return sign | (uint16_t)r;   /* r == 1024 is exactly the smallest normal's bits */
  }
  double r = nearbyint(ldexp(a, 10 - e));   /* significand in [1024, 2048] */
  if (r >= 2048.0) { r = 1024.0; ++e; }
  if (e > 15) return sign | 0x7C00;
  return sign | (uint16_t)(((e + 15) << 10) | ((int)r - 1024));
}

uint16_t r4o_f32_to_f16(float f) { return r4o_f64_to_f16((double)f); }

float r4o_bf16_to_f32(uint16_t h) { return f32_of((uint32_t)h << 16); }

/* dtype.hpp:64-73 FloatToBf16: nearest-even on the top half, NaN kept quiet. */
uint16_t r4o_f32_to_bf16(float f) {
  const uint32_t u = bits_of(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  const uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7FFFu + lsb) >> 16);
}

/* ---- trellis format ---------------------------------------------------------------------------- */
/* trellis_ref.hpp:40-53: the "mul1" codebook.  x = s * 0x83DCD12D mod 2^32, bs = byte sum of x,
 * value = f16((1024 + bs) * f16(0x1EEE) + f16(0xC931)) rounded once (the fp64 value is exact). */
void r4o_codebook(uint16_t* out) {
  const double kinv = (double)r4o_f16_to_f32(0x1EEE), kbias = (double)r4o_f16_to_f32(0xC931);
  for (uint32_t s = 0; s < 65536u; ++s) {
    const uint32_t x = s * 0x83DCD12Du;
    const uint32_t bs = (x & 0xFFu) + ((x >> 8) & 0xFFu) + ((x >> 16) & 0xFFu) + (x >> 24);
    out[s] = r4o_f64_to_f16((1024.0 + (double)bs) * kinv + kbias);
  }
}

/* trellis_ref.hpp:56-62: the 16 ring bits ending at bit KB*(p+1), stream bit i at bit 31 - i%32 of
 * word i/32, the ring of 256*KB bits wrapping around (tail-biting). */
uint32_t r4o_trellis_state(const uint32_t* ring, int KB, int p) {
  const int R = 256 * KB, nw = 8 * KB;
  const int start = ((KB * (p + 1) - 16) % R + R) % R;
  const int i0 = start / 32, off = start % 32;
  const uint64_t win = ((uint64_t)ring[i0] << 32) | (uint64_t)ring[(i0 + 1) % nw];
  return (uint32_t)((win >> (48 - off)) & 0xFFFFu);
}

/* trellis_ref.hpp:65-70: position p = 8t + j -> tile element r*16 + c (r = k, c = n). */
int r4o_tc_perm(int p) {
  const int t = p / 8, j = p % 8;
  const int r0 = (t % 4) * 2, c0 = t / 4;
  const int rr = (j & 3) < 2 ? r0 + (j & 1) : r0 + 8 + (j & 1);
  return rr * 16 + c0 + (j >= 4 ? 8 : 0);
}

/* trellis_ref.hpp:81-83 / docs/trellis-kernel.md:103-130: the pair grid. */
size_t r4o_pair_grid_index(int64_t K, int KB, int64_t tn, int64_t tk) {
  return (size_t)((((tn >> 1) * (K / 16) + tk) * 2 + (tn & 1)) * 8 * KB);
}

void r4o_to_pair_grid(const uint32_t* words, int64_t K, int64_t N, int KB, uint32_t* grid) {
  const int nw = 8 * KB;
  for (int64_t tk = 0; tk < K / 16; ++tk)
    for (int64_t tn = 0; tn < N / 16; ++tn)
      memcpy(grid + r4o_pair_grid_index(K, KB, tn, tk), words + (size_t)(tk * (N / 16) + tn) * nw,
             (size_t)nw * 4);
}

static const uint16_t* codebook_table(void) {
  static uint16_t cb[65536];
  static int ready = 0;
#pragma omp critical(r4o_cb)
  {
    if (!ready) { r4o_codebook(cb); ready = 1; }
  }
  return cb;
}

/* trellis_ref.hpp:72-79, 109-115: every tile of the pair grid into Q[K][N]. */
void r4o_decode_pair_grid(const uint32_t* grid, int64_t K, int64_t N, int KB, uint16_t* q,
                          int nthreads) {
  const uint16_t* cb = codebook_table();
  int perm[256];
  for (int p = 0; p < 256; ++p) perm[p] = r4o_tc_perm(p);
  const int64_t tiles_n = N / 16, tiles_k = K / 16;
#pragma omp parallel for num_threads(NT(nthreads)) schedule(static)
  for (int64_t tn = 0; tn < tiles_n; ++tn)
    for (int64_t tk = 0; tk < tiles_k; ++tk) {
      const uint32_t* ring = grid + r4o_pair_grid_index(K, KB, tn, tk);
      for (int p = 0; p < 256; ++p) {
        const int e = perm[p];
        q[(16 * tk + e / 16) * N + 16 * tn + e % 16] = cb[r4o_trellis_state(ring, KB, p)];
      }
    }
}

/* ---- FWHT-128 and the linear around the decode ------------------------------------------------ */
/* trellis_ref.hpp:120-131 FwhtLdsF32: stages lg = 0..6, (a + b, a - b) on (i, i + 2^lg), fp32. */
void r4o_fwht128_f32(float* v) {
  for (int h = 1; h < 128; h <<= 1)
    for (int i0 = 0; i0 < 128; i0 += 2 * h)
      for (int i = i0; i < i0 + h; ++i) {
        const float a = v[i], b = v[i + h];
        v[i] = a + b;
        v[i + h] = a - b;
      }
}

void r4o_fwht128_f64(double* v) {
  for (int h = 1; h < 128; h <<= 1)
    for (int i0 = 0; i0 < 128; i0 += 2 * h)
      for (int i = i0; i < i0 + h; ++i) {
        const double a = v[i], b = v[i + h];
        v[i] = a + b;
        v[i + h] = a - b;
      }
}

/* ---- the activation producers in front of the transform ----------------------------------------- */
/* src/kernels/src/r4dx_kernels.hip:38 Sigmoid: 1 / (1 + expf(-x)) in fp32 (the host libm's expf here; the
 * GPU's device-library expf may differ from it by an ulp, so the producers are pinned within one bf16 ulp). */
static float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

/* src/kernels/src/r4dx_kernels.hip:416-470 SiluMulWideKernel's element (and trellis_transform.hip:119-123):
 * h = bf16(g * sigmoid(g) * u), g = gate_up[r][i], u = gate_up[r][intermediate + i], two fp32 products in that
 * order, then nearest-even bf16.  out [rows][intermediate]. */
void r4o_silu_mul_bf16(const uint16_t* gate_up, int64_t rows, int64_t intermediate, int64_t in_row_stride,
                       uint16_t* out) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t i = 0; i < intermediate; ++i) {
      const float g = r4o_bf16_to_f32(gate_up[r * in_row_stride + i]);
      const float u = r4o_bf16_to_f32(gate_up[r * in_row_stride + intermediate + i]);
      const float gs = g * sigmoid_f32(g);
      out[r * intermediate + i] = r4o_f32_to_bf16(gs * u);
    }
}

/* trellis_transform.hip:152-170 GateMulTrellisKernel's element (attn_kernels.hip's GateMulKernel):
 * h = bf16(a * (1 / (1 + expf(-g)))) over n elements. */
void r4o_attn_gate_mul_bf16(const uint16_t* attn_out, const uint16_t* gate, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i)
    out[i] = r4o_f32_to_bf16(r4o_bf16_to_f32(attn_out[i]) * sigmoid_f32(r4o_bf16_to_f32(gate[i])));
}

/* trellis_ref.hpp:146-148: float(2^s / sqrt(128)), one rounding from double. */
float r4o_transform_scale(int prescale_log2) {
  return (float)(ldexp(1.0, prescale_log2) / sqrt(128.0));
}

/* trellis_ref.hpp:150-169 TransformInput (and trellis_transform.hip:63-100): per 128-block,
 * v = fp32(x) * suh (fp32), FWHT in fp32, a = f16(fp32(v * scale)). */
void r4o_transform_input(const uint16_t* x, int x_is_bf16, int64_t M, int64_t K,
                         const float* suh, int prescale_log2, uint16_t* a) {
  const float scale = r4o_transform_scale(prescale_log2);
  float v[128];
  for (int64_t m = 0; m < M; ++m)
    for (int64_t k0 = 0; k0 < K; k0 += 128) {
      for (int i = 0; i < 128; ++i) {
        const uint16_t b = x[m * K + k0 + i];
        const float xv = x_is_bf16 ? r4o_bf16_to_f32(b) : r4o_f16_to_f32(b);
        v[i] = xv * suh[k0 + i];
      }
      r4o_fwht128_f32(v);
      for (int i = 0; i < 128; ++i) {
        const float s = v[i] * scale;
        a[m * K + k0 + i] = r4o_f32_to_f16(s);
      }
    }
}

void r4o_raw_sums_f64(const uint16_t* a0, const uint16_t* a1, int64_t n_split, int64_t M,
                      int64_t K, int64_t N, const uint16_t* q, double* s, int nthreads) {
  if (!a1) { a1 = a0; n_split = N; }
  float* qf = (float*)malloc((size_t)(K * N) * sizeof(float));
#pragma omp parallel for num_threads(NT(nthreads)) schedule(static)
  for (int64_t i = 0; i < K * N; ++i) qf[i] = r4o_f16_to_f32(q[i]);
  for (int64_t m = 0; m < M; ++m) {
    double* row = s + m * N;
#pragma omp parallel num_threads(NT(nthreads))
    {
      /* each thread owns a column range: the k loop stays sequential per column */
#ifdef _OPENMP
      const int nt = omp_get_num_threads(), tid = omp_get_thread_num();
#else
      const int nt = 1, tid = 0;
#endif
      const int64_t c0 = N * tid / nt, c1 = N * (tid + 1) / nt;
      for (int64_t n = c0; n < c1; ++n) row[n] = 0.0;
      for (int64_t k = 0; k < K; ++k) {
        const double v0 = (double)r4o_f16_to_f32(a0[m * K + k]);
        const double v1 = (double)r4o_f16_to_f32(a1[m * K + k]);
        const float* qr = qf + k * N;
        for (int64_t n = c0; n < c1; ++n) row[n] += (n < n_split ? v0 : v1) * (double)qr[n];
      }
    }
  }
  free(qf);
}

/* trellis_ref.hpp:173-196 LinearFromA: fp64 2^-s/sqrt(128) * svh[n] * FWHT128_n(A_p(n) @ Q). */
void r4o_linear_from_a(const uint16_t* a0, const uint16_t* a1, int64_t n_split, int64_t M,
                       int64_t K, int64_t N, const uint16_t* q, const float* svh,
                       int prescale_log2, double* y, int nthreads) {
  r4o_raw_sums_f64(a0, a1, n_split, M, K, N, q, y, nthreads);
  const double out_scale = ldexp(1.0, -prescale_log2) / sqrt(128.0);
  for (int64_t m = 0; m < M; ++m) {
    double* row = y + m * N;
    for (int64_t n0 = 0; n0 < N; n0 += 128) r4o_fwht128_f64(row + n0);
    for (int64_t n = 0; n < N; ++n) row[n] = row[n] * out_scale * (double)svh[n];
  }
}

/* trellis_ref.hpp:231-247 EpilogueFromRaw: FWHT in fp32, (y * svh) * out_scale, one bf16 rounding. */
void r4o_epilogue_from_raw(const float* s, int64_t M, int64_t N, const float* svh,
                           float out_scale, uint16_t* c) {
  float v[128];
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n0 = 0; n0 < N; n0 += 128) {
      memcpy(v, s + m * N + n0, sizeof v);
      r4o_fwht128_f32(v);
      for (int i = 0; i < 128; ++i) {
        const float y = v[i] * svh[n0 + i];
        const float z = y * out_scale;
        c[m * N + n0 + i] = r4o_f32_to_bf16(z);
      }
    }
}

/* ---- int8 ------------------------------------------------------------------------------------- */
/* int8_gemm_proto_ref.h:57-63: rs = f16(min(1/s, 60000)), s_eff = 1 / rs. */
uint16_t r4o_i8_rs_half(float s) {
  float r = 1.0f / s;
  if (r > 60000.0f) r = 60000.0f;
  return r4o_f32_to_f16(r);
}
float r4o_i8_seff(float s) { return 1.0f / r4o_f16_to_f32(r4o_i8_rs_half(s)); }

static float wscale0(float amax) { return amax > 0.f ? amax / 127.0f : 1.0f; }

/* int8_gemm_proto_ref.h:74-77 QuantWTrick: low byte of f16(w * rs + 1536), rounded once. */
int8_t r4o_i8_quant_w(uint16_t wbits, uint16_t rsbits) {
  const double v = (double)r4o_f16_to_f32(wbits) * (double)r4o_f16_to_f32(rsbits) + 1536.0;
  return (int8_t)(uint8_t)(r4o_f64_to_f16(v) & 0xFFu);
}

/* int8_gemm_proto_ref.h:84-89 QuantAct: clamp(rint(x / s), -127, 127), IEEE fp32 division. */
int8_t r4o_i8_quant_act(float x, float s) {
  float q = nearbyintf(x / s);
  if (q < -127.f) q = -127.f;
  if (q > 127.f) q = 127.f;
  return (int8_t)(int)q;
}

void r4o_i8_quant_act_blk(const uint16_t* x, int M, int K, float* sa, int8_t* ap) {
  const int nkb = K / 128;
  for (int r = 0; r < M; ++r)
    for (int kb = 0; kb < nkb; ++kb) {
      float amax = 0.f;
      for (int k = kb * 128; k < kb * 128 + 128; ++k)
        amax = fmaxf(amax, fabsf(r4o_f16_to_f32(x[(size_t)r * K + k])));
      const float s = wscale0(amax);
      sa[(size_t)kb * M + r] = s;
      for (int k = kb * 128; k < kb * 128 + 128; ++k)
        ap[(size_t)r * K + k] = r4o_i8_quant_act(r4o_f16_to_f32(x[(size_t)r * K + k]), s);
    }
}

void r4o_i8_quant_act_row(const uint16_t* x, int M, int K, float* sa, int8_t* ap) {
  for (int r = 0; r < M; ++r) {
    float amax = 0.f;
    for (int k = 0; k < K; ++k) amax = fmaxf(amax, fabsf(r4o_f16_to_f32(x[(size_t)r * K + k])));
    const float s = wscale0(amax);
    sa[r] = s;
    for (int k = 0; k < K; ++k)
      ap[(size_t)r * K + k] = r4o_i8_quant_act(r4o_f16_to_f32(x[(size_t)r * K + k]), s);
  }
}

static void quant_w_range(const uint16_t* q, int K, int N, int n, int k0, int k1, float* sw_out,
                          int8_t* wp) {
  float amax = 0.f;
  for (int k = k0; k < k1; ++k) amax = fmaxf(amax, fabsf(r4o_f16_to_f32(q[(size_t)k * N + n])));
  const uint16_t rs = r4o_i8_rs_half(wscale0(amax));
  *sw_out = 1.0f / r4o_f16_to_f32(rs);
  for (int k = k0; k < k1; ++k) wp[(size_t)n * K + k] = r4o_i8_quant_w(q[(size_t)k * N + n], rs);
}

/* int8_gemm_proto_ref.h:124-137 QuantizeWeightsRef */
void r4o_i8_quant_w_blk(const uint16_t* q, int K, int N, float* sw, int8_t* wp) {
  for (int kb = 0; kb < K / 128; ++kb)
    for (int n = 0; n < N; ++n) quant_w_range(q, K, N, n, kb * 128, kb * 128 + 128, &sw[(size_t)kb * N + n], wp);
}
/* int8_gemm_proto_ref.h:164-176 QuantizeWeightsColRef */
void r4o_i8_quant_w_col(const uint16_t* q, int K, int N, float* sw, int8_t* wp) {
  for (int n = 0; n < N; ++n) quant_w_range(q, K, N, n, 0, K, &sw[n], wp);
}

void r4o_i8_gemm_i32(const int8_t* a, const int8_t* w, int M, int N, int K, int32_t* acc,
                     int nthreads) {
#pragma omp parallel for num_threads(NT(nthreads)) schedule(static) collapse(2)
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n) {
      int64_t s = 0;
      const int8_t* ar = a + (size_t)m * K;
      const int8_t* wr = w + (size_t)n * K;
      for (int k = 0; k < K; ++k) s += (int32_t)ar[k] * (int32_t)wr[k];
      acc[(size_t)m * N + n] = (int32_t)s;
    }
}

/* int8_gemm_proto_ref.h:95-110 RefGemmInt8 */
void r4o_i8_gemm_ref(const int8_t* a, const float* sa, const int8_t* w, const float* sw, int M,
                     int N, int K, int mask, double* c, int nthreads) {
  const int nkb = K / 128;
#pragma omp parallel for num_threads(NT(nthreads)) schedule(static) collapse(2)
  for (int r = 0; r < M; ++r)
    for (int n = 0; n < N; ++n) {
      double acc = 0.0;
      for (int kb = 0; kb < nkb; ++kb) {
        int64_t s = 0;
        for (int k = kb * 128; k < kb * 128 + 128; ++k)
          s += (int32_t)a[(size_t)r * K + k] * (int32_t)w[(size_t)n * K + k];
        const float sav = (mask & 1) ? sa[r] : sa[(size_t)kb * M + r];
        const float swv = (mask & 2) ? sw[n] : sw[(size_t)kb * N + n];
        acc += (double)sav * (double)swv * (double)s;
      }
      c[(size_t)r * N + n] = acc;
    }
}

/* r4d_trellis_i8_layout.h:32-45: element (row r, k) of the plain A in the A8 fragment layout. */
size_t r4o_a8_offset(int r, int k, int K) {
  const int k16 = k & 15;
  const int h = (k16 >> 2) & 1, e = 4 * (k16 >> 3) + (k16 & 3);
  const int lane = (r & 15) + 16 * h;
  const int rg = r >> 6, kt = k >> 4, i = (r >> 4) & 3, KT = K >> 4;
  return ((((size_t)rg * KT + kt) * 4 + i) * 32 + lane) * 8 + e;
}

/* r4d_trellis_i8_layout.h:24-27,56-64 W8Offset: the (32-column pair, 16-k tile) block is 512 B; lane L's
 * 16 B = fragment F0 then F1, element e of F on lane L is column 32 pair + 16 ((L >> 3) & 1) + 8 F + (L & 7)
 * and k = 16 kt + 8 (e >> 2) + 4 (L >> 4) + (e & 3). */
size_t r4o_w8_offset(int n, int k, int K) {
  const int k16 = k & 15;
  const int h = (k16 >> 2) & 1, e = 4 * (k16 >> 3) + (k16 & 3);
  const int pair = n >> 5, j = n & 31, t = j >> 4, F = (j >> 3) & 1, c = j & 7;
  const int lane = 16 * h + 8 * t + c;
  return ((size_t)pair * (K >> 4) + (k >> 4)) * 512 + (size_t)lane * 16 + F * 8 + e;
}

void r4o_pack_w8(const int8_t* wp, int N, int K, int8_t* w8) {
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k) w8[r4o_w8_offset(n, k, K)] = wp[(size_t)n * K + k];
}

void r4o_pack_a8(const int8_t* ap, int K, int8_t* a8) {
  for (int r = 0; r < 256; ++r)
    for (int k = 0; k < K; ++k) a8[r4o_a8_offset(r, k, K)] = ap[(size_t)r * K + k];
}

/* ---- w4a16 ------------------------------------------------------------------------------------ */
static int32_t round_haz(float x) {   /* quant_int4.hpp:65-68: half away from zero, in fp32 */
  return x >= 0.0f ? (int32_t)floorf(x + 0.5f) : (int32_t)ceilf(x - 0.5f);
}
static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* quant_int4.hpp:95-160 QuantizeInt4Asymmetric */
void r4o_w4_quantize(const float* w, int N, int K, int group, uint8_t* q, float* scale,
                     uint8_t* zero) {
  const int gpr = K / group;
  for (int n = 0; n < N; ++n)
    for (int g = 0; g < gpr; ++g) {
      const float* wg = w + (size_t)n * K + (size_t)g * group;
      float lo = wg[0], hi = wg[0];
      for (int k = 1; k < group; ++k) { lo = fminf(lo, wg[k]); hi = fmaxf(hi, wg[k]); }
      const float range = hi - lo;
      float sc;
      int zp, dz = 0;
      if (range <= 0.0f) {
        if (hi == 0.0f) { sc = 0.0f; zp = 0; dz = 1; }
        else { sc = fabsf(hi); zp = hi >= 0.0f ? 0 : 15; }
      } else {
        sc = fmaxf(range, 1e-12f) / 15.0f;
        zp = clampi(round_haz(-lo / sc), 0, 15);
      }
      scale[(size_t)n * gpr + g] = sc;
      zero[(size_t)n * gpr + g] = (uint8_t)zp;
      for (int k = 0; k < group; ++k)
        q[(size_t)n * K + (size_t)g * group + k] =
            (uint8_t)(dz ? 0 : clampi(round_haz(wg[k] / sc) + zp, 0, 15));
    }
}

/* The k offset, inside a 16-k step and a lane half, of nibble i of a packed dword
 * (quant_int4.hpp:56 kNibbleKOffset, derived there from the RDNA4 kernel's fragment order). */
static const int kNibK[8] = {0, 8, 1, 9, 2, 10, 3, 11};

/* quant_int4.hpp:171-198 PackW4Nibbles: dword (((t*KB64 + kb)*2 + lh)*16 + r)*4 + s, nibble i =
 * q[16t + r][64kb + 16s + 4lh + kNibK[i]] ^ 8. */
void r4o_w4_pack(const uint8_t* q, int N, int K, uint32_t* wq) {
  const int kblocks = K / 64;
  for (int t = 0; t < N / 16; ++t)
    for (int kb = 0; kb < kblocks; ++kb)
      for (int lh = 0; lh < 2; ++lh)
        for (int r = 0; r < 16; ++r)
          for (int s = 0; s < 4; ++s) {
            uint32_t d = 0;
            for (int i = 0; i < 8; ++i) {
              const int k = kb * 64 + s * 16 + 4 * lh + kNibK[i];
              d |= ((uint32_t)(q[(size_t)(16 * t + r) * K + k] ^ 8u) & 0xFu) << (4 * i);
            }
            wq[((((size_t)t * kblocks + kb) * 2 + lh) * 16 + r) * 4 + s] = d;
          }
}

/* quant_int4.hpp:222-244 PackW4A16Scales: low half f16(scale), high half f16(-(1024 + zero)). */
void r4o_w4_pack_scales(const float* scale, const uint8_t* zero, int N, int K, int group,
                        uint32_t* wsz) {
  const int gpr = K / group;
  size_t o = 0;
  for (int t = 0; t < N / 16; ++t)
    for (int g = 0; g < gpr; ++g)
      for (int r = 0; r < 16; ++r, ++o) {
        const size_t gi = (size_t)(16 * t + r) * gpr + g;
        const uint16_t sc = r4o_f32_to_f16(scale[gi]);
        const uint16_t nz = r4o_f32_to_f16(-(1024.0f + (float)zero[gi]));
        wsz[o] = (uint32_t)sc | ((uint32_t)nz << 16);
      }
}

static void w4_unpack_row_group(const uint32_t* wsz, int N, int K, int group, int n, int g,
                                float* sc, float* zf) {
  (void)N;
  const int gpr = K / group;
  const uint32_t d = wsz[((size_t)(n / 16) * gpr + g) * 16 + (n % 16)];
  *sc = r4o_f16_to_f32((uint16_t)(d & 0xFFFFu));
  *zf = -r4o_f16_to_f32((uint16_t)(d >> 16)) - 1024.0f;   /* the integer zero point */
}

static int w4_code(const uint32_t* wq, int K, int n, int k) {
  const int kblocks = K / 64, t = n / 16, r = n % 16, kb = k / 64, kk = k % 64;
  const int s = kk / 16, k16 = kk % 16, lh = (k16 >> 2) & 1;
  const int j = k16 & 3, hi8 = k16 >> 3;   /* k16 = 4lh + kNibK[i]: kNibK[i] = j + 8*hi8 */
  const int i = 2 * j + hi8;
  const uint32_t d = wq[((((size_t)t * kblocks + kb) * 2 + lh) * 16 + r) * 4 + s];
  return (int)(((d >> (4 * i)) & 0xFu) ^ 8u);
}

void r4o_w4_dequant(const uint32_t* wq, const uint32_t* wsz, int N, int K, int group, float* w) {
  for (int n = 0; n < N; ++n)
    for (int g = 0; g < K / group; ++g) {
      float sc, zf;
      w4_unpack_row_group(wsz, N, K, group, n, g, &sc, &zf);
      for (int k = g * group; k < (g + 1) * group; ++k)
        w[(size_t)n * K + k] = sc * ((float)w4_code(wq, K, n, k) - zf);
    }
}

void r4o_w4_gemm_ref(const uint16_t* a, const uint32_t* wq, const uint32_t* wsz, int M, int N,
                     int K, int group, double* y, int nthreads) {
  const int gpr = K / group;
  double* af = (double*)malloc((size_t)M * K * sizeof(double));
  for (size_t i = 0; i < (size_t)M * K; ++i) af[i] = (double)r4o_f16_to_f32(a[i]);
#pragma omp parallel num_threads(NT(nthreads))
  {
    int* codes = (int*)malloc((size_t)K * sizeof(int));
#pragma omp for schedule(static)
    for (int n = 0; n < N; ++n) {
      for (int k = 0; k < K; ++k) codes[k] = w4_code(wq, K, n, k);
      for (int m = 0; m < M; ++m) {
        double acc = 0.0;
        for (int g = 0; g < gpr; ++g) {
          float sc, zf;
          w4_unpack_row_group(wsz, N, K, group, n, g, &sc, &zf);
          double s = 0.0;
          for (int k = g * group; k < (g + 1) * group; ++k)
            s += af[(size_t)m * K + k] * (double)(codes[k] - (int)zf);
          acc += (double)sc * s;
        }
        y[(size_t)m * N + n] = acc;
      }
    }
    free(codes);
  }
  free(af);
}

/* argmax_ref.hpp:22-41: seed (-inf, 0); a larger value wins, an equal one the lower index; a NaN
 * never compares greater, so it never wins. */
int32_t r4o_argmax_f32(const float* x, int64_t n, float* best_val) {
  float bv = -INFINITY;
  int32_t bi = 0;
  for (int64_t i = 0; i < n; ++i)
    if (x[i] > bv || (x[i] == bv && (int32_t)i < bi)) { bv = x[i]; bi = (int32_t)i; }
  if (best_val) *best_val = bv;
  return bi;
}

/* ---- weight fake-quant (src/model/fake_quant_w.h:96-140) ----------------------------------------------------
 * A group is `group` consecutive k of one column n of Q; s = max|w| / 127 in fp32 (1 for an all-zero group);
 * a value becomes f16(clamp(rint(w * (1 / s)), -127, 127) * s), every step but the last in fp32 (nearbyintf
 * under the default rounding mode is round half to even). */
void r4o_wq_table(const uint16_t* q, int64_t K, int64_t N, int group, float* t) {
  for (int64_t g = 0; g < K / group; ++g)
    for (int64_t n = 0; n < N; ++n) {
      float amax = 0.0f;
      for (int i = 0; i < group; ++i) amax = fmaxf(amax, fabsf(r4o_f16_to_f32(q[(g * group + i) * N + n])));
      t[g * N + n] = amax > 0.0f ? amax / 127.0f : 1.0f;
    }
}

void r4o_wq_apply(const uint16_t* q, int64_t K, int64_t N, int group, const float* t, uint16_t* out) {
  for (int64_t k = 0; k < K; ++k)
    for (int64_t n = 0; n < N; ++n) {
      const float s = t[(k / group) * N + n];
      const float rs = 1.0f / s;
      float v = nearbyintf(r4o_f16_to_f32(q[k * N + n]) * rs);
      v = fminf(fmaxf(v, -127.0f), 127.0f);
      const float p = v * s;
      out[k * N + n] = r4o_f32_to_f16(p);
    }
}
