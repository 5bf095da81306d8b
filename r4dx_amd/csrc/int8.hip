// int8.hip -- the activation quantizers of the int8 x int8 prefill GEMMs and the W8 packer on gfx950.
//
// Quantizers (the reference's arithmetic: tests/kernels/int8_gemm_proto_ref.h:84-89,138-189,
// third_party/libr4d/r4d_trellis_i8.h:160-208): s = amax / 127 (1 for an all-zero group), q = clamp(
// rint(x / s), -127, 127) with IEEE fp32 division, amax over a row (coarse) or over each (row, 128 k)
// block. They write the reference's A8 fragment layout (r4d_trellis_i8_layout.h:32-45, what
// r4d_trellis_i8_quant_act / _row produce, what the GEMMs read) or a plain [M][K] layout. The GEMMs
// themselves (trellis and dense) are in trellis_i8.hip.
#include "r4d_dev.h"
#include "r4d_host.h"
#include "r4d_mi355x.h"

namespace {

// ---- the A8 fragment layout (r4d_trellis_i8_layout.h:32-45) -----------------------------------------
__host__ __device__ inline size_t a8_offset(int r, int k, int K) {
  const int k16 = k & 15, h = (k16 >> 2) & 1, e = 4 * (k16 >> 3) + (k16 & 3);
  const int lane = (r & 15) + 16 * h;
  return ((((size_t)(r >> 6) * (K >> 4) + (k >> 4)) * 4 + ((r >> 4) & 3)) * 32 + lane) * 8 + e;
}

// ---- quantizers -----------------------------------------------------------------------------------
__device__ __forceinline__ float q_scale(float amax) { return amax > 0.f ? amax / 127.0f : 1.0f; }
__device__ __forceinline__ int q_one(float x, float s) {
  float q = __builtin_rintf(x / s);
  q = __builtin_fminf(__builtin_fmaxf(q, -127.f), 127.f);
  return (int)q;
}
// Four consecutive k of row r (k % 4 == 0) to their bytes, in the chosen layout (in the A8 layout four
// consecutive k are four consecutive bytes of one lane's fragment).
__device__ __forceinline__ void q_store4(signed char* __restrict__ out, bool ref_layout, int r, int k, int K,
                                         unsigned packed) {
  const size_t off = ref_layout ? a8_offset(r, k, K) : (size_t)r * K + k;
  *(unsigned*)(out + off) = packed;
}
__device__ __forceinline__ unsigned q_pack4(const float (&v)[4], float s) {
  unsigned p = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) p |= ((unsigned)q_one(v[j], s) & 0xFFu) << (8 * j);
  return p;
}

// Row scales: one workgroup (kQRowWaves waves) per (row, part). x f16 [M][K] (+ part * part_stride). In the A8
// layout (M = 256) XCD x (workgroups are dealt to the 8 XCDs in turn) takes rows 32 x .. 32 x + 31, so the 8-byte
// pieces of one 256-byte A8 block (16 rows) are all written through one L2.
constexpr int kQRowWaves = 16;
__global__ __launch_bounds__(64 * kQRowWaves) void q_row_kernel(const unsigned short* __restrict__ x,
                                                                signed char* __restrict__ a8, float* __restrict__ sa,
                                                                int M, int K, long long part_stride, int ref_layout) {
  __shared__ float red[kQRowWaves];
  const int row = ref_layout ? 32 * (blockIdx.x & 7) + (blockIdx.x >> 3) : blockIdx.x, part = blockIdx.y;
  const unsigned short* xr = x + part * part_stride + (size_t)row * K;
  float amax = 0.f;
  for (int k = threadIdx.x * 4; k < K; k += 4 * 64 * kQRowWaves) {
    const r4u2 raw = *(const r4u2*)(xr + k);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      amax = __builtin_fmaxf(amax, __builtin_fabsf(r4_f16_to_f32((unsigned short)((j < 2 ? raw[0] : raw[1]) >> (16 * (j & 1))))));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) amax = __builtin_fmaxf(amax, __shfl_xor(amax, o, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int i = 1; i < kQRowWaves; ++i) m = __builtin_fmaxf(m, red[i]);
  const float s = q_scale(m);
  if (threadIdx.x == 0) sa[(size_t)part * M + row] = s;
  signed char* out = a8 + (size_t)part * M * K;
  for (int k = threadIdx.x * 4; k < K; k += 4 * 64 * kQRowWaves) {
    const r4u2 raw = *(const r4u2*)(xr + k);
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = r4_f16_to_f32((unsigned short)((j < 2 ? raw[0] : raw[1]) >> (16 * (j & 1))));
    q_store4(out, ref_layout, row, k, K, q_pack4(v, s));
  }
}

// Per-(row, 128) scales: one wave per (row, block); lane l takes k = 128 b + 2 l, 2 l + 1. sa [K/128][M]. In the
// A8 layout (M = 256) XCD x takes rows 32 x .. 32 x + 31, as in q_row_kernel.
__global__ __launch_bounds__(256) void q_blk_kernel(const unsigned short* __restrict__ x, signed char* __restrict__ a8,
                                                    float* __restrict__ sa, int M, int K, long long part_stride,
                                                    int ref_layout) {
  const int lane = threadIdx.x & 63;
  const int nkb = K >> 7;
  int row, kb;
  if (ref_layout) {
    const long long j = (long long)(blockIdx.x >> 3) * 4 + (threadIdx.x >> 6);
    if (j >= 32LL * nkb) return;
    row = 32 * (int)(blockIdx.x & 7) + (int)(j & 31);
    kb = (int)(j >> 5);
  } else {
    const long long id = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (id >= (long long)M * nkb) return;
    row = (int)(id / nkb);
    kb = (int)(id % nkb);
  }
  const int part = blockIdx.y;
  const unsigned short* xr = x + part * part_stride + (size_t)row * K + kb * 128;
  const unsigned raw = *(const unsigned*)(xr + 2 * lane);
  const float v0 = r4_f16_to_f32((unsigned short)(raw & 0xFFFFu)), v1 = r4_f16_to_f32((unsigned short)(raw >> 16));
  float amax = __builtin_fmaxf(__builtin_fabsf(v0), __builtin_fabsf(v1));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) amax = __builtin_fmaxf(amax, __shfl_xor(amax, o, 64));
  const float s = q_scale(amax);
  if (lane == 0) sa[((size_t)part * nkb + kb) * M + row] = s;
  // pairs of lanes hold four consecutive k: lane 2i carries them
  const unsigned q01 = ((unsigned)q_one(v0, s) & 0xFFu) | (((unsigned)q_one(v1, s) & 0xFFu) << 8);
  const unsigned q23 = (unsigned)__shfl_xor((int)q01, 1, 64);
  if ((lane & 1) == 0) q_store4(a8 + (size_t)part * M * K, ref_layout, row, kb * 128 + 2 * lane, K, q01 | (q23 << 16));
}

// ---- the input transform fused with the quantizers (kernels.h:149-179) --------------------------------------
// The transform's f16 A (r4dx_trellis_input_bf16's arithmetic: f16(FWHT128(fp32(x) * suh) * scale)) is not
// stored; each (row, 128-block) goes through the quantizers above, byte for byte what r4d_trellis_i8_quant_act(_row)
// makes from the stored A. x is bf16 [256][K]; output o gets suh[o], a8[o] (A8 layout) and sa[o].
constexpr int kXqMaxOut = 3;
struct XqOut {
  const float* suh[kXqMaxOut];
  signed char* a8[kXqMaxOut];
  float* sa[kXqMaxOut];
};
// the transformed block of (row, k0) for output o: lane l gets the f16 bits of elements l and l + 64
// (s0, s1: suh of elements l and l + 64)
__device__ __forceinline__ void xq_transform_s(float x0, float x1, float s0, float s1, int lane, float scale,
                                               unsigned short& h0, unsigned short& h1) {
  float v0 = x0 * s0;
  float v1 = x1 * s1;
  r4_fwht128_wave(v0, v1, lane);
  h0 = r4_f16_rn(v0 * scale);
  h1 = r4_f16_rn(v1 * scale);
}

// per-(row, 128) scales: one wave per (row, kXqBlkU consecutive blocks), every load of its blocks issued before
// the first transform (a block past the row re-reads the last one and is dropped); each block goes through a
// wave-private LDS slot to reach q_blk_kernel's lane map (lane l: k = 2 l, 2 l + 1)
constexpr int kXqBlkU = 4;
template <int SRC>
__global__ __launch_bounds__(256) void xq_blk_kernel(R4XSrc src, int K, int nout, XqOut p, float scale) {
  __shared__ unsigned short buf[4][128];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int nkb = K >> 7, ngr = (nkb + kXqBlkU - 1) / kXqBlkU;
  // workgroups are dealt to the 8 XCDs in turn: XCD x takes rows 32 x .. 32 x + 31 (two 16-row tiles of the A8
  // layout), so the 8-byte pieces of one 256-byte A8 block are all written through one L2
  const int xcd = blockIdx.x & 7;
  const long long j = (long long)(blockIdx.x >> 3) * 4 + w;
  if (j >= 32LL * ngr) return;
  const int row = 32 * xcd + (int)(j & 31), kbase = (int)(j >> 5) * kXqBlkU;
  float x0[kXqBlkU], x1[kXqBlkU];
  size_t k0[kXqBlkU];
#pragma unroll
  for (int u = 0; u < kXqBlkU; ++u) {
    k0[u] = (size_t)min(kbase + u, nkb - 1) * 128;
    x0[u] = r4_xsrc<SRC, true>(src, row, (long long)k0[u] + lane);
    x1[u] = r4_xsrc<SRC, true>(src, row, (long long)k0[u] + lane + 64);
  }
  for (int o = 0; o < nout; ++o) {
    float s0[kXqBlkU], s1[kXqBlkU];
#pragma unroll
    for (int u = 0; u < kXqBlkU; ++u) {
      s0[u] = p.suh[o][k0[u] + lane];
      s1[u] = p.suh[o][k0[u] + 64 + lane];
    }
#pragma unroll
    for (int u = 0; u < kXqBlkU; ++u) {
      if (kbase + u >= nkb) break;
      unsigned short h0, h1;
      xq_transform_s(x0[u], x1[u], s0[u], s1[u], lane, scale, h0, h1);
      buf[w][lane] = h0;
      buf[w][lane + 64] = h1;
      // the wave reads what other lanes wrote: keep the read after the writes (and the next block's writes
      // after this read) -- without the clobber the compiler hoists the read above the stores
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      const unsigned raw = *(const unsigned*)&buf[w][2 * lane];
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      const float v0 = r4_f16_to_f32((unsigned short)(raw & 0xFFFFu)), v1 = r4_f16_to_f32((unsigned short)(raw >> 16));
      float amax = __builtin_fmaxf(__builtin_fabsf(v0), __builtin_fabsf(v1));
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) amax = __builtin_fmaxf(amax, __shfl_xor(amax, m, 64));
      const float sc = q_scale(amax);
      const int kb = kbase + u;
      if (lane == 0) p.sa[o][(size_t)kb * 256 + row] = sc;
      const unsigned q01 = ((unsigned)q_one(v0, sc) & 0xFFu) | (((unsigned)q_one(v1, sc) & 0xFFu) << 8);
      const unsigned q23 = (unsigned)__shfl_xor((int)q01, 1, 64);
      if ((lane & 1) == 0) q_store4(p.a8[o], true, row, (int)k0[u] + 2 * lane, K, q01 | (q23 << 16));
    }
  }
}

// one scale per row: a workgroup (kXqRowWaves waves) per row transforms every block into LDS (f16, [nout][K]),
// takes the row's amax, then quantizes like q_row_kernel. 16 waves per row: with 4 (one per SIMD) each wave walked
// its blocks one memory round trip at a time (K 17408: 26 us per launch)
constexpr int kXqRowWaves = 16;
template <int SRC>
__global__ __launch_bounds__(64 * kXqRowWaves) void xq_row_kernel(R4XSrc src, int K, int nout, XqOut p, float scale) {
  extern __shared__ unsigned short rowbuf[];
  __shared__ float red[kXqMaxOut][kXqRowWaves];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // XCD x (workgroups are dealt to the 8 XCDs in turn) takes rows 32 x .. 32 x + 31: the 8-byte pieces of one
  // 256-byte A8 block (16 rows) are then all written through one L2
  const int row = 32 * (blockIdx.x & 7) + (blockIdx.x >> 3), nkb = K >> 7;
  float amax[kXqMaxOut] = {0.f, 0.f, 0.f};
  // kXqRowU blocks per pass, all their loads issued first (a block past the row re-reads the last one and is
  // dropped), so a wave waits for one memory round trip per pass instead of one per block
  constexpr int kXqRowU = 3;
  for (int kb = w; kb < nkb; kb += kXqRowU * kXqRowWaves) {
    float x0[kXqRowU], x1[kXqRowU];
    size_t k0[kXqRowU];
#pragma unroll
    for (int u = 0; u < kXqRowU; ++u) {
      const int b = min(kb + u * kXqRowWaves, nkb - 1);
      k0[u] = (size_t)b * 128;
      x0[u] = r4_xsrc<SRC, true>(src, row, (long long)k0[u] + lane);
      x1[u] = r4_xsrc<SRC, true>(src, row, (long long)k0[u] + lane + 64);
    }
#pragma unroll
    for (int o = 0; o < kXqMaxOut; ++o) {
      if (o >= nout) break;
      float s0[kXqRowU], s1[kXqRowU];
#pragma unroll
      for (int u = 0; u < kXqRowU; ++u) {
        s0[u] = p.suh[o][k0[u] + lane];
        s1[u] = p.suh[o][k0[u] + 64 + lane];
      }
#pragma unroll
      for (int u = 0; u < kXqRowU; ++u) {
        unsigned short h0, h1;
        xq_transform_s(x0[u], x1[u], s0[u], s1[u], lane, scale, h0, h1);
        if (kb + u * kXqRowWaves < nkb) {
          rowbuf[(size_t)o * K + k0[u] + lane] = h0;
          rowbuf[(size_t)o * K + k0[u] + lane + 64] = h1;
          amax[o] = __builtin_fmaxf(amax[o], __builtin_fmaxf(__builtin_fabsf(r4_f16_to_f32(h0)),
                                                             __builtin_fabsf(r4_f16_to_f32(h1))));
        }
      }
    }
  }
#pragma unroll
  for (int o = 0; o < kXqMaxOut; ++o) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) amax[o] = __builtin_fmaxf(amax[o], __shfl_xor(amax[o], m, 64));
    if (lane == 0) red[o][w] = amax[o];
  }
  __syncthreads();
  for (int o = 0; o < nout; ++o) {
    float m = red[o][0];
#pragma unroll
    for (int i = 1; i < kXqRowWaves; ++i) m = __builtin_fmaxf(m, red[o][i]);
    const float s = q_scale(m);
    if (threadIdx.x == 0) p.sa[o][row] = s;
    for (int k = threadIdx.x * 4; k < K; k += 4 * 64 * kXqRowWaves) {
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = r4_f16_to_f32(rowbuf[(size_t)o * K + k + j]);
      q_store4(p.a8[o], true, row, k, K, q_pack4(v, s));
    }
  }
}

template <int SRC>
void xq_launch(bool row_scale, const R4XSrc& src, int64_t K, int nout, const XqOut& p, float scale, int64_t stream,
               const char* entry) {
  hipStream_t st = (hipStream_t)stream;
  if (row_scale) {
    const size_t lds = (size_t)nout * K * 2;
    // the row's values plus the kernel's 192 static bytes must fit the 160 KiB of a workgroup
    if (lds > 160 * 1024 - 256) r4d::fail(entry, "nout K 2 bytes must stay below 160 KiB of LDS");
    static std::atomic<unsigned long long> lds_set{0};
    if (lds > 64 * 1024) r4d::allow_lds((const void*)xq_row_kernel<SRC>, lds_set, entry);
    hipLaunchKernelGGL((xq_row_kernel<SRC>), dim3(256), dim3(64 * kXqRowWaves), lds, st, src, (int)K, nout, p, scale);
  } else {
    const long long waves = 256LL * ((K / 128 + kXqBlkU - 1) / kXqBlkU);
    hipLaunchKernelGGL((xq_blk_kernel<SRC>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, src, (int)K, nout,
                       p, scale);
  }
  r4d::launch_ok(entry);
}

// float(2^s / sqrt(128)), rounded once from double (trellis_ref.hpp:146-148)
float xq_scale(int prescale_log2, const char* entry) {
  if (prescale_log2 < -24 || prescale_log2 > 24) r4d::fail(entry, "|prescale_log2| must be <= 24");
  return (float)(__builtin_ldexp(1.0, prescale_log2) / __builtin_sqrt(128.0));
}

void xq_run(bool row_scale, int64_t x, int64_t M, int64_t K, int nout, const int64_t* suh, const int64_t* a8,
            const int64_t* sa, int prescale_log2, int64_t stream, const char* entry) {
  if (M != 256) r4d::fail(entry, "M must be 256 (the A8 layout's rows)");
  if (K <= 0 || K % 128) r4d::fail(entry, "K must be a positive multiple of 128");
  if (nout < 1 || nout > kXqMaxOut) r4d::fail(entry, "nout must be 1..3");
  const float scale = xq_scale(prescale_log2, entry);
  if (!x || !suh || !a8 || !sa) r4d::fail(entry, "null pointer");
  XqOut p{};
  for (int o = 0; o < nout; ++o) {
    if (!suh[o] || !a8[o] || !sa[o]) r4d::fail(entry, "null suh, a8 or sa");
    p.suh[o] = (const float*)suh[o];
    p.a8[o] = (signed char*)a8[o];
    p.sa[o] = (float*)sa[o];
  }
  xq_launch<R4_SRC_X>(row_scale, R4XSrc{(const unsigned short*)x, nullptr, (long long)K, 0}, K, nout, p, scale, stream,
                      entry);
}

// The fused producers' int8 forms (trellis_transform.hip:971-1000, 1038-1070): the producers' preconditions
// (K a positive multiple of 128, |prescale_log2| <= 24, non-null suh) plus rows == 256 and non-null a8 and sa.
void xq_producer(bool row_scale, int SRC, const R4XSrc& src, int64_t rows, int64_t K, int64_t suh, int64_t a8,
                 int64_t sa, int prescale_log2, int64_t stream, const char* entry) {
  if (K <= 0 || K % 128) r4d::fail(entry, "K must be a positive multiple of 128");
  const float scale = xq_scale(prescale_log2, entry);
  if (!suh) r4d::fail(entry, "suh must be non-null");
  if (rows != 256) r4d::fail(entry, "rows must be 256 (the int8 A8 layout)");
  if (!a8 || !sa) r4d::fail(entry, "a8 and sa must be non-null");
  XqOut p{};
  p.suh[0] = (const float*)suh;
  p.a8[0] = (signed char*)a8;
  p.sa[0] = (float*)sa;
  if (SRC == R4_SRC_SILU) xq_launch<R4_SRC_SILU>(row_scale, src, K, 1, p, scale, stream, entry);
  else xq_launch<R4_SRC_GATE>(row_scale, src, K, 1, p, scale, stream, entry);
}

// plain int8 [N][K] -> the W8 block layout (r4d_trellis_i8_layout.h:24-27): one thread per output
// dword, which is four consecutive k of one column
__global__ __launch_bounds__(256) void w8_pack_kernel(const signed char* __restrict__ wp, unsigned* __restrict__ w8,
                                                      int N, int K) {
  const long long d = (long long)blockIdx.x * 256 + threadIdx.x;
  if (d >= (long long)N * K / 4) return;
  const long long byte = d * 4;
  const int KT = K >> 4;
  const long long blk = byte >> 9;
  const int pair = (int)(blk / KT), kt = (int)(blk % KT);
  const int in = (int)(byte & 511), L = in >> 4, Fq = (in >> 3) & 1, eh = (in >> 2) & 1;
  const int n = 32 * pair + 16 * ((L >> 3) & 1) + 8 * Fq + (L & 7);
  const int k = 16 * kt + 8 * eh + 4 * (L >> 4);
  w8[d] = *(const unsigned*)(wp + (size_t)n * K + k);
}

void quant_run(bool blk, int64_t x, int64_t a8, int64_t sa, int parts, int64_t part_stride, int M, int K,
               bool ref_layout, int64_t stream, const char* entry) {
  if (K <= 0 || K % 128) r4d::fail(entry, "K must be a positive multiple of 128");
  if (parts != 1 && parts != 2) r4d::fail(entry, "parts must be 1 or 2");
  if (parts == 2 && part_stride < (int64_t)M * K) r4d::fail(entry, "part_stride must be >= M K for two parts");
  if (ref_layout && M != 256) r4d::fail(entry, "the A8 layout is for M = 256");
  if (M < 1) r4d::fail(entry, "M must be >= 1");
  if (!x || !a8 || !sa) r4d::fail(entry, "null buffer");
  hipStream_t st = (hipStream_t)stream;
  if (blk) {
    const long long waves = (long long)M * (K / 128);
    hipLaunchKernelGGL(q_blk_kernel, dim3((unsigned)((waves + 3) / 4), (unsigned)parts), dim3(256), 0, st,
                       (const unsigned short*)x, (signed char*)a8, (float*)sa, M, K, (long long)part_stride,
                       ref_layout ? 1 : 0);
  } else {
    hipLaunchKernelGGL(q_row_kernel, dim3((unsigned)M, (unsigned)parts), dim3(64 * kQRowWaves), 0, st, (const unsigned short*)x,
                       (signed char*)a8, (float*)sa, M, K, (long long)part_stride, ref_layout ? 1 : 0);
  }
  r4d::launch_ok(entry);
}

}  // namespace

extern "C" {

// r4d.h:490-491 r4d_trellis_i8_quant_act: per-(row, 128) scales, A8 layout, SA [K/128][256] per part.
void r4d_trellis_i8_quant_act(int64_t x, int64_t a8, int64_t sa, int parts, int64_t part_stride, int K, int64_t stream) {
  quant_run(true, x, a8, sa, parts, part_stride, 256, K, true, stream, "trellis_i8_quant_act");
}
// r4d.h:517-518 r4d_trellis_i8_quant_act_row: one scale per row, A8 layout, SA [256] per part.
void r4d_trellis_i8_quant_act_row(int64_t x, int64_t a8, int64_t sa, int parts, int64_t part_stride, int K,
                                  int64_t stream) {
  quant_run(false, x, a8, sa, parts, part_stride, 256, K, true, stream, "trellis_i8_quant_act_row");
}
// This build's plain-layout quantizers (any M): a8 [M][K] row-major; blk: sa [K/128][M], else sa [M].
void r4d_i8_quant_act_plain(int64_t x, int64_t a8, int64_t sa, int M, int K, int blk, int64_t stream) {
  quant_run(blk != 0, x, a8, sa, 1, 0, M, K, false, stream, "i8_quant_act_plain");
}

// kernels.h:160-161: the input transform fused with the per-(row, 128) quantizer
void r4dx_trellis_input_i8(int64_t x, int64_t M, int64_t K, int nout, const int64_t* suh, const int64_t* a8,
                           const int64_t* sa, int prescale_log2, int64_t stream) {
  xq_run(false, x, M, K, nout, suh, a8, sa, prescale_log2, stream, "trellis_input_i8");
}
// kernels.h:174-175: ... with one scale per row
void r4dx_trellis_input_i8r(int64_t x, int64_t M, int64_t K, int nout, const int64_t* suh, const int64_t* a8,
                            const int64_t* sa, int prescale_log2, int64_t stream) {
  xq_run(true, x, M, K, nout, suh, a8, sa, prescale_log2, stream, "trellis_input_i8r");
}

// kernels.h:149-163, 167-177: r4dx_silu_mul_trellis_bf16's producer and transform, quantized like
// r4dx_trellis_input_i8 (per (row, 128) scales) / _i8r (one scale per row); rows must be 256.
void r4dx_silu_mul_trellis_i8(int64_t gate_up, int64_t rows, int64_t intermediate, int64_t in_row_stride, int64_t suh,
                              int64_t a8, int64_t sa, int prescale_log2, int64_t stream) {
  const char* e = "silu_mul_trellis_i8";
  if (!gate_up) r4d::fail(e, "gate_up is null");
  if (in_row_stride < 2 * intermediate) r4d::fail(e, "in_row_stride must be >= 2 * intermediate");
  xq_producer(false, R4_SRC_SILU, R4XSrc{(const unsigned short*)gate_up, nullptr, (long long)in_row_stride,
                                          (long long)intermediate},
              rows, intermediate, suh, a8, sa, prescale_log2, stream, e);
}
void r4dx_silu_mul_trellis_i8r(int64_t gate_up, int64_t rows, int64_t intermediate, int64_t in_row_stride,
                               int64_t suh, int64_t a8, int64_t sa, int prescale_log2, int64_t stream) {
  const char* e = "silu_mul_trellis_i8r";
  if (!gate_up) r4d::fail(e, "gate_up is null");
  if (in_row_stride < 2 * intermediate) r4d::fail(e, "in_row_stride must be >= 2 * intermediate");
  xq_producer(true, R4_SRC_SILU, R4XSrc{(const unsigned short*)gate_up, nullptr, (long long)in_row_stride,
                                         (long long)intermediate},
              rows, intermediate, suh, a8, sa, prescale_log2, stream, e);
}
// kernels.h:164-165, 178-179: the same for r4dx_attn_gate_mul_trellis_bf16's producer.
void r4dx_attn_gate_mul_trellis_i8(int64_t attn_out, int64_t gate, int64_t rows, int64_t K, int64_t suh, int64_t a8,
                                   int64_t sa, int prescale_log2, int64_t stream) {
  const char* e = "attn_gate_mul_trellis_i8";
  if (!attn_out || !gate) r4d::fail(e, "attn_out and gate must be non-null");
  xq_producer(false, R4_SRC_GATE, R4XSrc{(const unsigned short*)attn_out, (const unsigned short*)gate, (long long)K, 0},
              rows, K, suh, a8, sa, prescale_log2, stream, e);
}
void r4dx_attn_gate_mul_trellis_i8r(int64_t attn_out, int64_t gate, int64_t rows, int64_t K, int64_t suh, int64_t a8,
                                    int64_t sa, int prescale_log2, int64_t stream) {
  const char* e = "attn_gate_mul_trellis_i8r";
  if (!attn_out || !gate) r4d::fail(e, "attn_out and gate must be non-null");
  xq_producer(true, R4_SRC_GATE, R4XSrc{(const unsigned short*)attn_out, (const unsigned short*)gate, (long long)K, 0},
              rows, K, suh, a8, sa, prescale_log2, stream, e);
}
// plain int8 [N][K] -> W8 block layout (N K bytes), once per weight
void r4d_i8_pack_w(int64_t wp, int64_t w8, int N, int K, int64_t stream) {
  if (N <= 0 || K <= 0 || N % 32 || K % 16) r4d::fail("i8_pack_w", "N must be a multiple of 32 and K of 16");
  if (!wp || !w8) r4d::fail("i8_pack_w", "null buffer");
  const long long n = (long long)N * K / 4;
  hipLaunchKernelGGL(w8_pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const signed char*)wp, (unsigned*)w8, N, K);
  r4d::launch_ok("i8_pack_w");
}
}  // extern "C"
