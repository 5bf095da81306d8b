// int8.hip -- the int8 x int8 prefill GEMM with its activation quantizers on gfx950.
//
// Quantizers (the reference's arithmetic: tests/kernels/int8_gemm_proto_ref.h:84-89,138-189,
// third_party/libr4d/r4d_trellis_i8.h:160-208): s = amax / 127 (1 for an all-zero group), q = clamp(
// rint(x / s), -127, 127) with IEEE fp32 division, amax over a row (coarse) or over each (row, 128 k)
// block. They write the reference's A8 fragment layout (r4d_trellis_i8_layout.h:32-45, what
// r4d_trellis_i8_quant_act / _row produce) or a plain [M][K] layout.
//
// The dense GEMM (plain int8 weights W8 [N][K] with an fp32 scale per output
// column, activations quantized per row or per (row, 128)): C[m][n] = f16(acc), acc = sa[m] * sw[n] *
// int32(A8 . W8) (row scales) or sw[n] * sum_kb sa[kb][m] * int32_kb (per-128 activation scales), the
// int32 sums exact. This build's entries; the reference has the dense form only as a bench kernel
// (r4d_trellis_i8.h:19-20, i8g_kernel<TRELLIS = false>).
//
// DESIGN (MI355X): v_mfma_i32_16x16x64_i8. A workgroup is 8 waves = 256 rows x 128 columns x one K
// slice; wave w owns rows 32 w .. 32 w + 31 (2 row tiles) x the 8 column tiles. Each wave keeps a
// 4-step register ring of its column tile of W8 (16 columns x 64 bytes per step) and its two row tiles
// of A8; per step it stores its column tile into a double-buffered LDS slot, one barrier, and every
// wave runs 2 x 8 MFMAs against the 8 tiles. Split K: each slice's exact int32 sums
// (row scales) or fp32 partial sums (per-128) go to ws and a second launch adds the slices in order
// and applies the scales and the f16 rounding.
#include "r4d_dev.h"
#include "r4d_host.h"
#include "r4d_mi355x.h"

namespace {

typedef __amdgpu_buffer_rsrc_t r4_rsrc;
__device__ __forceinline__ r4_rsrc mk_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)bytes, 0x00020000);
}

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

// Row scales: one workgroup (256 threads) per (row, part). x f16 [M][K] (+ part * part_stride).
__global__ __launch_bounds__(256) void q_row_kernel(const unsigned short* __restrict__ x, signed char* __restrict__ a8,
                                                    float* __restrict__ sa, int M, int K, long long part_stride,
                                                    int ref_layout) {
  __shared__ float red[4];
  const int row = blockIdx.x, part = blockIdx.y;
  const unsigned short* xr = x + part * part_stride + (size_t)row * K;
  float amax = 0.f;
  for (int k = threadIdx.x * 4; k < K; k += 1024) {
    const r4u2 raw = *(const r4u2*)(xr + k);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      amax = __builtin_fmaxf(amax, __builtin_fabsf(r4_f16_to_f32((unsigned short)((j < 2 ? raw[0] : raw[1]) >> (16 * (j & 1))))));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) amax = __builtin_fmaxf(amax, __shfl_xor(amax, o, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  const float s = q_scale(__builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3])));
  if (threadIdx.x == 0) sa[(size_t)part * M + row] = s;
  signed char* out = a8 + (size_t)part * M * K;
  for (int k = threadIdx.x * 4; k < K; k += 1024) {
    const r4u2 raw = *(const r4u2*)(xr + k);
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = r4_f16_to_f32((unsigned short)((j < 2 ? raw[0] : raw[1]) >> (16 * (j & 1))));
    q_store4(out, ref_layout, row, k, K, q_pack4(v, s));
  }
}

// Per-(row, 128) scales: one wave per (row, block); lane l takes k = 128 b + 2 l, 2 l + 1. sa [K/128][M].
__global__ __launch_bounds__(256) void q_blk_kernel(const unsigned short* __restrict__ x, signed char* __restrict__ a8,
                                                    float* __restrict__ sa, int M, int K, long long part_stride,
                                                    int ref_layout) {
  const int lane = threadIdx.x & 63;
  const int nkb = K >> 7;
  const long long id = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (id >= (long long)M * nkb) return;
  const int row = (int)(id / nkb), kb = (int)(id % nkb), part = blockIdx.y;
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

// ---- dense int8 GEMM ----------------------------------------------------------------------------------
constexpr int kI8Waves = 8;

__device__ __forceinline__ r4i4 mfma_i8(r4i4 a, r4i4 b, r4i4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// SCALE_BLK: activation scales per (row, 128) [K/128][M], else per row [M]. OUT: 0 = f16 C (finished),
// 1 = int32 partial sums to ws (row scales), 2 = fp32 partial sums to ws (per-128 scales).
template <bool SCALE_BLK>
__global__ __launch_bounds__(64 * kI8Waves, 1) void i8_dense_kernel(
    const signed char* __restrict__ A8, const float* __restrict__ SA, const signed char* __restrict__ W8,
    const float* __restrict__ SW, void* __restrict__ Cv, void* __restrict__ ws, int M, int K, int N, int SKG,
    int out_mode) {
  __shared__ r4i4 bsh[2][8][64];                 // [buffer][column tile][lane]: 8 KiB per buffer
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * 128, ky = blockIdx.y;
  const int kslice = K / SKG, k0 = ky * kslice, nst = kslice >> 6;
  const int m16 = lane & 15, g = lane >> 4;

  // B: wave w loads column tile w: lane l -> W8[n0 + 16 w + (l & 15)][k + 16 (l >> 4) .. + 16]
  const r4_rsrc br = mk_rsrc(W8, (unsigned)((size_t)N * K));
  const unsigned boff = (unsigned)((size_t)(n0 + 16 * wave + m16) * K + k0 + 16 * g);
  // A: rows 32 w + 16 i + (l & 15), the lane's 16 bytes of the step's k-tile g
  const r4_rsrc ar = mk_rsrc(A8, (unsigned)((size_t)M * K));
  unsigned aoff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) aoff[i] = (unsigned)((size_t)(32 * wave + 16 * i + m16) * K + k0 + 16 * g);

  struct St {
    r4i4 b;
    r4i4 a[2];
  };
  // step st (clamped: a prefetch past the end re-reads the last step, a cached line)
  auto load = [&](St& s, int st) {
    const unsigned so = (unsigned)min(st, nst - 1) * 64u;
    s.b = __builtin_bit_cast(r4i4, __builtin_amdgcn_raw_buffer_load_b128(br, boff + so, 0, 0));
#pragma unroll
    for (int i = 0; i < 2; ++i)
      s.a[i] = __builtin_bit_cast(r4i4, __builtin_amdgcn_raw_buffer_load_b128(ar, aoff[i] + so, 0, 0));
  };

  r4i4 iacc[2][8];
  r4f4 facc[2][8];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      iacc[i][c] = (r4i4){0, 0, 0, 0};
      facc[i][c] = (r4f4){0.f, 0.f, 0.f, 0.f};
    }
  // lane's output rows (C layout of 16x16: column l & 15, rows 4 (l >> 4) + j)
  auto row_of = [&](int i, int j) { return 32 * wave + 16 * i + 4 * g + j; };

  auto step = [&](const St& s, int st) {
    const int buf = st & 1;
    bsh[buf][wave][lane] = s.b;
    // LDS stores of every wave done before anyone reads (a bare s_barrier keeps the prefetches in flight)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    r4i4 b[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) b[c] = bsh[buf][c][lane];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      iacc[0][c] = mfma_i8(s.a[0], b[c], iacc[0][c]);
      iacc[1][c] = mfma_i8(s.a[1], b[c], iacc[1][c]);
    }
    if constexpr (SCALE_BLK) {
      if ((st & 1) == 1) {   // a 128-k block is complete: facc += float(int32) * sa[kb][row]
        const int kb = (k0 >> 7) + (st >> 1);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float sv = SA[(size_t)kb * M + row_of(i, j)];
#pragma unroll
            for (int c = 0; c < 8; ++c) {
              facc[i][c][j] = __builtin_fmaf((float)iacc[i][c][j], sv, facc[i][c][j]);
              iacc[i][c][j] = 0;
            }
          }
      }
    }
  };

  // A statically indexed ring: slot i is reloaded right after its step, so at its next use it is the
  // oldest load in flight.
  constexpr int PF = 4;
  St ring[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) load(ring[i], i);
  int st = 0;
  for (; st + PF <= nst; st += PF) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      step(ring[i], st + i);
      load(ring[i], st + i + PF);
    }
  }
#pragma unroll
  for (int i = 0; i < PF - 1; ++i)
    if (st + i < nst) step(ring[i], st + i);

  // output: column n0 + 16 c + (l & 15), rows row_of(i, j)
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = row_of(i, j);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int n = n0 + 16 * c + m16;
        if (out_mode == 1) ((int*)ws)[((size_t)ky * M + r) * N + n] = iacc[i][c][j];
        else if (out_mode == 2) ((float*)ws)[((size_t)ky * M + r) * N + n] = facc[i][c][j];
        else {
          const float v = SCALE_BLK ? facc[i][c][j] * SW[n] : (float)iacc[i][c][j] * (SA[r] * SW[n]);
          ((unsigned short*)Cv)[(size_t)r * N + n] = __builtin_bit_cast(unsigned short, (_Float16)v);
        }
      }
    }
}

// Second pass of a split launch: slices added in order (int32 exactly, or fp32 in slice order), then
// the scales and the f16 rounding; raw_i32 stores the int32 sums instead.
__global__ __launch_bounds__(256) void i8_finish_kernel(const void* __restrict__ ws, const float* __restrict__ SA,
                                                        const float* __restrict__ SW, void* __restrict__ Cv, int M,
                                                        int N, int SKG, int scale_blk, int raw_i32) {
  const long long id = (long long)blockIdx.x * 256 + threadIdx.x;
  if (id >= (long long)M * N) return;
  const int r = (int)(id / N), n = (int)(id % N);
  const size_t sy = (size_t)M * N;
  if (!scale_blk) {
    int acc = 0;
    for (int y = 0; y < SKG; ++y) acc += ((const int*)ws)[y * sy + id];
    if (raw_i32) { ((int*)Cv)[id] = acc; return; }
    const float v = (float)acc * (SA[r] * SW[n]);
    ((unsigned short*)Cv)[id] = __builtin_bit_cast(unsigned short, (_Float16)v);
  } else {
    float acc = ((const float*)ws)[id];
    for (int y = 1; y < SKG; ++y) acc += ((const float*)ws)[y * sy + id];
    const float v = acc * SW[n];
    ((unsigned short*)Cv)[id] = __builtin_bit_cast(unsigned short, (_Float16)v);
  }
}

std::string i8_check(int M, int K, int N, int SKG) {
  if (M != 256) return "M must be 256 (the prefill chunk)";
  if (K <= 0 || N <= 0 || K % 128 || N % 128) return "K and N must be positive multiples of 128";
  if (SKG < 1 || SKG > 64 || K % (128 * SKG)) return "SKG must be 1..64 with K divisible by 128 SKG";
  return "";
}

void i8_run(int64_t a8, int64_t sa, int64_t w8, int64_t sw, int64_t c, int64_t ws, int M, int K, int N, int SKG,
            bool scale_blk, bool raw_i32, int64_t stream, const char* entry) {
  r4d::require(entry, i8_check(M, K, N, SKG));
  if (!a8 || !w8 || !c || (!raw_i32 && (!sa || !sw))) r4d::fail(entry, "null buffer");
  const bool split = SKG > 1 || raw_i32;
  if (split && !ws) r4d::fail(entry, "a split (SKG > 1) or raw launch needs ws");
  hipStream_t st = (hipStream_t)stream;
  dim3 grid(N / 128, SKG), block(64 * kI8Waves);
  const int mode = split ? (scale_blk ? 2 : 1) : 0;
  if (scale_blk)
    hipLaunchKernelGGL(i8_dense_kernel<true>, grid, block, 0, st, (const signed char*)a8, (const float*)sa,
                       (const signed char*)w8, (const float*)sw, (void*)c, (void*)ws, M, K, N, SKG, mode);
  else
    hipLaunchKernelGGL(i8_dense_kernel<false>, grid, block, 0, st, (const signed char*)a8, (const float*)sa,
                       (const signed char*)w8, (const float*)sw, (void*)c, (void*)ws, M, K, N, SKG, mode);
  if (split) {
    const long long n = (long long)M * N;
    hipLaunchKernelGGL(i8_finish_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, (const void*)ws,
                       (const float*)sa, (const float*)sw, (void*)c, M, N, SKG, scale_blk ? 1 : 0, raw_i32 ? 1 : 0);
  }
  r4d::launch_ok(entry);
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
    hipLaunchKernelGGL(q_row_kernel, dim3((unsigned)M, (unsigned)parts), dim3(256), 0, st, (const unsigned short*)x,
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
// This build's plain-layout quantizers (the dense GEMM's A): a8 [M][K] row-major; blk: sa [K/128][M],
// else sa [M].
void r4d_i8_quant_act_plain(int64_t x, int64_t a8, int64_t sa, int M, int K, int blk, int64_t stream) {
  quant_run(blk != 0, x, a8, sa, 1, 0, M, K, false, stream, "i8_quant_act_plain");
}

const char* r4d_gemm_i8_dense_check(int M, int K, int N, int SKG) { return r4d::check_result(i8_check(M, K, N, SKG)); }
size_t r4d_gemm_i8_dense_ws_bytes(int M, int N, int SKG) { return (size_t)SKG * M * N * 4; }

// The dense int8 GEMM: a8 plain [256][K] (r4d_i8_quant_act_plain), w8 plain [N][K], sw [N] fp32; scale_blk
// selects sa [K/128][256] (per-128 activation scales) over sa [256] (row scales). C f16 [256][N]. ws fp32/int32
// ws_bytes(M, N, SKG) when SKG > 1.
void r4d_gemm_i8_dense(int64_t a8, int64_t sa, int64_t w8, int64_t sw, int64_t c, int64_t ws, int M, int K, int N,
                       int SKG, int scale_blk, int64_t stream) {
  i8_run(a8, sa, w8, sw, c, ws, M, K, N, SKG, scale_blk != 0, false, stream, "gemm_i8_dense");
}
// Test entry: the exact int32 sums C[m][n] = sum_k A8[m][k] W8[n][k] (int32 [256][N]), through the same
// kernel and split (ws int32 ws_bytes(M, N, SKG)).
void r4d_gemm_i8_dense_raw(int64_t a8, int64_t w8, int64_t c, int64_t ws, int M, int K, int N, int SKG,
                           int64_t stream) {
  i8_run(a8, 0, w8, 0, c, ws, M, K, N, SKG, false, true, stream, "gemm_i8_dense_raw");
}
// This build's K split for the dense int8 GEMM: about two workgroups per CU.
int r4d_mi355x_i8_skg(int K, int N) {
  const int G = N / 128;
  int best = 1;
  for (int d = 1; d <= 16; ++d) {
    if (K % (128 * d) || K / d < 512) continue;
    best = d;
    if ((long long)G * d >= 384) break;
  }
  return best;
}

}  // extern "C"
