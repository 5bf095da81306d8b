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

// ---- the int8 GEMM ----------------------------------------------------------------------------------
// One kernel for the dense weights (W8 block layout) and, later in this file, the trellis words. A
// workgroup is 4 waves = 256 rows x 128 columns (4 pairs of 32) x one K slice. Wave w owns rows
// 64 w .. 64 w + 63 = row group w of A8 (4 row tiles) against all 8 column tiles. Per 64-k step
// (4 k-tiles) each wave
//   * reads its 4 A fragments straight from A8: 2 x 8 B per lane per fragment, 16 lanes = 128
//     contiguous bytes (v_mfma_i32_16x16x64_i8: lane l holds row l & 15 and 16 k of k-tile l >> 4;
//     the 16 bytes are the A8 halves h = 0 then h = 1, i.e. k {0-3, 8-11, 4-7, 12-15} of the tile);
//   * loads pair w's 4 W8 blocks (2 KiB contiguous) into its slot of a double-buffered LDS stage;
//   * after one barrier reads the 8 B-fragments (the same two-halves byte order, so the k order of
//     A and B agree) and runs 4 x 8 MFMAs.
// Loads run in a statically indexed 4-step register ring. Per-128 scales fold the int32 sums into
// fp32 every second step. Split K (SKG slices): the partials go to ws, the last workgroup of a
// column group (a self-resetting ticket per group, the reference's protocol, r4d.h:482-486) sums the
// slices in slice order and runs the epilogue.
constexpr int kSCoarse = 0, kSABlk = 1, kSBlk = 2;     // scale modes
constexpr int kOutF16 = 0, kOutI32 = 1, kOutBf16Fwht = 2;

struct I8Args {
  const signed char* a8[2];
  const float* sa[2];
  int n_split;
  const unsigned char* w;
  const float* sw;
  const float* svh;
  void* c;
  void* ws;
  unsigned* tickets;
  int K, N, SKG;
  float out_scale;
};

__device__ __forceinline__ r4i4 mfma_i8(r4i4 a, r4i4 b, r4i4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
// The split handoff's 16-byte accesses: buffer loads and stores with the sc1 cache policy (agent scope,
// write-through past this XCD's L2; aux bit 4), visible to the compiler's wait-count tracking.
constexpr int kSc1 = 16;
template <typename T>
__device__ __forceinline__ void st_coherent4(r4_rsrc r, unsigned off, T v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(r4u4, v), r, off, 0, kSc1);
}
template <typename T>
__device__ __forceinline__ T ld_coherent4(r4_rsrc r, unsigned off) {
  return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSc1));
}

// the W8 block layout's in-block byte offsets through LDS, with bit 7 flipped on odd k-tiles so the
// two 16-lane halves of a 64-bit read hit different banks
__device__ __forceinline__ int lds_sw(int byte) { return byte ^ (((byte >> 9) & 1) << 7); }

// The epilogue of one row tile's values (lane layout of the 16 x 16 MFMA: element j of v[pc] is row
// 16 ti + 4 (lane >> 4) + j, column 128 tile + 16 pc + 8 F + cc). T is r4i4 (exact int32 sums) or r4f4
// (scaled fp32 values). split: the values go to this slice's ws slot (16 B per lane, lane order).
template <int OUT, typename T>
__device__ __forceinline__ void i8_put(const T (&v)[8], const I8Args& p, int tile, int ky, int ti, int lane,
                                       bool split) {
  const int N = p.N, g = lane >> 4, F = (lane >> 3) & 1, cc = lane & 7;
  if (split) {
    const r4_rsrc wr = mk_rsrc(p.ws, (unsigned)p.SKG * 256u * (unsigned)N * 4u);
    const unsigned unit = (unsigned)ky * 256u * (unsigned)N * 4u + ((unsigned)tile * 16u + (unsigned)ti) * 8192u;
#pragma unroll
    for (int pc = 0; pc < 8; ++pc) st_coherent4(wr, unit + (pc * 64 + lane) * 16, v[pc]);
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 16 * ti + 4 * g + j;
#pragma unroll
    for (int pc = 0; pc < 8; ++pc) {
      const int n = 128 * tile + 16 * pc + 8 * F + cc;
      if constexpr (OUT == kOutI32)
        ((int*)p.c)[(size_t)r * N + n] = v[pc][j];
      else
        ((unsigned short*)p.c)[(size_t)r * N + n] = __builtin_bit_cast(unsigned short, (_Float16)v[pc][j]);
    }
  }
}
// The last workgroup of a split column group: each of this wave's RT row tiles from every slice's ws, added
// in slice order (as integers for T = r4i4), then stored.
template <int OUT, typename T, int RT>
__device__ __forceinline__ void i8_reduce(const I8Args& p, int tile, int ti0, int lane) {
  const unsigned N = (unsigned)p.N;
  const r4_rsrc wr = mk_rsrc(p.ws, (unsigned)p.SKG * 256u * N * 4u);
#pragma unroll 1
  for (int i = 0; i < RT; ++i) {
    T acc[8];
    for (int y = 0; y < p.SKG; ++y) {
      const unsigned unit = (unsigned)y * 256u * N * 4u + ((unsigned)tile * 16u + (unsigned)(ti0 + i)) * 8192u;
      T t8[8];
#pragma unroll
      for (int pc = 0; pc < 8; ++pc) t8[pc] = ld_coherent4<T>(wr, unit + (pc * 64 + lane) * 16);
#pragma unroll
      for (int pc = 0; pc < 8; ++pc) acc[pc] = y == 0 ? t8[pc] : acc[pc] + t8[pc];
    }
    i8_put<OUT>(acc, p, tile, 0, ti0 + i, lane, false);
  }
}

// Stage layout (bytes): A [row group 4][4 k-tiles x 1 KiB], B [pair 4][4 k-tiles x 512 B], then for the
// per-128 modes SA [256 fp32] of the step's 128-k block and SW [128 fp32] (kSBlk). Within A and B, bit 7 of
// the offset is flipped on odd k-tiles (the two 16-lane halves of a 64-bit LDS read then use different banks):
// the DMA writes lane l's 16 bytes at 16 l, so lane l fetches the global chunk that belongs there.
constexpr int kStA = 0, kStB = 16384, kStSA = 24576, kStSW = 25600;
template <int SC>
constexpr int stage_bytes() { return SC == kSCoarse ? 24576 : (SC == kSABlk ? 25600 : 26112); }
__device__ __forceinline__ int swz_a(int x) { return x ^ (((x >> 10) & 1) << 7); }   // within 4 KiB of a row group
__device__ __forceinline__ int swz_b(int x) { return x ^ (((x >> 9) & 1) << 7); }    // within 2 KiB of a pair
__device__ __forceinline__ void dma16(const void* src, unsigned char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_wave_base, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* src, unsigned char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_wave_base, 4, 0, 0);
}

// RT row tiles per consumer wave: 4 (4 consumer waves, each a whole row group) or 2 (8 consumer waves, half a
// row group each; the per-128 modes, which hold int32 and fp32 accumulators). Two producer waves follow the
// consumers.
template <int SC, int OUT, int RT>
__global__ __launch_bounds__(64 * (16 / RT + 2), 1) void i8_gemm_kernel(I8Args p) {
  constexpr int CW = 16 / RT, SB = stage_bytes<SC>();
  constexpr int NST = (160 * 1024 - 64) / SB < 6 ? (160 * 1024 - 64) / SB : 6;   // LDS stages
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  int* flag = (int*)(lds + NST * SB);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = blockIdx.x, ky = blockIdx.y;
  const int K = p.K, N = p.N, KT = K >> 4;
  const int n0 = tile * 128;
  const int kslice = K / p.SKG, k0 = ky * kslice, nst = kslice >> 6;
  const int part = (p.a8[1] != nullptr && n0 >= p.n_split) ? 1 : 0;

  if (wave >= CW) {
    // ---- producers: q = 0 fetches row groups 0, 1 and pairs 0, 1 (+ SA); q = 1 row groups 2, 3 and pairs 2, 3
    // (+ SW); NST - 1 steps ahead. Steps past the slice re-read the last step into a stage nobody reads again,
    // so every iteration issues the same loads and one wait count fits all.
    const int q = wave - CW;
    const unsigned char* A8 = (const unsigned char*)p.a8[part];
    auto issue = [&](int st) {
      const int so = min(st, nst - 1);
      unsigned char* stg = lds + (st % NST) * SB;
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int rg = 2 * q + r;
        const unsigned char* src = A8 + ((size_t)rg * KT + (k0 >> 4) + 4 * so) * 1024;
#pragma unroll
        for (int c = 0; c < 4; ++c) dma16(src + swz_a(c * 1024 + lane * 16), stg + kStA + rg * 4096 + c * 1024);
      }
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int pp = 2 * q + r;
        const unsigned char* src = p.w + ((size_t)(tile * 4 + pp) * KT + (k0 >> 4) + 4 * so) * 512;
#pragma unroll
        for (int c = 0; c < 2; ++c) dma16(src + swz_b(c * 1024 + lane * 16), stg + kStB + pp * 2048 + c * 1024);
      }
      if constexpr (SC != kSCoarse) {
        const int kb = (k0 + 64 * so) >> 7;
        if (q == 0) dma16(p.sa[part] + (size_t)kb * 256 + lane * 4, stg + kStSA);
        if constexpr (SC == kSBlk) {
          if (q == 1) {
            dma4(p.sw + (size_t)kb * N + n0 + lane, stg + kStSW);
            dma4(p.sw + (size_t)kb * N + n0 + 64 + lane, stg + kStSW + 256);
          }
        }
      }
    };
#pragma unroll 1
    for (int i = 0; i < NST - 1; ++i) issue(i);
    for (int st = 0; st < nst; ++st) {
      // this producer's loads of stage st landed (the per-step count differs between the two producers)
      if (SC == kSCoarse) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(12 * (NST - 2)) : "memory");
      else if (SC == kSABlk) {
        if (q == 0) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(13 * (NST - 2)) : "memory");
        else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(12 * (NST - 2)) : "memory");
      } else {
        if (q == 0) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(13 * (NST - 2)) : "memory");
        else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(14 * (NST - 2)) : "memory");
      }
      __builtin_amdgcn_s_barrier();
      issue(st + NST - 1);   // into the stage read at step st - 1
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (p.SKG > 1) r4_ticket_last(p.tickets + tile, (unsigned)p.SKG, flag);   // its two barriers
    return;
  }

  // ---- consumers: wave w = row tiles RT (w % (4 / RT)) .. of row group w / (4 / RT), all 8 column tiles
  constexpr int WPG = 4 / RT;                  // consumer waves per row group
  const int rg = wave / WPG, i0 = RT * (wave % WPG);
  const int g = lane >> 4, rho = lane & 15, F = rho >> 3, cc = rho & 7;

  r4i4 iacc[RT][8];
  r4f4 facc[SC == kSCoarse ? 1 : RT][8];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int pc = 0; pc < 8; ++pc) iacc[i][pc] = (r4i4){0, 0, 0, 0};
  if constexpr (SC != kSCoarse) {
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int pc = 0; pc < 8; ++pc) facc[i][pc] = (r4f4){0.f, 0.f, 0.f, 0.f};
  }
  const int aoff = kStA + rg * 4096 + g * 1024 + rho * 8;       // + 256 i (+ 128 for the h = 1 half)
  const int boff = kStB + g * 512 + 16 * cc + 8 * F;           // + 2048 pp + 128 t (+ 256 for h = 1)

#pragma unroll 2
  for (int st = 0; st < nst; ++st) {
    // every consumer's reads of the previous stage done, then meet the producers' "stage st landed"
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    const unsigned char* stg = lds + (st % NST) * SB;
    r4i4 a[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const int o = aoff + (i0 + i) * 256;
      const r4u2 lo = *(const r4u2*)(stg + swz_a(o - kStA - rg * 4096) + kStA + rg * 4096);
      const r4u2 hi = *(const r4u2*)(stg + swz_a(o + 128 - kStA - rg * 4096) + kStA + rg * 4096);
      a[i] = (r4i4){(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
    }
#pragma unroll
    for (int pc = 0; pc < 8; ++pc) {
      const int pp = pc >> 1, t = pc & 1;
      const int o = boff - kStB + 128 * t;     // within the pair's 2 KiB
      const r4u2 lo = *(const r4u2*)(stg + kStB + pp * 2048 + swz_b(o));
      const r4u2 hi = *(const r4u2*)(stg + kStB + pp * 2048 + swz_b(o + 256));
      const r4i4 b = (r4i4){(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
#pragma unroll
      for (int i = 0; i < RT; ++i) iacc[i][pc] = mfma_i8(a[i], b, iacc[i][pc]);
    }
    if constexpr (SC != kSCoarse) {
      if (st & 1) {   // a 128-k block complete: acc += float(int32) * scale
        float swv[8];
#pragma unroll
        for (int pc = 0; pc < 8; ++pc)
          swv[pc] = SC == kSBlk ? *(const float*)(stg + kStSW + (16 * pc + 8 * F + cc) * 4) : 1.f;
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          const r4f4 sav = *(const r4f4*)(stg + kStSA + (64 * rg + 16 * (i0 + i) + 4 * g) * 4);
#pragma unroll
          for (int pc = 0; pc < 8; ++pc)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float sc = SC == kSBlk ? sav[j] * swv[pc] : sav[j];
              facc[i][pc][j] = __builtin_fmaf((float)iacc[i][pc][j], sc, facc[i][pc][j]);
              iacc[i][pc][j] = 0;
            }
        }
      }
    }
  }

  // this slice's values, one row tile at a time: row 64 rg + 16 i + 4 g + j, column n0 + 16 pc + 8 F + cc
  const bool split = p.SKG > 1;
  float swc[8];
  if constexpr (OUT != kOutI32) {
#pragma unroll
    for (int pc = 0; pc < 8; ++pc) swc[pc] = SC == kSBlk ? 1.f : p.sw[n0 + 16 * pc + 8 * F + cc];
  }
  const float* SA = p.sa[part];
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    const int ti = 4 * rg + i0 + i;   // row tile 0..15
    if constexpr (OUT == kOutI32) {
      i8_put<OUT>(iacc[i], p, tile, ky, ti, lane, split);
    } else {
      r4f4 v[8];
      r4f4 sar4 = (r4f4){1.f, 1.f, 1.f, 1.f};
      if constexpr (SC == kSCoarse) sar4 = *(const r4f4*)(SA + 16 * ti + 4 * g);
#pragma unroll
      for (int pc = 0; pc < 8; ++pc)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (SC == kSCoarse) v[pc][j] = (float)iacc[i][pc][j] * (sar4[j] * swc[pc]);
          else v[pc][j] = facc[i][pc][j] * swc[pc];
        }
      i8_put<OUT>(v, p, tile, ky, ti, lane, split);
    }
  }
  if (split && r4_ticket_last(p.tickets + tile, (unsigned)p.SKG, flag)) {
    if constexpr (OUT == kOutI32) i8_reduce<OUT, r4i4, RT>(p, tile, 4 * rg + i0, lane);
    else i8_reduce<OUT, r4f4, RT>(p, tile, 4 * rg + i0, lane);
  }
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

std::string i8_check(int M, int K, int N, int SKG) {
  if (M != 256) return "M must be 256 (the prefill chunk)";
  if (K <= 0 || N <= 0 || K % 128 || N % 128) return "K and N must be positive multiples of 128";
  if ((long long)N * K >= (1LL << 32)) return "N K must be below 2^32 bytes";
  if (SKG > 1 && (long long)SKG * 256 * N * 4 >= (1LL << 32)) return "the split workspace SKG 256 N 4 must be below 2^32 bytes";
  if (SKG < 1 || SKG > 64 || (K / 128) % SKG) return "SKG must be 1..64 and divide K / 128";
  return "";
}

template <int SC, int OUT>
void i8_launch(const I8Args& a, int K, int N, int SKG, hipStream_t st) {
  constexpr int RT = SC == kSCoarse ? 4 : 2;
  constexpr int SB = stage_bytes<SC>();
  constexpr int NST = (160 * 1024 - 64) / SB < 6 ? (160 * 1024 - 64) / SB : 6;
  const unsigned lds = NST * SB + 16;
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void*)i8_gemm_kernel<SC, OUT, RT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)lds);
    attr = true;
  }
  hipLaunchKernelGGL((i8_gemm_kernel<SC, OUT, RT>), dim3(N / 128, SKG), dim3(64 * (16 / RT + 2)), lds, st, a);
}

void i8_dense_run(int64_t a8, int64_t sa, int64_t w8, int64_t sw, int64_t c, int64_t ws, int64_t tickets, int M,
                  int K, int N, int SKG, int scale_mode, bool raw_i32, int64_t stream, const char* entry) {
  r4d::require(entry, i8_check(M, K, N, SKG));
  if (scale_mode < 0 || scale_mode > 2) r4d::fail(entry, "scale_mode must be 0 (row / column), 1 (per-128 "
                                                         "activation, column weight) or 2 (per-128 both)");
  if (!a8 || !w8 || !c || (!raw_i32 && (!sa || !sw))) r4d::fail(entry, "null buffer");
  if (SKG > 1 && (!ws || !tickets)) r4d::fail(entry, "a split launch (SKG > 1) needs ws and tickets");
  I8Args a{};
  a.a8[0] = (const signed char*)a8;
  a.sa[0] = (const float*)sa;
  a.n_split = N;
  a.w = (const unsigned char*)w8;
  a.sw = (const float*)sw;
  a.c = (void*)c;
  a.ws = (void*)ws;
  a.tickets = (unsigned*)tickets;
  a.K = K;
  a.N = N;
  a.SKG = SKG;
  a.out_scale = 1.f;
  hipStream_t st = (hipStream_t)stream;
  if (raw_i32) i8_launch<kSCoarse, kOutI32>(a, K, N, SKG, st);
  else if (scale_mode == 0) i8_launch<kSCoarse, kOutF16>(a, K, N, SKG, st);
  else if (scale_mode == 1) i8_launch<kSABlk, kOutF16>(a, K, N, SKG, st);
  else i8_launch<kSBlk, kOutF16>(a, K, N, SKG, st);
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
size_t r4d_gemm_i8_dense_ws_bytes(int M, int N, int SKG) { return SKG > 1 ? (size_t)SKG * M * N * 4 : 0; }

// The dense int8 GEMM: a8 in the A8 layout (r4d_trellis_i8_quant_act / _row), w8 in the W8 block layout
// (r4d_i8_pack_w), C f16 [256][N]. scale_mode 0: sa [256], sw [N]; 1: sa [K/128][256], sw [N]; 2: sa
// [K/128][256], sw [K/128][N]. SKG > 1: ws (ws_bytes) and tickets u32 [N/128] (zero before the first
// call, self-resetting).
void r4d_gemm_i8_dense(int64_t a8, int64_t sa, int64_t w8, int64_t sw, int64_t c, int64_t ws, int64_t tickets, int M,
                       int K, int N, int SKG, int scale_mode, int64_t stream) {
  i8_dense_run(a8, sa, w8, sw, c, ws, tickets, M, K, N, SKG, scale_mode, false, stream, "gemm_i8_dense");
}
// Test entry: the exact int32 sums C[m][n] = sum_k A[m][k] W[n][k] (int32 [256][N]) through the same kernel
// and split.
void r4d_gemm_i8_dense_raw(int64_t a8, int64_t w8, int64_t c, int64_t ws, int64_t tickets, int M, int K, int N,
                           int SKG, int64_t stream) {
  i8_dense_run(a8, 0, w8, 0, c, ws, tickets, M, K, N, SKG, 0, true, stream, "gemm_i8_dense_raw");
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
// This build's K split for the int8 GEMM (one workgroup per CU): the split that measured fastest at the
// config-4 shapes; others get the fewest slices that reach ~128 workgroups.
int r4d_mi355x_i8_skg(int K, int N) {
  const int G = N / 128, nkb = K / 128;
  int best = 1;
  for (int d = 1; d <= 16; ++d) {
    if (nkb % d) continue;
    best = d;
    if ((long long)G * d >= 128) break;
  }
  return best;
}

}  // extern "C"
