// trellis_m256.hip -- the trellis linear for a 256- (or 128-) row prefill chunk in one launch on gfx950:
// r4d_gemm_trellis_nt_m256, _check, _ws_bytes (the C ABI of the reference's third_party/libr4d/r4d.h:
// 395-423) and this build's _raw fp32 entry.
//
// C[m][n] = bf16((FWHT128(A_p(n) @ Q)[m][n] * svh[n]) * out_scale), A f16 [M][K] (M = 128 or 256).
//
// DESIGN (MI355X): MFMA-bound. A workgroup is 4 waves = all M rows x one 128-column group x one K slice
// (SKG slices across the grid). Per step of 4 k-tiles each wave loads one tile pair's 1 KiB with one
// dwordx4 per lane, decodes it with the GEMV's decode (r4d_dev.h) into four B fragments and writes
// them to a double-buffered LDS slot; after one barrier every wave reads the group's 16 fragments and
// runs (M / 64) x 4 pairs x 2 column slots x 2 k-halves v_mfma_f32_16x16x32_f16 against its own row
// tiles' A fragments, which it prefetched from global memory one step ahead. Each weight is decoded
// once for all M rows, so the decode VALU overlaps the MFMA stream. Unsplit, the epilogue applies the
// FWHT-128 in the accumulator layout -- column bits 0-2 and 4 across lanes, bits 3, 5 and 6 across
// registers, stages in the reference's order -- then svh, out_scale, one bf16 rounding. Split K
// (chosen only where it shortens the critical path: the partial sums are M x N fp32 per slice)
// writes each slice to ws and a second launch, tq_m256_finish, adds the slices in order and finishes.
#include "r4d_dev.h"
#include "r4d_host.h"
#include "r4d_mi355x.h"

namespace {

typedef __amdgpu_buffer_rsrc_t r4_rsrc;
__device__ __forceinline__ r4_rsrc mk_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)bytes, 0x00020000);
}

// RT = row tiles per wave (4 at M = 256, 2 at M = 128).
template <int KB, int RT>
__global__ __launch_bounds__(256, 2) void tq_m256_kernel(
    const unsigned short* __restrict__ A0, const unsigned short* __restrict__ A1, int n_split,
    const unsigned* __restrict__ W, const float* __restrict__ svh, void* __restrict__ Cv,
    float* __restrict__ ws, unsigned* __restrict__ tickets, int M, int K, int N, int SKG, int full,
    float out_scale) {
  constexpr int BLK = 16 * KB;                    // words per (pair, k-tile) block
  constexpr unsigned kStepBytes = 4 * BLK * 4;
  __shared__ r4u4 bfrag[2][4][4][64];             // [buf][pair][cs * 2 + h][lane]: 16 KiB x 2
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int group = blockIdx.x, ky = blockIdx.y;
  const int KT = K >> 4, ktw = KT / SKG, kt0 = ky * ktw;
  const int nst = ktw >> 2;
  const int q = lane >> 4, t = (lane >> 3) & 1, c = lane & 7, mrow = lane & 15;
  const unsigned short* __restrict__ A = group * 128 >= n_split ? A1 : A0;

  // this wave's weights: pair group * 4 + wave, k-tiles [kt0, kt0 + ktw)
  const int pair = group * 4 + wave;
  const r4_rsrc wr = mk_rsrc(W + ((size_t)pair * KT + kt0) * BLK, (unsigned)ktw * BLK * 4u);
  const unsigned tile = (unsigned)(q * 16 * KB + t * 8 * KB);
  const unsigned own = (tile + KB * c) * 4u, hist = (tile + (KB * c - 1 + 8 * KB) % (8 * KB)) * 4u;
  // this wave's A rows: 16 RT rows from wave * 16 RT; lane row mrow of each tile, k-tile q of a step
  const r4_rsrc ar = mk_rsrc(A, (unsigned)((size_t)M * K * 2));
  unsigned aoff[RT];
#pragma unroll
  for (int i = 0; i < RT; ++i)
    aoff[i] = (unsigned)(((size_t)(wave * 16 * RT + i * 16 + mrow) * K + (size_t)(kt0 + q) * 16) * 2);

  auto load_w = [&](unsigned (&w)[KB + 1], int st) {
    const unsigned so = (unsigned)st * kStepBytes;
    if constexpr (KB == 4) {
      const r4u4 v = __builtin_bit_cast(r4u4, __builtin_amdgcn_raw_buffer_load_b128(wr, own + so, 0, 0));
      w[1] = v[0]; w[2] = v[1]; w[3] = v[2]; w[4] = v[3];
    } else {
#pragma unroll
      for (int i = 0; i < KB; ++i) w[1 + i] = __builtin_amdgcn_raw_buffer_load_b32(wr, own + so + 4 * i, 0, 0);
    }
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(wr, hist + so, 0, 0);
  };
  auto load_a = [&](r4u4 (&a)[RT][2], int st) {
    const unsigned so = (unsigned)st * 4 * 32;   // 4 k-tiles of 16 halves
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      a[i][0] = __builtin_bit_cast(r4u4, __builtin_amdgcn_raw_buffer_load_b128(ar, aoff[i] + so, 0, 0));
      a[i][1] = __builtin_bit_cast(r4u4, __builtin_amdgcn_raw_buffer_load_b128(ar, aoff[i] + so + 16, 0, 0));
    }
  };

  r4f4 acc[RT][4][2];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int p = 0; p < 4; ++p) acc[i][p][0] = acc[i][p][1] = (r4f4){0.f, 0.f, 0.f, 0.f};

  unsigned wcur[KB + 1], wnext[KB + 1];
  r4u4 acur[RT][2], anext[RT][2];
  if (nst > 0) {
    load_w(wcur, 0);
    load_a(acur, 0);
  }
  for (int st = 0; st < nst; ++st) {
    const int buf = st & 1;
    if (st + 1 < nst) {
      load_w(wnext, st + 1);
      load_a(anext, st + 1);
    }
    {
      unsigned d[2][2][4];
      r4_decode<KB>(wcur, d);
#pragma unroll
      for (int cs = 0; cs < 2; ++cs)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          bfrag[buf][wave][cs * 2 + h][lane] = (r4u4){d[cs][h][0], d[cs][h][1], d[cs][h][2], d[cs][h][3]};
    }
    __syncthreads();
    // A fragments of this step: h = 0 takes k 0..3 and 8..11 of the lane's k-tile, h = 1 the rest
    r4h8 af[RT][2];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const r4u4 lo = acur[i][0], hi = acur[i][1];
      af[i][0] = __builtin_bit_cast(r4h8, (r4u4){lo[0], lo[1], hi[0], hi[1]});
      af[i][1] = __builtin_bit_cast(r4h8, (r4u4){lo[2], lo[3], hi[2], hi[3]});
    }
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int cs = 0; cs < 2; ++cs)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const r4h8 b = __builtin_bit_cast(r4h8, bfrag[buf][p][cs * 2 + h][lane]);
#pragma unroll
          for (int i = 0; i < RT; ++i) acc[i][p][cs] = r4_mfma16(af[i][h], b, acc[i][p][cs]);
        }
    if (st + 1 < nst) {
#pragma unroll
      for (int i = 0; i <= KB; ++i) wcur[i] = wnext[i];
#pragma unroll
      for (int i = 0; i < RT; ++i) { acur[i][0] = anext[i][0]; acur[i][1] = anext[i][1]; }
    }
  }

  // Lane l holds, for row tile i, rows 16 i + 4 (l >> 4) + j (+ this wave's base) and, for pair p
  // and slot cs, group column 32 p + 16 (nb >> 3) + (nb & 7) + 8 cs with nb = l & 15.
  const int nb = lane & 15, rq = lane >> 4;
  const int n0 = group * 128;
  const int row0 = wave * 16 * RT;
  if (SKG > 1) {
    // split K: this slice's sums to ws[ky]; tq_m256_finish adds the slices after this launch
    float* wsy = ws + (size_t)ky * M * N;
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = row0 + 16 * i + 4 * rq + j;
#pragma unroll
        for (int p = 0; p < 4; ++p)
#pragma unroll
          for (int cs = 0; cs < 2; ++cs)
            wsy[(size_t)r * N + n0 + 32 * p + 16 * (nb >> 3) + (nb & 7) + 8 * cs] = acc[i][p][cs][j];
      }
    return;
  }
  float* Cf = (float*)Cv;
  unsigned short* Cb = (unsigned short*)Cv;
  if (!full) {
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = row0 + 16 * i + 4 * rq + j;
#pragma unroll
        for (int p = 0; p < 4; ++p)
#pragma unroll
          for (int cs = 0; cs < 2; ++cs)
            Cf[(size_t)r * N + n0 + 32 * p + 16 * (nb >> 3) + (nb & 7) + 8 * cs] = acc[i][p][cs][j];
      }
    return;
  }
  // FWHT-128 over each row's group columns, stage lg = 0..6 on column bit lg: bits 0-2 are lane bits
  // 0-2 (partner lane ^ 1, 2, 4), bit 3 is cs, bit 4 is lane bit 3 (partner lane ^ 8), bits 5-6 are p.
  // The lower index keeps a + b, the upper takes a - b.
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v[4][2];
#pragma unroll
      for (int p = 0; p < 4; ++p) { v[p][0] = acc[i][p][0][j]; v[p][1] = acc[i][p][1][j]; }
      auto lane_stage = [&](int mask) {
        const bool upper = (lane & mask) != 0;
#pragma unroll
        for (int p = 0; p < 4; ++p)
#pragma unroll
          for (int cs = 0; cs < 2; ++cs) {
            const float o = __shfl_xor(v[p][cs], mask, 64);
            v[p][cs] = upper ? o - v[p][cs] : v[p][cs] + o;
          }
      };
      lane_stage(1);
      lane_stage(2);
      lane_stage(4);
#pragma unroll
      for (int p = 0; p < 4; ++p) {            // bit 3: cs
        const float a = v[p][0], b = v[p][1];
        v[p][0] = a + b;
        v[p][1] = a - b;
      }
      lane_stage(8);
#pragma unroll
      for (int cs = 0; cs < 2; ++cs) {         // bit 5: p ^ 1
        const float a0 = v[0][cs], b0 = v[1][cs], a1 = v[2][cs], b1 = v[3][cs];
        v[0][cs] = a0 + b0; v[1][cs] = a0 - b0;
        v[2][cs] = a1 + b1; v[3][cs] = a1 - b1;
      }
#pragma unroll
      for (int cs = 0; cs < 2; ++cs) {         // bit 6: p ^ 2
        const float a0 = v[0][cs], b0 = v[2][cs], a1 = v[1][cs], b1 = v[3][cs];
        v[0][cs] = a0 + b0; v[2][cs] = a0 - b0;
        v[1][cs] = a1 + b1; v[3][cs] = a1 - b1;
      }
      const int r = row0 + 16 * i + 4 * rq + j;
#pragma unroll
      for (int p = 0; p < 4; ++p)
#pragma unroll
        for (int cs = 0; cs < 2; ++cs) {
          const int n = n0 + 32 * p + 16 * (nb >> 3) + (nb & 7) + 8 * cs;
          const float y = v[p][cs] * svh[n];
          Cb[(size_t)r * N + n] = r4_bf16_rn(y * out_scale);
        }
    }
}

// The split form's second pass: a workgroup per (128-column group, 32 rows) sums the SKG slices of
// ws in slice order (coalesced: a thread per column, 16 rows each) into LDS, then one wave per row
// applies the group's FWHT-128 (r4_fwht128_wave, the reference's stage order), svh, out_scale and
// the bf16 rounding -- or, raw, stores the fp32 sums.
__global__ __launch_bounds__(256) void tq_m256_finish(const float* __restrict__ ws, const float* __restrict__ svh,
                                                      void* __restrict__ Cv, int M, int N, int SKG, int full,
                                                      float out_scale) {
  __shared__ float sums[32][128];
  const int group = blockIdx.x, r0 = blockIdx.y * 32;
  const int col = threadIdx.x & 127, rh = threadIdx.x >> 7;
  const int n0 = group * 128;
  const size_t sy = (size_t)M * N;
  float v[16];
#pragma unroll
  for (int u = 0; u < 16; ++u) v[u] = ws[(size_t)(r0 + rh + 2 * u) * N + n0 + col];
  for (int y = 1; y < SKG; ++y) {
    float t[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) t[u] = ws[(size_t)y * sy + (size_t)(r0 + rh + 2 * u) * N + n0 + col];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] += t[u];
  }
  if (!full) {
    float* Cf = (float*)Cv;
#pragma unroll
    for (int u = 0; u < 16; ++u) Cf[(size_t)(r0 + rh + 2 * u) * N + n0 + col] = v[u];
    return;
  }
#pragma unroll
  for (int u = 0; u < 16; ++u) sums[rh + 2 * u][col] = v[u];
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  unsigned short* Cb = (unsigned short*)Cv;
  const float sv0 = svh[n0 + lane], sv1 = svh[n0 + lane + 64];
  for (int r = wave; r < 32; r += 4) {
    float v0 = sums[r][lane], v1 = sums[r][lane + 64];
    r4_fwht128_wave(v0, v1, lane);
    const float y0 = v0 * sv0, y1 = v1 * sv1;
    Cb[(size_t)(r0 + r) * N + n0 + lane] = r4_bf16_rn(y0 * out_scale);
    Cb[(size_t)(r0 + r) * N + n0 + lane + 64] = r4_bf16_rn(y1 * out_scale);
  }
}

std::string m256_check(int M, int K, int N, int n_split, int KB, int SKG) {
  using r4d::str;
  if (M != 128 && M != 256) return "M must be 128 or 256";
  if (K <= 0 || N <= 0 || K % 128 || N % 128) return "K and N must be positive multiples of 128";
  if (KB != 3 && KB != 4 && KB != 5) return "KB " + str(KB) + " is not instantiated (3, 4, 5)";
  if (SKG < 1 || SKG > 64 || (K / 16) % (4 * SKG)) return "SKG must be 1..64 with (K/16) divisible by 4 SKG";
  if (n_split < 0 || n_split > N || n_split % 128) return "n_split must be in 0..N and a multiple of 128";
  return "";
}

template <int KB>
void m256_launch(int M, const unsigned short* a0, const unsigned short* a1, int n_split, const unsigned* w,
                 const float* svh, void* c, float* ws, unsigned* tickets, int K, int N, int SKG, int full,
                 float out_scale, hipStream_t st) {
  dim3 grid(N / 128, SKG), block(256);
  if (M == 256)
    hipLaunchKernelGGL((tq_m256_kernel<KB, 4>), grid, block, 0, st, a0, a1, n_split, w, svh, c, ws, tickets, M,
                       K, N, SKG, full, out_scale);
  else
    hipLaunchKernelGGL((tq_m256_kernel<KB, 2>), grid, block, 0, st, a0, a1, n_split, w, svh, c, ws, tickets, M,
                       K, N, SKG, full, out_scale);
}

void m256_run(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t svh, int64_t c, int64_t ws,
              int64_t tickets, int M, int K, int N, int KB, int SKG, int full, float out_scale, int64_t stream,
              const char* entry) {
  r4d::require(entry, m256_check(M, K, N, n_split, KB, SKG));
  if (!a0 || !w || !c) r4d::fail(entry, "null A, W or C");
  if (full && !svh) r4d::fail(entry, "svh must be non-null");
  if (SKG > 1 && !ws) r4d::fail(entry, "SKG > 1 needs ws");
  auto A0 = (const unsigned short*)a0, A1 = (const unsigned short*)(a1 ? a1 : a0);
  auto Wp = (const unsigned*)w;
  auto S = (const float*)svh;
  auto WS = (float*)ws;
  auto T = (unsigned*)tickets;
  hipStream_t st = (hipStream_t)stream;
  if (KB == 4) m256_launch<4>(M, A0, A1, n_split, Wp, S, (void*)c, WS, T, K, N, SKG, full, out_scale, st);
  else if (KB == 5) m256_launch<5>(M, A0, A1, n_split, Wp, S, (void*)c, WS, T, K, N, SKG, full, out_scale, st);
  else m256_launch<3>(M, A0, A1, n_split, Wp, S, (void*)c, WS, T, K, N, SKG, full, out_scale, st);
  if (SKG > 1)
    hipLaunchKernelGGL(tq_m256_finish, dim3(N / 128, M / 32), dim3(256), 0, st, (const float*)WS, S, (void*)c, M, N,
                       SKG, full, out_scale);
  r4d::launch_ok(entry);
}

}  // namespace

extern "C" {

// r4d.h:416-419. SK, NP, U and skw are the reference's geometry knobs: accepted, not used.
void r4d_gemm_trellis_nt_m256(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t svh, int64_t c,
                              int64_t ws, int64_t tickets, int M, int K, int N, int KB, int SK, int NP,
                              int SKG, int U, float out_scale, int64_t stream, int skw) {
  (void)SK; (void)NP; (void)U; (void)skw;
  m256_run(a0, a1, n_split, w, svh, c, ws, tickets, M, K, N, KB, SKG, 1, out_scale, stream,
           "gemm_trellis_nt_m256");
}

const char* r4d_gemm_trellis_nt_m256_check(int M, int K, int N, int n_split, int KB, int SK, int NP, int SKG,
                                           int U, int skw) {
  (void)SK; (void)NP; (void)U; (void)skw;
  return r4d::check_result(m256_check(M, K, N, n_split, KB, SKG));
}

size_t r4d_gemm_trellis_nt_m256_ws_bytes(int M, int N, int SKG) {
  return (size_t)SKG * (size_t)M * (size_t)N * sizeof(float);
}

void r4d_gemm_trellis_nt_m256_raw(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t c, int64_t ws,
                                  int64_t tickets, int M, int K, int N, int KB, int SKG, int64_t stream) {
  m256_run(a0, a1, n_split, w, 0, c, ws, tickets, M, K, N, KB, SKG, 0, 1.f, stream, "gemm_trellis_nt_m256_raw");
}

// This build's K split for the prefill GEMM: the workgroup count per CU decides the critical path
// (at most two resident per CU, sharing its MFMA pipes), so SKG minimises ceil(G SKG / CUs) x steps
// per slice plus the cost of the second pass (SKG x M x N fp32 written and read back).
int r4d_mi355x_trellis_m256_skg(int K, int N, int KB) {
  (void)KB;
  const int KT = K / 16, G = N / 128;
  if (KT <= 0 || G <= 0) return 1;
  int cus = 256, dev = 0;
  if (hipGetDevice(&dev) == hipSuccess) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) cus = n;
  }
  int best = 1;
  double best_cost = 1e30;
  for (int d = 1; d <= 16; ++d) {
    if (KT % (4 * d)) continue;
    const double rounds = (double)(((long long)G * d + cus - 1) / cus);
    const double steps = (double)KT / (4 * d);
    // one step ~ 0.43 us of MFMA; partials ~ 256 * 128 * 4 * 2 bytes per workgroup-slice at ~6 TB/s
    const double cost = rounds * steps * 0.43 + (d > 1 ? (double)G * d * 262144.0 / 6e6 + 2.0 : 0.0);
    if (cost < best_cost) {
      best_cost = cost;
      best = d;
    }
  }
  return best;
}

}  // extern "C"
