// trellis_gemv.hip -- the trellis linear for M = 1..64 rows on gfx950: r4d_gemm_trellis_nt_m64, its
// _raw fp32 entry, r4d_trellis_reconstruct_f16 and the ticket helpers (the C ABI of the reference's
// third_party/libr4d/r4d.h:344-393, kernel semantics of r4d_gemm_trellis_nt_m64.hip:215-503).
//
// C[m][n] = bf16((FWHT128(A_p(n) @ Q)[m][n] * svh[n]) * out_scale)   (full), or fp32 A @ Q (_raw).
//
// DESIGN (MI355X): decode is VALU work and the multiply-accumulate is MFMA work, so they run on
// different pipes. Each wave streams one tile pair's k-range in 1 KiB steps (one dwordx4 per lane,
// four (pair, k-tile) blocks at KB = 4), decodes its 32 weights per lane into four B fragments
// (r4d_dev.h) and issues 4 x MT v_mfma_f32_16x16x32_f16 per step; at M <= 16 one row tile carries
// the whole batch, so the MFMA cost per weight is independent of M up to 16. A workgroup is four
// waves = four pairs = one 128-column FWHT group; SKG workgroups split K. Partial sums go to ws
// [SKG][M][N] and the last workgroup of a group (ticket) sums them in slice order and finishes:
// FWHT-128 in fp32 in the reference's stage order, * svh, * out_scale, one bf16 rounding. A row's
// bits depend on (K, N, KB, SKG) only -- never on M or the other rows -- so decode rows equal verify
// rows for every M <= 64 with the same SKG.
#include "r4d_dev.h"
#include "r4d_host.h"
#include "r4d_mi355x.h"

namespace {

constexpr int kWaves = 4;                      // pairs per workgroup = one 128-column group
constexpr int kThreads = kWaves * R4_WAVE;

template <int KB>
struct Words {
  unsigned w[KB + 1];   // [0] history, [1..KB] own words
};

// Loads the lane's ring words of block (pair, k-tile kt): own words KB c .. KB c + KB - 1 of tile t,
// and the history word before them.
template <int KB>
__device__ __forceinline__ void load_words(Words<KB>& s, const unsigned* __restrict__ blk, int t, int c) {
  const unsigned* tile = blk + t * 8 * KB;
  if constexpr (KB == 4) {
    const r4u4 v = *(const r4u4*)(tile + 4 * c);
    s.w[1] = v[0]; s.w[2] = v[1]; s.w[3] = v[2]; s.w[4] = v[3];
    s.w[0] = tile[(4 * c + 31) & 31];
  } else {
#pragma unroll
    for (int i = 0; i <= KB; ++i) s.w[i] = tile[r4_lane_word<KB>(c, i)];
  }
}

// The lane's two A fragments (h = 0, 1) of row r, k-tile kt: k 16kt + {0..3, 8..11} and {4..7, 12..15}.
__device__ __forceinline__ void load_a(r4h8 (&af)[2], const unsigned short* __restrict__ arow, int kt) {
  const r4u4 lo = *(const r4u4*)(arow + 16 * kt);
  const r4u4 hi = *(const r4u4*)(arow + 16 * kt + 8);
  const r4u4 f0 = {lo[0], lo[1], hi[0], hi[1]}, f1 = {lo[2], lo[3], hi[2], hi[3]};
  af[0] = __builtin_bit_cast(r4h8, f0);
  af[1] = __builtin_bit_cast(r4h8, f1);
}

template <int KB, int MT>
struct Stage {
  Words<KB> w;
  r4h8 a[MT][2];
};

template <int KB, int MT>
__global__ __launch_bounds__(kThreads) void tq_gemv_kernel(
    const unsigned short* __restrict__ A0, const unsigned short* __restrict__ A1, int n_split,
    const unsigned* __restrict__ W, const float* __restrict__ svh, void* __restrict__ Cv,
    float* __restrict__ ws, unsigned* __restrict__ tickets, int M, int K, int N, int SKG, int full,
    float out_scale) {
  extern __shared__ float red[];               // [MT * 16][128] + flag
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int group = blockIdx.x, ky = blockIdx.y;
  const int pair = group * kWaves + wave;
  const int KT = K >> 4, ktw = KT / SKG, kt0 = ky * ktw;
  const int steps = (ktw + 3) >> 2;
  const unsigned short* __restrict__ A = group * 128 >= n_split ? A1 : A0;
  const int q = lane >> 4, t = (lane >> 3) & 1, c = lane & 7, mrow = lane & 15;
  constexpr int BLK = 16 * KB;                 // words per (pair, k-tile) block

  const unsigned* __restrict__ wpair = W + ((size_t)pair * KT + kt0) * BLK;
  const unsigned short* arow[MT];
  bool arow_ok[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int r = i * 16 + mrow;
    arow_ok[i] = r < M;
    arow[i] = A + (size_t)(r < M ? r : 0) * K;
  }

  r4f4 acc[MT][2];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i][0] = acc[i][1] = (r4f4){0.f, 0.f, 0.f, 0.f};

  auto load = [&](Stage<KB, MT>& s, int st) {
    const int ktl = st * 4 + q;                // k-tile inside the slice
    const bool ok = ktl < ktw;
    if (ok) {
      load_words<KB>(s.w, wpair + (size_t)ktl * BLK, t, c);
    } else {
#pragma unroll
      for (int i = 0; i <= KB; ++i) s.w.w[i] = 0u;
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      if (ok && arow_ok[i]) {
        load_a(s.a[i], arow[i], kt0 + ktl);
      } else {
        s.a[i][0] = s.a[i][1] = (r4h8){0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
  };
  auto compute = [&](const Stage<KB, MT>& s) {
    unsigned d[2][2][4];
    r4_decode<KB>(s.w.w, d);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const r4h8 b0 = r4_frag(d[0][h]), b1 = r4_frag(d[1][h]);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        acc[i][0] = r4_mfma16(s.a[i][h], b0, acc[i][0]);
        acc[i][1] = r4_mfma16(s.a[i][h], b1, acc[i][1]);
      }
    }
  };

  {
    Stage<KB, MT> s0, s1;
    load(s0, 0);
    int st = 0;
    for (; st + 1 < steps; st += 2) {
      load(s1, st + 1);
      compute(s0);
      if (st + 2 < steps) load(s0, st + 2);
      compute(s1);
    }
    if (st < steps) compute(s0);
  }

  // Lane l holds rows 16 i + 4 (l >> 4) + j of column slot nb = l & 15 of fragment cs: true column
  // 32 pair + 16 (nb >> 3) + (nb & 7) + 8 cs.
  const int nb = lane & 15, rq = lane >> 4;
  const int colp = 16 * (nb >> 3) + (nb & 7);  // + 8 cs, inside the pair
  const int gcol0 = wave * 32 + colp;          // inside the group
  float* Cf = (float*)Cv;
  unsigned short* Cb = (unsigned short*)Cv;
  const int n0 = group * 128;

  if (SKG == 1 && !full) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 16 * i + 4 * rq + j;
        if (r < M) {
          Cf[(size_t)r * N + n0 + gcol0] = acc[i][0][j];
          Cf[(size_t)r * N + n0 + gcol0 + 8] = acc[i][1][j];
        }
      }
    return;
  }
  if (SKG == 1) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 16 * i + 4 * rq + j;
        if (r < M) {
          red[r * 128 + gcol0] = acc[i][0][j];
          red[r * 128 + gcol0 + 8] = acc[i][1][j];
        }
      }
    __syncthreads();
  } else {
    float* wsy = ws + (size_t)ky * M * N;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 16 * i + 4 * rq + j;
        if (r < M) {
          wsy[(size_t)r * N + n0 + gcol0] = acc[i][0][j];
          wsy[(size_t)r * N + n0 + gcol0 + 8] = acc[i][1][j];
        }
      }
    int* flag = (int*)(red + MT * 16 * 128);
    if (!r4_ticket_last(&tickets[group], (unsigned)SKG, flag)) return;
    // Sum the SKG partials in slice order.
    for (int idx = threadIdx.x; idx < M * 128; idx += kThreads) {
      const int r = idx >> 7, col = idx & 127;
      const float* p = ws + (size_t)r * N + n0 + col;
      float v = p[0];
      for (int y = 1; y < SKG; ++y) v += p[(size_t)y * M * N];
      if (full) red[idx] = v;
      else Cf[(size_t)r * N + n0 + col] = v;
    }
    if (!full) return;
    __syncthreads();
  }
  // The epilogue: one wave per row, the group's 128 sums as (lane, lane + 64).
  const float sv0 = svh[n0 + lane], sv1 = svh[n0 + lane + 64];
  for (int r = wave; r < M; r += kWaves) {
    float v0 = red[r * 128 + lane], v1 = red[r * 128 + lane + 64];
    r4_fwht128_wave(v0, v1, lane);
    const float y0 = v0 * sv0, y1 = v1 * sv1;
    Cb[(size_t)r * N + n0 + lane] = r4_bf16_rn(y0 * out_scale);
    Cb[(size_t)r * N + n0 + lane + 64] = r4_bf16_rn(y1 * out_scale);
  }
}

// One wave per (tile pair, 4-k-tile step): every lane decodes its 32 weights with the GEMM's own
// decode and scatters them to their true (k, n).
template <int KB>
__global__ __launch_bounds__(256) void tq_reconstruct_kernel(const unsigned* __restrict__ W,
                                                            unsigned short* __restrict__ Q, int K, int N) {
  const int lane = threadIdx.x & 63;
  const int KT = K >> 4, steps = (KT + 3) >> 2;
  const long long id = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (id >= (long long)(N >> 5) * steps) return;
  const int pair = (int)(id / steps), st = (int)(id - (long long)pair * steps);
  const int q = lane >> 4, t = (lane >> 3) & 1, c = lane & 7;
  const int kt = st * 4 + q;
  if (kt >= KT) return;
  Words<KB> s;
  load_words<KB>(s, W + ((size_t)pair * KT + kt) * (16 * KB), t, c);
  unsigned d[2][2][4];
  r4_decode<KB>(s.w, d);
#pragma unroll
  for (int cs = 0; cs < 2; ++cs) {
    const int n = pair * 32 + 16 * t + c + 8 * cs;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int k = kt * 16 + 8 * (e >> 2) + 4 * h + (e & 3);
        Q[(size_t)k * N + n] = (unsigned short)(d[cs][h][e >> 1] >> (16 * (e & 1)));
      }
  }
}

template <int KB, int MT>
void launch_gemv(const r4d_gemv_args& a) {
  dim3 grid(a.N / 128, a.SKG), block(kThreads);
  const size_t smem = (size_t)MT * 16 * 128 * sizeof(float) + 16;
  hipLaunchKernelGGL((tq_gemv_kernel<KB, MT>), grid, block, smem, (hipStream_t)a.stream,
                     (const unsigned short*)a.a0, (const unsigned short*)(a.a1 ? a.a1 : a.a0), a.n_split,
                     (const unsigned*)a.w, (const float*)a.svh, (void*)a.c, (float*)a.ws,
                     (unsigned*)a.tickets, a.M, a.K, a.N, a.SKG, a.full, a.out_scale);
}

template <int KB>
void launch_gemv_kb(const r4d_gemv_args& a) {
  const int mt = (a.M + 15) / 16;
  if (mt <= 1) launch_gemv<KB, 1>(a);
  else if (mt <= 2) launch_gemv<KB, 2>(a);
  else launch_gemv<KB, 4>(a);
}

}  // namespace

// ---- host entries ------------------------------------------------------------------------------
extern "C" {

const char* r4d_gemm_trellis_nt_m64_check(int M, int K, int N, int n_split, int KB, int SKG,
                                          int full, int have_svh, int have_ws) {
  using r4d::str;
  std::string e;
  if (M < 1 || M > 64) e = "M must be 1..64";
  else if (K <= 0 || N <= 0 || K % 128 || N % 128) e = "K and N must be positive multiples of 128";
  else if (KB != 3 && KB != 4 && KB != 5) e = "KB " + str(KB) + " is not instantiated (3, 4, 5)";
  else if (SKG < 1 || SKG > 64 || (K / 16) % SKG) e = "SKG must be 1..64 and divide K/16";
  else if (n_split < 0 || n_split > N || n_split % 128) e = "n_split must be in 0..N and a multiple of 128";
  else if (SKG > 1 && !have_ws) e = "SKG > 1 needs ws and tickets";
  else if (full && !have_svh) e = "svh must be non-null";
  return r4d::check_result(e);
}

static void tq_run(r4d_gemv_args& a, const char* entry) {
  if (!a.a0 || !a.w || !a.c) r4d::fail(entry, "null A, W or C");
  if (const char* m = r4d_gemm_trellis_nt_m64_check(a.M, a.K, a.N, a.n_split, a.KB, a.SKG, a.full,
                                                    a.svh != 0, a.ws != 0 && a.tickets != 0))
    r4d::fail(entry, m);
  if (a.KB == 4) launch_gemv_kb<4>(a);
  else if (a.KB == 5) launch_gemv_kb<5>(a);
  else launch_gemv_kb<3>(a);
  r4d::launch_ok(entry);
}

void r4d_gemm_trellis_nt_m64(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t svh, int64_t c,
                             int64_t ws, int64_t tickets, int M, int K, int N, int KB, int WV, int SK,
                             int MT, int NP, int SKG, int U, int NT, float out_scale, int64_t stream) {
  (void)WV; (void)SK; (void)MT; (void)NP; (void)U; (void)NT;
  r4d_gemv_args a{a0, a1, n_split, w, svh, c, ws, tickets, M, K, N, KB, SKG, 1, out_scale, stream};
  tq_run(a, "gemm_trellis_nt_m64");
}

void r4d_gemm_trellis_nt_m64_raw(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t c, int64_t ws,
                                 int64_t tickets, int M, int K, int N, int KB, int WV, int SK, int MT,
                                 int NP, int SKG, int U, int NT, int64_t clk, int64_t stream) {
  (void)WV; (void)SK; (void)MT; (void)NP; (void)U; (void)NT; (void)clk;
  r4d_gemv_args a{a0, a1, n_split, w, 0, c, ws, tickets, M, K, N, KB, SKG, 0, 1.f, stream};
  tq_run(a, "gemm_trellis_nt_m64_raw");
}

int r4d_gemm_trellis_nt_m64_has_rate(int KB) { return KB == 3 || KB == 4 || KB == 5; }
int r4d_gemm_trellis_nt_m64_max_m(void) { return 64; }
size_t r4d_gemm_trellis_nt_m64_ws_bytes(int M, int N, int SKG) {
  return (size_t)SKG * (size_t)M * (size_t)N * sizeof(float);
}
size_t r4d_gemm_trellis_nt_m64_tickets_bytes(int N) { return (size_t)(N > 0 ? N / 128 : 0) * sizeof(unsigned); }

void r4d_gemm_trellis_nt_m64_zero_tickets(int64_t tickets, size_t bytes, int64_t stream) {
  if (bytes == 0) return;
  if (tickets == 0) r4d::fail("gemm_trellis_nt_m64_zero_tickets", "null buffer");
  const hipError_t e = hipMemsetAsync((void*)tickets, 0, bytes, (hipStream_t)stream);
  if (e != hipSuccess) r4d::fail("gemm_trellis_nt_m64_zero_tickets", hipGetErrorString(e));
}

void r4d_trellis_reconstruct_f16(int64_t w, int64_t q, int K, int N, int KB, int64_t stream) {
  const char* entry = "trellis_reconstruct_f16";
  if (K <= 0 || N <= 0 || K % 16 || N % 32)
    r4d::fail(entry, "K must be a multiple of 16 and N of 32 (whole tile pairs)");
  if (KB != 3 && KB != 4 && KB != 5) r4d::fail(entry, "KB must be 3, 4 or 5");
  if (!w || !q) r4d::fail(entry, "null buffer");
  const long long waves = (long long)(N / 32) * ((K / 16 + 3) / 4);
  dim3 grid((unsigned)((waves + 3) / 4)), block(256);
  hipStream_t st = (hipStream_t)stream;
  auto W = (const unsigned*)w;
  auto Q = (unsigned short*)q;
  if (KB == 4) hipLaunchKernelGGL(tq_reconstruct_kernel<4>, grid, block, 0, st, W, Q, K, N);
  else if (KB == 5) hipLaunchKernelGGL(tq_reconstruct_kernel<5>, grid, block, 0, st, W, Q, K, N);
  else hipLaunchKernelGGL(tq_reconstruct_kernel<3>, grid, block, 0, st, W, Q, K, N);
  r4d::launch_ok(entry);
}

// This build's split choice for the GEMV: the smallest divisor SKG of K/16 that puts at least 512
// workgroups (two per CU) on the chip while every slice keeps >= 8 k-tiles; independent of M, so
// every M <= 64 gets the same row bits.
int r4d_mi355x_trellis_gemv_skg(int K, int N, int KB) {
  (void)KB;
  const int KT = K / 16, groups = N / 128;
  if (KT <= 0 || groups <= 0) return 1;
  int best = 1;
  for (int d = 1; d <= 64 && d <= KT; ++d) {
    if (KT % d) continue;
    if (KT / d < 8) break;
    best = d;
    if (groups * d >= 512) break;
  }
  return best;
}

}  // extern "C"
