// w4a16.hip -- the 4-bit group-quantized skinny GEMM on gfx950 (LM head and drafters): the C ABI of the
// reference's third_party/libr4d/r4d.h:324-342 (r4d_gemm_w4a16_nt_m64, _g, _max_m, _group, _has_group)
// over its packed layout (src/convert/include/r4dx_convert/quant_int4.hpp:171-244), plus this build's
// fp32-output entry for logits.
//
// C[m][n] = sum over groups g of scale[n][g] * sum_{k in g} A[m][k] * (q[n][k] - zero[n][g]),
// q = stored nibble ^ 8, q - zero formed exactly in f16, the group sum in fp32, scaled in fp32
// (the reference's order of operations, r4d_gemm_w4a16_nt_m64.hip:139-164).
//
// THE PACKED LAYOUT. Wq dword (((t * K/64 + kb) * 2 + lh) * 16 + r) * 4 + s holds row n = 16 t + r,
// k = 64 kb + 16 s + 4 lh + {0, 8, 1, 9, 2, 10, 3, 11}[i] in nibble i. Wsz (t, group, r): f16 scale in the
// low half, f16(-(1024 + zero)) in the high half.
//
// DESIGN (MI355X): HBM-bound. A wave streams two row tiles (32 output columns) over all of K, one
// coalesced dwordx4 per lane per 64-k block: lane l takes tile 2p + ((l & 31) >> 4), lh = l >> 5,
// r = l & 15 -- exactly the B operand of v_mfma_f32_32x32x16_f16 (lane = column l & 31, k-half l >> 5)
// for each of its four dwords s. Dequant per dword: one xor (the ^ 8), four and_or into the f16 bits
// of 1024 + q, four packed f16 adds of -(1024 + zero): element e of the fragment is nibble
// {0, 4, 1, 5, 2, 6, 3, 7}[e]. A is staged once per workgroup in LDS in that element order. A group's
// MFMA chain starts from zero and is added into the fp32 accumulator times the lane's column scale.
// N = 248 320 gives 7 760 waves of work, so no split of K is needed.
#include "r4d_dev.h"
#include "r4d_host.h"
#include "r4d_mi355x.h"

namespace {

typedef __amdgpu_buffer_rsrc_t r4_rsrc;
__device__ __forceinline__ r4_rsrc mk_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ r4f16 mfma32(r4h8 a, r4h8 b, r4f16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// The k offset (inside a 16-k step, before the lane half's 4 lh) of fragment element e.
__host__ __device__ constexpr int w4_elem_k(int e) {
  // e -> nibble {0,4,1,5,2,6,3,7}[e] -> k {0,8,1,9,2,10,3,11}[nibble]
  return e == 0 ? 0 : e == 1 ? 2 : e == 2 ? 8 : e == 3 ? 10 : e == 4 ? 1 : e == 5 ? 3 : e == 6 ? 9 : 11;
}

constexpr int kWaves = 8;      // 8 waves = 256 output columns per workgroup
constexpr int kPF = 6;         // weight steps in flight per wave

// MT = row tiles of 32 (M <= 32: 1, M <= 64: 2). G = group (32 or 64). OUTF = fp32 output.
template <int G, int MT, bool OUTF>
__global__ __launch_bounds__(64 * kWaves) void w4_kernel(const unsigned short* __restrict__ A,
                                                          const unsigned* __restrict__ Wq,
                                                          const unsigned* __restrict__ Wsz,
                                                          void* __restrict__ Cv, int M, int K, int N) {
  extern __shared__ r4u4 alds[];             // [kb][s][lh][M][8 halves] + a zero block
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int KB64 = K >> 6, groups = K / G;
  const int tiles = N >> 4;
  const int t0 = (blockIdx.x * kWaves + wave) * 2;     // this wave's first row tile
  const int tl = t0 + ((lane & 31) >> 4), lh = lane >> 5, r = lane & 15;
  const size_t zero_blk = (size_t)KB64 * 4 * 2 * M;

  // Stage A in the fragment element order: fragment (kb, s, lh, m) element e = A[m][64 kb + 16 s + 4 lh + w4_elem_k(e)].
  for (int i = threadIdx.x; i < KB64 * 4 * 2 * M; i += 64 * kWaves) {
    const int m = i % M, rest = i / M, h = rest & 1, ks = rest >> 1;   // ks = kb * 4 + s
    const unsigned short* src = A + (size_t)m * K + 16 * ks + 4 * h;
    const r4u2 lo = *(const r4u2*)src, hi = *(const r4u2*)(src + 8);   // k +0..3, +8..11
    // elements: (k0, k2) (k8, k10) (k1, k3) (k9, k11)
    r4u4 v;
    v[0] = __builtin_amdgcn_perm(lo[1], lo[0], 0x05040100u);
    v[1] = __builtin_amdgcn_perm(hi[1], hi[0], 0x05040100u);
    v[2] = __builtin_amdgcn_perm(lo[1], lo[0], 0x07060302u);
    v[3] = __builtin_amdgcn_perm(hi[1], hi[0], 0x07060302u);
    alds[i] = v;
  }
  if (threadIdx.x == 0) alds[zero_blk] = (r4u4){0u, 0u, 0u, 0u};
  __syncthreads();
  if (t0 >= tiles) return;

  // lane's weights: 16 bytes of block (tl, kb) at lh, r; the tile's blocks are consecutive in kb
  const r4_rsrc wr = mk_rsrc(Wq, (unsigned)((size_t)N * K / 2));
  const unsigned wlane = (unsigned)((((size_t)tl * KB64) * 2 + lh) * 16 + r) * 16u;
  const r4_rsrc sr = mk_rsrc(Wsz, (unsigned)((size_t)N * groups * 4));
  const unsigned slane = (unsigned)(((size_t)tl * groups * 16) + r) * 4u;

  // A fragment address per row tile: (kb, s) advance; rows >= M read the zero block
  unsigned a_lane[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int m = i * 32 + (lane & 31);
    a_lane[i] = m < M ? (unsigned)((lh * M + m) * 16) : 0xFFFFFFFFu;
  }
  auto afrag = [&](int i, int kb, int s) -> r4h8 {
    const unsigned off = a_lane[i] != 0xFFFFFFFFu ? (unsigned)((kb * 4 + s) * 2 * M * 16) + a_lane[i]
                                                  : (unsigned)(zero_blk * 16);
    return __builtin_bit_cast(r4h8, *(const r4u4*)((const char*)alds + off));
  };

  r4f16 acc[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.f;

  struct St {
    r4u4 w;
    unsigned sz[G == 32 ? 2 : 1];
  };
  auto load = [&](St& s, int kb) {
    const int kc = kb < KB64 ? kb : KB64 - 1;
    s.w = __builtin_bit_cast(r4u4, __builtin_amdgcn_raw_buffer_load_b128(wr, wlane + (unsigned)kc * 512u, 0, 0));
    if constexpr (G == 64) {
      s.sz[0] = __builtin_amdgcn_raw_buffer_load_b32(sr, slane + (unsigned)kc * 64u, 0, 0);
    } else {
      s.sz[0] = __builtin_amdgcn_raw_buffer_load_b32(sr, slane + (unsigned)(2 * kc) * 64u, 0, 0);
      s.sz[1] = __builtin_amdgcn_raw_buffer_load_b32(sr, slane + (unsigned)(2 * kc + 1) * 64u, 0, 0);
    }
  };
  auto compute = [&](const St& s, int kb) {
    // dequant the four dwords: (q - zero) as f16 pairs in fragment order
    r4h8 b[4];
#pragma unroll
    for (int sI = 0; sI < 4; ++sI) {
      const unsigned nzw = s.sz[G == 32 ? (sI >> 1) : 0] >> 16;
      const r4h2 nz = __builtin_bit_cast(r4h2, nzw | (nzw << 16));
      const unsigned x = s.w[sI] ^ 0x88888888u;
      r4u4 f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const unsigned p = ((x >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
        f[j] = __builtin_bit_cast(unsigned, __builtin_bit_cast(r4h2, p) + nz);
      }
      b[sI] = __builtin_bit_cast(r4h8, f);
    }
#pragma unroll
    for (int gi = 0; gi < (G == 32 ? 2 : 1); ++gi) {
      const float sc = r4_f16_to_f32((unsigned short)(s.sz[gi] & 0xFFFFu));
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        r4f16 tmp;
#pragma unroll
        for (int e = 0; e < 16; ++e) tmp[e] = 0.f;
#pragma unroll
        for (int sI = gi * (G / 16); sI < (gi + 1) * (G / 16); ++sI) tmp = mfma32(afrag(i, kb, sI), b[sI], tmp);
        // only the rows this launch has: row = (e / 4) * 8 + lh * 4 + e % 4
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (i * 32 + (e >> 2) * 8 < M) acc[i][e] = __builtin_fmaf(tmp[e], sc, acc[i][e]);
      }
    }
  };

  St ring[kPF];
#pragma unroll
  for (int i = 0; i < kPF; ++i) load(ring[i], i);
  for (int kb = 0; kb < KB64; ++kb) {
    compute(ring[0], kb);
#pragma unroll
    for (int i = 0; i + 1 < kPF; ++i) ring[i] = ring[i + 1];
    load(ring[kPF - 1], kb + kPF);
  }

  // lane holds column n = 16 t0 + (lane & 31), rows (e / 4) * 8 + lh * 4 + e % 4 of each row tile
  const int n = 16 * t0 + (lane & 31);
  if (n >= N) return;
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = i * 32 + (e >> 2) * 8 + lh * 4 + (e & 3);
      if (m < M) {
        if constexpr (OUTF) ((float*)Cv)[(size_t)m * N + n] = acc[i][e];
        else ((unsigned short*)Cv)[(size_t)m * N + n] = r4_bf16_rn(acc[i][e]);
      }
    }
}

std::string w4_check(int group, int M, int K, int N) {
  if (group != 32 && group != 64) return "group " + r4d::str(group) + " is not instantiated (32, 64)";
  if (M < 1 || M > 64) return "M must be 1..64";
  if (N <= 0 || N % 16) return "N must be a positive multiple of 16";
  if (K <= 0 || K % 64) return "K must be a positive multiple of 64 (the packed 64-k block)";
  if ((size_t)(K / 64) * 8 * M * 16 + 16 > 144 * 1024) return "M x K too large for the LDS copy of A";
  return "";
}

template <int G, bool OUTF>
void w4_launch(int64_t a, int64_t wq, int64_t wsz, int64_t c, int M, int K, int N, hipStream_t st) {
  const int tiles = N / 16;
  const int waves = (tiles + 1) / 2;
  dim3 grid((waves + kWaves - 1) / kWaves), block(64 * kWaves);
  const size_t smem = (size_t)(K / 64) * 8 * M * 16 + 16;
  auto Ap = (const unsigned short*)a;
  auto Wp = (const unsigned*)wq;
  auto Sp = (const unsigned*)wsz;
  if (M <= 32) hipLaunchKernelGGL((w4_kernel<G, 1, OUTF>), grid, block, smem, st, Ap, Wp, Sp, (void*)c, M, K, N);
  else hipLaunchKernelGGL((w4_kernel<G, 2, OUTF>), grid, block, smem, st, Ap, Wp, Sp, (void*)c, M, K, N);
}

void w4_run(int group, int64_t a, int64_t wq, int64_t wsz, int64_t c, int M, int K, int N, bool outf,
            int64_t stream, const char* entry) {
  r4d::require(entry, w4_check(group, M, K, N));
  if (!a || !wq || !wsz || !c) r4d::fail(entry, "null buffer");
  hipStream_t st = (hipStream_t)stream;
  if (group == 32) {
    if (outf) w4_launch<32, true>(a, wq, wsz, c, M, K, N, st);
    else w4_launch<32, false>(a, wq, wsz, c, M, K, N, st);
  } else {
    if (outf) w4_launch<64, true>(a, wq, wsz, c, M, K, N, st);
    else w4_launch<64, false>(a, wq, wsz, c, M, K, N, st);
  }
  r4d::launch_ok(entry);
}

// ---- argmax ------------------------------------------------------------------------------------------
// (value, index) as one 64-bit key whose unsigned order is the reference's total order (larger value
// first, then lower index; src/kernels/include/r4dx/kernels/argmax_ref.hpp:22-41): the value's bits made
// order-preserving in the high word, the complemented index in the low word. A NaN gets key 0 (it never
// wins); the seed (-inf, 0) is the key of an element (-inf, 0), so a row whose elements are all -inf or
// NaN yields (-inf, 0). The maximum of keys is partition- and order-independent, so the multi-workgroup
// reduction is exact and deterministic.
__device__ __forceinline__ unsigned long long am_key(float v, unsigned idx) {
  unsigned u = __builtin_bit_cast(unsigned, v);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0ull;
  if ((u & 0x7FFFFFFFu) == 0u) u = 0u;                 // -0 == +0: equal values, the index decides
  const unsigned ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)ord << 32) | (unsigned long long)(~idx);
}
__device__ __forceinline__ void am_decode(unsigned long long key, int* idx, float* val) {
  const unsigned long long seed = am_key(-__builtin_inff(), 0u);
  if (key < seed) key = seed;
  const unsigned ord = (unsigned)(key >> 32);
  const unsigned u = (ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord;
  *idx = (int)(~(unsigned)key);
  *val = __builtin_bit_cast(float, u);
}
__device__ __forceinline__ unsigned long long am_max(unsigned long long a, unsigned long long b) { return a > b ? a : b; }
__device__ __forceinline__ unsigned long long am_wave_max(unsigned long long k) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const unsigned lo = __shfl_xor((unsigned)k, o, 64), hi = __shfl_xor((unsigned)(k >> 32), o, 64);
    k = am_max(k, ((unsigned long long)hi << 32) | lo);
  }
  return k;
}

constexpr int kAmParts = 128;         // partial keys per row (first pass workgroups per row)
constexpr int kAmMaxRows = 64;
// Library-owned partials of the two-pass argmax: each row's kAmParts keys. Every call on a device
// shares it (calls that overlap on one device race; stream-ordered calls do not).
__device__ unsigned long long g_am_part[kAmMaxRows * kAmParts];

template <bool BF16>
__global__ __launch_bounds__(256) void am_pass1(const void* __restrict__ x, long long row_stride, long long vocab) {
  const int row = blockIdx.y;
  const long long chunk = (vocab + kAmParts - 1) / kAmParts;
  const long long b = (long long)blockIdx.x * chunk, e = b + chunk < vocab ? b + chunk : vocab;
  unsigned long long k = 0;
  for (long long i = b + threadIdx.x; i < e; i += 256) {
    const float v = BF16 ? r4_bf16_to_f32(((const unsigned short*)x)[row * row_stride + i])
                         : ((const float*)x)[row * row_stride + i];
    k = am_max(k, am_key(v, (unsigned)i));
  }
  __shared__ unsigned long long red[4];
  k = am_wave_max(k);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = k;
  __syncthreads();
  if (threadIdx.x == 0) g_am_part[row * kAmParts + blockIdx.x] = am_max(am_max(red[0], red[1]), am_max(red[2], red[3]));
}

template <bool BF16>
__global__ __launch_bounds__(64) void am_pass2(const void* __restrict__ x, long long row_stride,
                                               int* __restrict__ out_idx, float* __restrict__ out_val,
                                               long long out_stride) {
  const int row = blockIdx.x;
  unsigned long long k = 0;
  for (int i = threadIdx.x; i < kAmParts; i += 64) k = am_max(k, g_am_part[row * kAmParts + i]);
  k = am_wave_max(k);
  if (threadIdx.x == 0) {
    int idx;
    float val;
    am_decode(k, &idx, &val);
    out_idx[row * out_stride] = idx;
    // the winner's own bits (a -0 stays -0); the seed's value when nothing beat it
    if (out_val)
      out_val[row * out_stride] = k < am_key(-__builtin_inff(), 0u) ? val
                                  : BF16 ? r4_bf16_to_f32(((const unsigned short*)x)[row * row_stride + idx])
                                         : ((const float*)x)[row * row_stride + idx];
  }
}

void am_run(bool bf16, int64_t x, int64_t row_stride, int64_t out_idx, int64_t out_val, int64_t out_stride,
            int64_t rows, int64_t vocab, int64_t stream, const char* entry) {
  if (rows < 1 || rows > kAmMaxRows) r4d::fail(entry, "rows must be 1..64");
  if (vocab < 1 || vocab > 0x7FFFFFFFLL) r4d::fail(entry, "vocab must be 1..2^31-1");
  if (!x || !out_idx) r4d::fail(entry, "null buffer");
  hipStream_t st = (hipStream_t)stream;
  if (bf16) hipLaunchKernelGGL(am_pass1<true>, dim3(kAmParts, (unsigned)rows), dim3(256), 0, st, (const void*)x,
                               (long long)row_stride, (long long)vocab);
  else hipLaunchKernelGGL(am_pass1<false>, dim3(kAmParts, (unsigned)rows), dim3(256), 0, st, (const void*)x,
                          (long long)row_stride, (long long)vocab);
  if (bf16) hipLaunchKernelGGL(am_pass2<true>, dim3((unsigned)rows), dim3(64), 0, st, (const void*)x,
                               (long long)row_stride, (int*)out_idx, (float*)out_val, (long long)out_stride);
  else hipLaunchKernelGGL(am_pass2<false>, dim3((unsigned)rows), dim3(64), 0, st, (const void*)x,
                          (long long)row_stride, (int*)out_idx, (float*)out_val, (long long)out_stride);
  r4d::launch_ok(entry);
}

}  // namespace

extern "C" {

// r4d.h:331-333: the build-default group (64). WV, SK, MB, NPW, NT are the reference's geometry knobs:
// accepted, not used.
void r4d_gemm_w4a16_nt_m64(int64_t a, int64_t wq, int64_t wsz, int64_t c, int M, int K, int N, int WV, int SK,
                           int MB, int NPW, int NT, int64_t stream) {
  (void)WV; (void)SK; (void)MB; (void)NPW; (void)NT;
  w4_run(64, a, wq, wsz, c, M, K, N, false, stream, "gemm_w4a16_nt_m64");
}
int r4d_gemm_w4a16_nt_m64_max_m(void) { return 64; }
int r4d_gemm_w4a16_nt_m64_group(void) { return 64; }
int r4d_gemm_w4a16_nt_m64_has_group(int group) { return group == 32 || group == 64; }
void r4d_gemm_w4a16_nt_m64_g(int group, int64_t a, int64_t wq, int64_t wsz, int64_t c, int M, int K, int N, int WV,
                             int SK, int MB, int NPW, int NT, int64_t stream) {
  (void)WV; (void)SK; (void)MB; (void)NPW; (void)NT;
  w4_run(group, a, wq, wsz, c, M, K, N, false, stream, "gemm_w4a16_nt_m64_g");
}
const char* r4d_gemm_w4a16_nt_m64_check(int group, int M, int K, int N) {
  return r4d::check_result(w4_check(group, M, K, N));
}
void r4d_gemm_w4a16_nt_m64_f32(int group, int64_t a, int64_t wq, int64_t wsz, int64_t c, int M, int K, int N,
                               int64_t stream) {
  w4_run(group, a, wq, wsz, c, M, K, N, true, stream, "gemm_w4a16_nt_m64_f32");
}

void r4dx_argmax_f32(int64_t logits, int64_t out_idx, int64_t vocab, int64_t stream) {
  am_run(false, logits, 0, out_idx, 0, 1, 1, vocab, stream, "argmax_f32");
}
void r4dx_argmax_val_f32(int64_t logits, int64_t out_idx, int64_t out_val, int64_t vocab, int64_t stream) {
  am_run(false, logits, 0, out_idx, out_val, 1, 1, vocab, stream, "argmax_val_f32");
}
void r4dx_argmax_bf16(int64_t logits, int64_t out_idx, int64_t vocab, int64_t stream) {
  am_run(true, logits, 0, out_idx, 0, 1, 1, vocab, stream, "argmax_bf16");
}
void r4dx_argmax_val_bf16(int64_t logits, int64_t out_idx, int64_t out_val, int64_t vocab, int64_t stream) {
  am_run(true, logits, 0, out_idx, out_val, 1, 1, vocab, stream, "argmax_val_bf16");
}
void r4dx_argmax_rows_f32(int64_t logits, int64_t row_stride, int64_t out_idx, int64_t out_val, int64_t out_stride,
                          int64_t rows, int64_t vocab, int64_t stream) {
  am_run(false, logits, row_stride, out_idx, out_val, out_stride, rows, vocab, stream, "argmax_rows_f32");
}

}  // extern "C"
