// trellis_i8.hip -- the int8 x int8 trellis prefill GEMM on gfx950: r4d_gemm_trellis_nt_i8 (per-128 scales) and
// r4d_gemm_trellis_nt_i8c (coarse scales), their weight scale tables (r4d_trellis_i8_wscale / _col), the int8 weight
// dumps (r4d_trellis_i8_dump_w / _col), _check and _ws_bytes: the C ABI of the reference's
// third_party/libr4d/r4d.h:456-521.
//
// C bf16 [256][N] = bf16((FWHT128(sum) * svh) * out_scale) with
//   per-128: sum = sum_kb float(int32(A8_kb . W8_kb)) * (sa[kb][row] * sw[kb][col])    (fp32, k-block order)
//   coarse:  sum = float(int32(A8 . W8 over the slice)) * (sa[row] * sw[col])
// where W8 is the decoded trellis weight Q quantized on the fly: rs = f16(min(1 / s_eff, 60000)) for the
// table's s_eff = 1 / rs, q = low byte of f16(w * rs + 1536) (one rounding: round(w * rs) lands in the
// low byte, the f16 spacing at 1536 being 1) -- the reference's rule (r4d_trellis_i8.h:129-151,
// tests/kernels/int8_gemm_proto_ref.h:57-77). The table: s = max|w| / 127 per (column, 128 k) or per column
// over K (1 for an all-zero group), rs as above, s_eff = 1 / rs (IEEE fp32).
//
// DESIGN (MI355X): v_mfma_i32_16x16x64_i8; a workgroup is 8 waves = 256 rows x one 128-column group x one K
// slice, in 64-k steps. Wave w owns rows 32 w .. 32 w + 31 (two row tiles of A8's row group w / 2) against
// all 8 column tiles; its A fragments come straight from the A8 layout (two 8-byte halves per lane, 128
// contiguous bytes per 16 lanes) through a register ring. B goes through a double-buffered 8 KiB LDS stage
// [k-tile][column][16 B]: the decode of the next step is shared out -- waves w and w + 4 take turns on tile
// pair w & 3 -- so every SIMD runs one decode and two waves' MFMAs per step. A decode lane's two fragment
// halves (element e of half h <-> k = 8 (e >> 2) + 4 h + (e & 3)) quantize, in that order, to exactly the
// 16 bytes an MFMA lane needs in A8's k order, so nothing is permuted. Unsplit, the FWHT-128 epilogue runs
// in registers (column bits 0-3 across lanes, 4-6 across column tiles); split K writes fp32 slices to ws
// and the split finish pass (trellis_m256.hip) adds them in order and runs the same epilogue.
#include "r4d_dev.h"
#include "r4d_host.h"
#include "r4d_mi355x.h"

namespace {

typedef __amdgpu_buffer_rsrc_t r4_rsrc;
__device__ __forceinline__ r4_rsrc mk_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ r4i4 mfma_i8(r4i4 a, r4i4 b, r4i4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// ---- the weight-side quantizer --------------------------------------------------------------------------
__device__ __forceinline__ float ti8_scale_from_amax(float amax) { return amax > 0.f ? amax / 127.0f : 1.0f; }
// rs as the f16 bits, duplicated into both halves; from s (the table builder) or from the table's s_eff
__device__ __forceinline__ unsigned ti8_rs_from_s(float s) {
  const _Float16 h = (_Float16)__builtin_fminf(1.0f / s, 60000.f);
  const unsigned b = __builtin_bit_cast(unsigned short, h);
  return b | (b << 16);
}
// The same rs from a table entry s_eff = 1 / rs (fp32) with the hardware reciprocal instead of the IEEE divide: rs is an
// f16 number in [1, 60000] and s_eff its correctly rounded reciprocal, so 1 / s_eff lies within an fp32 ulp of rs and
// any result within a few ulps converts back to rs (checked for every normal f16 up to 60000 at +-3 ulps).
__device__ __forceinline__ unsigned ti8_rs_from_seff(float seff) {
  const _Float16 h = (_Float16)__builtin_fminf(__builtin_amdgcn_rcpf(seff), 60000.f);
  const unsigned b = __builtin_bit_cast(unsigned short, h);
  return b | (b << 16);
}
// four f16 weights (two dwords, element order) -> four int8 bytes: low byte of f16(w * rs + 1536)
__device__ __forceinline__ unsigned ti8_q4(unsigned d0, unsigned d1, unsigned rs2) {
  const r4h2 c = {(_Float16)1536.f, (_Float16)1536.f};
  const r4h2 x0 = __builtin_elementwise_fma(__builtin_bit_cast(r4h2, d0), __builtin_bit_cast(r4h2, rs2), c);
  const r4h2 x1 = __builtin_elementwise_fma(__builtin_bit_cast(r4h2, d1), __builtin_bit_cast(r4h2, rs2), c);
  return __builtin_amdgcn_perm(__builtin_bit_cast(unsigned, x1), __builtin_bit_cast(unsigned, x0), 0x06040200u);
}
// max |w| over the lane's 16 values of column slot cs (fp32; exact)
__device__ __forceinline__ float ti8_amax16(const unsigned (&d)[2][2][4], int cs) {
  float m = 0.f;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const r4h2 v = __builtin_bit_cast(r4h2, d[cs][h][j]);
      m = __builtin_fmaxf(m, __builtin_fmaxf(__builtin_fabsf((float)v[0]), __builtin_fabsf((float)v[1])));
    }
  return m;
}

// The decode lane map of one (tile pair, 4 k-tiles) step (the GEMV's): lane q = l >> 4 takes k-tile q, t =
// (l >> 3) & 1 and c = l & 7 the columns 32 pair + 16 t + 8 cs + c (cs = 0, 1).
template <int KB>
struct TileWords {
  r4_rsrc r;
  unsigned own;   // the history word comes from lane c - 1 (r4_hist_word)
  __device__ __forceinline__ TileWords(const unsigned* W, int pair, int KT, int kt0, int ktw, int lane) {
    constexpr int BLK = 16 * KB;
    r = mk_rsrc(W + ((size_t)pair * KT + kt0) * BLK, (unsigned)ktw * BLK * 4u);
    const int q = lane >> 4, t = (lane >> 3) & 1, c = lane & 7;
    const unsigned tile = (unsigned)(q * 16 * KB + t * 8 * KB);
    own = (tile + KB * c) * 4u;
  }
  __device__ __forceinline__ void load(unsigned (&w)[KB + 1], int st) const {
    const unsigned so = (unsigned)st * (4u * 16u * KB * 4u);
    // one wide load per lane (dword alignment suffices): KB 4 a dwordx4, KB 5 a dwordx4 and a dword
    if constexpr (KB == 4 || KB == 5) {
      const r4u4 v = __builtin_bit_cast(r4u4, __builtin_amdgcn_raw_buffer_load_b128(r, own + so, 0, 0));
      w[1] = v[0]; w[2] = v[1]; w[3] = v[2]; w[4] = v[3];
      if constexpr (KB == 5) w[5] = __builtin_amdgcn_raw_buffer_load_b32(r, own + so + 16, 0, 0);
    } else {
#pragma unroll
      for (int i = 0; i < KB; ++i) w[1 + i] = __builtin_amdgcn_raw_buffer_load_b32(r, own + so + 4 * i, 0, 0);
    }
  }
};

// ---- the scale table: one wave per (tile pair, K range); COL: the range is the whole K ----------------------
template <int KB, bool COL>
__global__ __launch_bounds__(64) void ti8_wscale_kernel(const unsigned* __restrict__ W, float* __restrict__ sw, int K,
                                                        int N) {
  const int lane = threadIdx.x, pair = blockIdx.x, kb = blockIdx.y;
  const int KT = K >> 4;
  const int kt0 = COL ? 0 : kb * 8, ktw = COL ? KT : 8;
  const TileWords<KB> tw(W, pair, KT, kt0, ktw, lane);
  float m[2] = {0.f, 0.f};
  for (int st = 0; st < ktw / 4; ++st) {
    unsigned w[KB + 1], d[2][2][4];
    tw.load(w, st);
    w[0] = r4_hist_word(w[KB], lane);
    r4_decode<KB>(w, d);
    m[0] = __builtin_fmaxf(m[0], ti8_amax16(d, 0));
    m[1] = __builtin_fmaxf(m[1], ti8_amax16(d, 1));
  }
#pragma unroll
  for (int cs = 0; cs < 2; ++cs) {
    m[cs] = __builtin_fmaxf(m[cs], __shfl_xor(m[cs], 16, 64));
    m[cs] = __builtin_fmaxf(m[cs], __shfl_xor(m[cs], 32, 64));
  }
  if (lane < 16) {
    const int t = (lane >> 3) & 1, c = lane & 7;
#pragma unroll
    for (int cs = 0; cs < 2; ++cs) {
      const unsigned rs = ti8_rs_from_s(ti8_scale_from_amax(m[cs])) & 0xFFFFu;
      const float seff = 1.0f / (float)__builtin_bit_cast(_Float16, (unsigned short)rs);
      sw[(size_t)(COL ? 0 : kb) * N + 32 * pair + 16 * t + 8 * cs + c] = seff;
    }
  }
}

// ---- the int8 weights the GEMM uses: W8 block layout (w8) and, if wp, plain [N][K] --------------------------
template <int KB, bool COL>
__global__ __launch_bounds__(64) void ti8_dump_kernel(const unsigned* __restrict__ W, const float* __restrict__ sw,
                                                      unsigned char* __restrict__ w8, signed char* __restrict__ wp,
                                                      int K, int N) {
  const int lane = threadIdx.x, pair = blockIdx.x, st = blockIdx.y;   // one step = 4 k-tiles
  const int KT = K >> 4;
  const TileWords<KB> tw(W, pair, KT, 0, KT, lane);
  unsigned w[KB + 1], d[2][2][4];
  tw.load(w, st);
  w[0] = r4_hist_word(w[KB], lane);
  r4_decode<KB>(w, d);
  const int q = lane >> 4, t = (lane >> 3) & 1, c = lane & 7;
  const int kt = 4 * st + q, kb = kt >> 3;
#pragma unroll
  for (int cs = 0; cs < 2; ++cs) {
    const int n = 32 * pair + 16 * t + 8 * cs + c;
    const unsigned rs2 = ti8_rs_from_s(sw[(size_t)(COL ? 0 : kb) * N + n]);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const unsigned lo = ti8_q4(d[cs][h][0], d[cs][h][1], rs2), hi = ti8_q4(d[cs][h][2], d[cs][h][3], rs2);
      const int L = 16 * h + 8 * t + c;   // r4d_trellis_i8_layout.h:56-64 W8Offset's lane
      *(r4u2*)(w8 + ((size_t)pair * KT + kt) * 512 + L * 16 + cs * 8) = (r4u2){lo, hi};
      if (wp) {   // element e <-> k = 8 (e >> 2) + 4 h + (e & 3)
        *(unsigned*)(wp + (size_t)n * K + 16 * kt + 4 * h) = lo;
        *(unsigned*)(wp + (size_t)n * K + 16 * kt + 8 + 4 * h) = hi;
      }
    }
  }
}

// ---- the GEMM ---------------------------------------------------------------------------------------------
// SC: the scale mode. kSCoarse -- one int32 sum per slice, times sa[row] * sw[col] once; kSABlk -- per 128-k
// block acc += float(int32) * sa[kb][row], times sw[col] at the end (the dense per-128 activation variant);
// kSBlk -- per block acc += float(int32) * (sa[kb][row] * sw[kb][col]) (the trellis per-128 mode).
// OUT: kOutBf16 -- FWHT-128, svh, out_scale, bf16 (the trellis entries); kOutF16 -- plain f16; kOutI32 -- the
// exact int32 sums (test entry). DENSE: B is int8 in the W8 block layout instead of trellis words.
constexpr int kSCoarse = 0, kSABlk = 1, kSBlk = 2;
constexpr int kOutBf16 = 0, kOutF16 = 1, kOutI32 = 2;

struct TI8Args {
  const signed char* a8[2];
  const float* sa[2];
  int n_split;
  const void* w;        // trellis words or W8 bytes
  const float* sw;
  const float* svh;
  void* c;
  float* ws;
  int K, N, SKG;
  float out_scale;
  // stream-K (G > 0): G workgroups share the U = (N / 128) (K / 128) (column group, 128-k block) units
  // evenly; partial pieces of a group go to ws slot 2 c + (first group of c ? 0 : 1) and the last piece to
  // arrive (ticket) adds all of them in piece order, then finishes the group
  int G, U;
  unsigned* tickets;
};
constexpr int kStreamG = 256;                   // workgroups of a stream-K launch (one per CU)
constexpr int kSlot = 256 * 128;                // values per partial piece

// the B stage's column slot: bit 3 flipped on odd 16-column tiles (a decode lane writes columns 16 t + 8 cs +
// c of its pair: the t = 0 and t = 1 lanes of one write then use different banks)
__device__ __forceinline__ int ti8_bslot(int n) { return n ^ (((n >> 4) & 1) << 3); }

// the last workgroup c whose stream-K range [floor(c U / G), ...) starts at or before unit x
__device__ __forceinline__ int ti8_unit_owner(int x, int U, int G) {
  return (int)((((long long)x + 1) * G + U - 1) / U) - 1;
}

// One piece: column group `group`, k-tiles kt0 .. kt0 + 4 nst of it. slot < 0: the whole group's K range
// (or a classic split slice ky); slot >= 0: a stream-K partial piece (see TI8Args).
template <int KB, int SC, int OUT, bool DENSE>
__device__ __forceinline__ void ti8_piece(const TI8Args& p, unsigned char (*bst)[4][128][16], int* flag, int group,
                                          int ky, int kt0, int nst, int slot) {
  constexpr bool BLKA = SC != kSCoarse;           // per-128 activation scales: fp32 accumulators
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int K = p.K, N = p.N, KT = K >> 4;
  const int ktw = 4 * nst;
  const int n0 = group * 128;
  const int part = (p.a8[1] != nullptr && n0 >= p.n_split) ? 1 : 0;
  const int g = lane >> 4, r16 = lane & 15;

  // ---- B. Trellis: waves w and w + 4 take turns (steps of parity w >> 2) at decoding pair w & 3. Dense: every
  // wave copies its 1 KiB of the step's W8 blocks -- pair w >> 1, k-tiles 2 (w & 1) + (lane >> 5) -- every step.
  const int dpair = group * 4 + (wave & 3), dpar = wave >> 2;
  const TileWords<KB> tw((const unsigned*)p.w, dpair, KT, kt0, ktw, lane);
  const int dq = lane >> 4, dt = (lane >> 3) & 1, dc = lane & 7;
  const r4_rsrc wr8 = mk_rsrc(p.w, (unsigned)N * (unsigned)K);
  const int wpp = wave >> 1, wkt = 2 * (wave & 1) + (lane >> 5), wL = lane & 31;
  const unsigned w8base = ((unsigned)((group * 4 + wpp) * KT + kt0 + wkt)) * 512u + (unsigned)wL * 16u;
  // rs of the decode lane's two columns: coarse -- fixed for the launch; per-128 -- from the ring's s_eff
  unsigned rsc[2] = {0u, 0u};
  if constexpr (!DENSE && SC != kSBlk) {
#pragma unroll
    for (int cs = 0; cs < 2; ++cs) rsc[cs] = ti8_rs_from_s(p.sw[n0 + 32 * (wave & 3) + 16 * dt + 8 * cs + dc]);
  }
  auto put = [&](const unsigned (&w)[KB + 1], const float (&dsw)[2], const r4u4& wb, int st) {
    if constexpr (DENSE) {
      // W8 lane L = 16 h + 8 t + c holds fragment F0 then F1: columns 32 pair + 16 t + 8 F + c, k-half h
      const int h = wL >> 4, t = (wL >> 3) & 1, c = wL & 7;
      const int nl = 32 * wpp + 16 * t + c;
      *(r4u2*)&bst[st & 1][wkt][ti8_bslot(nl)][8 * h] = (r4u2){wb[0], wb[1]};
      *(r4u2*)&bst[st & 1][wkt][ti8_bslot(nl + 8)][8 * h] = (r4u2){wb[2], wb[3]};
    } else {
      unsigned d[2][2][4], wl[KB + 1];
      wl[0] = r4_hist_word(w[KB], lane);
#pragma unroll
      for (int i = 1; i <= KB; ++i) wl[i] = w[i];
      r4_decode<KB>(wl, d);
#pragma unroll
      for (int cs = 0; cs < 2; ++cs) {
        const int nl = 32 * (wave & 3) + 16 * dt + 8 * cs + dc;
        const unsigned rs2 = SC == kSBlk ? ti8_rs_from_seff(dsw[cs]) : rsc[cs];
        const r4u4 v = {ti8_q4(d[cs][0][0], d[cs][0][1], rs2), ti8_q4(d[cs][0][2], d[cs][0][3], rs2),
                        ti8_q4(d[cs][1][0], d[cs][1][1], rs2), ti8_q4(d[cs][1][2], d[cs][1][3], rs2)};
        *(r4u4*)&bst[st & 1][dq][ti8_bslot(nl)][0] = v;
      }
    }
  };
  auto load_b = [&](unsigned (&w)[KB + 1], float (&dsw)[2], r4u4& wb, int st) {
    if constexpr (DENSE) {
      wb = __builtin_bit_cast(r4u4, __builtin_amdgcn_raw_buffer_load_b128(wr8, w8base + (unsigned)st * 2048u, 0, 0));
    } else {
      tw.load(w, st);
      if constexpr (SC == kSBlk) {
        const int kb = (kt0 + 4 * st) >> 3;
#pragma unroll
        for (int cs = 0; cs < 2; ++cs) dsw[cs] = p.sw[(size_t)kb * N + n0 + 32 * (wave & 3) + 16 * dt + 8 * cs + dc];
      }
    }
  };

  // ---- this wave's A: rows 32 w + 16 ii + r16 = row group rg, row tiles i0, i0 + 1
  const int rg = wave >> 1, i0 = 2 * (wave & 1);
  const r4_rsrc ar = mk_rsrc(p.a8[part], 256u * (unsigned)K);
  const unsigned abase = ((unsigned)(rg * KT + kt0 + g) * 4u + (unsigned)i0) * 256u + (unsigned)r16 * 8u;
  const float* SA = p.sa[part];
  struct St {
    r4u2 a[2][2];
    unsigned w[KB + 1];   // trellis: the words of step st + 1 (what this wave decodes after step st's barrier)
    float dsw[2];         // trellis per-128: their columns' s_eff
    r4u4 wb;              // dense: this wave's W8 bytes of step st + 1
    r4f4 sa[2];           // per-128, odd steps: sa[kb][rows of the two row tiles]
    float sw[8];          // kSBlk, odd steps: sw[kb][column of each column tile]
  };
  auto load = [&](St& s, int st, bool odd) {
    const int sc = min(st, nst - 1);
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        s.a[ii][h] = __builtin_bit_cast(
            r4u2, __builtin_amdgcn_raw_buffer_load_b64(ar, abase + (unsigned)sc * 4096u + ii * 256u + h * 128u, 0, 0));
    load_b(s.w, s.dsw, s.wb, min(sc + 1, nst - 1));
    if constexpr (BLKA) {
      if (odd) {
        const int kb = (kt0 + 4 * sc) >> 3;
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) s.sa[ii] = *(const r4f4*)(SA + (size_t)kb * 256 + 32 * wave + 16 * ii + 4 * g);
        if constexpr (SC == kSBlk) {
#pragma unroll
          for (int ct = 0; ct < 8; ++ct) s.sw[ct] = p.sw[(size_t)kb * N + n0 + 16 * ct + r16];
        }
      }
    }
  };

  r4i4 iacc[2][8];
  r4f4 facc[BLKA ? 2 : 1][8];
#pragma unroll
  for (int ii = 0; ii < 2; ++ii)
#pragma unroll
    for (int ct = 0; ct < 8; ++ct) {
      iacc[ii][ct] = (r4i4){0, 0, 0, 0};
      if constexpr (BLKA) facc[ii][ct] = (r4f4){0.f, 0.f, 0.f, 0.f};
    }

  auto step = [&](const St& s, int st, bool odd) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();                 // stage st landed; stage st + 1 free
    if (st + 1 < nst && (DENSE || ((st + 1) & 1) == dpar)) put(s.w, s.dsw, s.wb, st + 1);
    const unsigned char* stg = &bst[st & 1][g][0][0];
    r4i4 a[2];
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
      a[ii] = (r4i4){(int)s.a[ii][0].x, (int)s.a[ii][0].y, (int)s.a[ii][1].x, (int)s.a[ii][1].y};
#pragma unroll
    for (int ct = 0; ct < 8; ++ct) {
      const r4i4 b = *(const r4i4*)(stg + ti8_bslot(16 * ct + r16) * 16);
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)   // per-128: a block's first step starts its int32 sums from 0 (the MFMA's C)
        iacc[ii][ct] = mfma_i8(a[ii], b, (BLKA && !odd) ? (r4i4){0, 0, 0, 0} : iacc[ii][ct]);
    }
    if constexpr (BLKA) {
      if (odd) {   // the 128-k block is complete: acc += float(int32) * scale
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int ct = 0; ct < 8; ++ct)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float sc = SC == kSBlk ? s.sa[ii][j] * s.sw[ct] : s.sa[ii][j];
              facc[ii][ct][j] = __builtin_fmaf((float)iacc[ii][ct][j], sc, facc[ii][ct][j]);
            }
      }
    }
  };

  // prologue: the waves that stage step 0 do so before the first barrier
  {
    unsigned w0[KB + 1];
    float d0[2] = {0.f, 0.f};
    r4u4 b0 = {0u, 0u, 0u, 0u};
    load_b(w0, d0, b0, 0);
    if (nst > 0 && (DENSE || dpar == 0)) put(w0, d0, b0, 0);
  }
  // statically indexed ring; PF even, so slot i always carries steps of parity i (a 128-k block = 2 steps);
  // deeper where the registers allow (the per-128 modes hold fp32 and int32 accumulators)
  constexpr int PF = BLKA ? 2 : 4;
  St ring[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) load(ring[i], i, (i & 1) != 0);
  int st = 0;
  for (; st + PF <= nst; st += PF) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      step(ring[i], st + i, (i & 1) != 0);
      load(ring[i], st + i + PF, (i & 1) != 0);
    }
  }
#pragma unroll
  for (int i = 0; i < PF - 1; ++i)
    if (st + i < nst) step(ring[i], st + i, (i & 1) != 0);

  // ---- stream-K partial piece (dense launches only): store it, take the group's ticket; the last piece adds
  // all pieces in order
  if (DENSE && slot >= 0) {
    const int nb = K >> 7;
    const int c_lo = ti8_unit_owner(group * nb, p.U, p.G), c_hi = ti8_unit_owner((group + 1) * nb - 1, p.U, p.G);
    auto slot_of = [&](int c) {
      const int first = (int)((long long)c * p.U / p.G) / nb;
      return 2 * c + (group == first ? 0 : 1);
    };
    // int32 pieces (coarse) and fp32 pieces (per-128) each through their own typed path
    auto idx = [&](int ii, int ct, int j) { return (((wave * 2 + ii) * 8 + ct) * 4 + j) * 64 + lane; };
    if constexpr (BLKA) {
      float* dst = p.ws + (size_t)slot * kSlot;
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int ct = 0; ct < 8; ++ct)
#pragma unroll
          for (int j = 0; j < 4; ++j) r4_store_coherent(&dst[idx(ii, ct, j)], facc[ii][ct][j]);
    } else {
      int* dst = (int*)p.ws + (size_t)slot * kSlot;
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int ct = 0; ct < 8; ++ct)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            __hip_atomic_store(&dst[idx(ii, ct, j)], iacc[ii][ct][j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!r4_ticket_last(&p.tickets[group], (unsigned)(c_hi - c_lo + 1), flag)) return;
    for (int c = c_lo; c <= c_hi; ++c) {
      if constexpr (BLKA) {
        const float* src = p.ws + (size_t)slot_of(c) * kSlot;
        float t[2][8][4];
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int ct = 0; ct < 8; ++ct)
#pragma unroll
            for (int j = 0; j < 4; ++j) t[ii][ct][j] = r4_load_coherent(&src[idx(ii, ct, j)]);
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int ct = 0; ct < 8; ++ct)
#pragma unroll
            for (int j = 0; j < 4; ++j) facc[ii][ct][j] = c == c_lo ? t[ii][ct][j] : facc[ii][ct][j] + t[ii][ct][j];
      } else {
        const int* src = (const int*)p.ws + (size_t)slot_of(c) * kSlot;
        int t[2][8][4];
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int ct = 0; ct < 8; ++ct)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              t[ii][ct][j] = __hip_atomic_load(&src[idx(ii, ct, j)], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int ct = 0; ct < 8; ++ct)
#pragma unroll
            for (int j = 0; j < 4; ++j) iacc[ii][ct][j] = (c == c_lo ? 0 : iacc[ii][ct][j]) + t[ii][ct][j];
      }
    }
  }

  // ---- this slice's values: rows 32 w + 16 ii + 4 g + j, column n0 + 16 ct + r16
  if constexpr (OUT == kOutI32) {
    if (p.SKG > 1) {
      int* dst = (int*)p.ws + (size_t)ky * 256 * N;
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int ct = 0; ct < 8; ++ct)
            dst[(size_t)(32 * wave + 16 * ii + 4 * g + j) * N + n0 + 16 * ct + r16] = iacc[ii][ct][j];
    } else {
      int* C = (int*)p.c;
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int ct = 0; ct < 8; ++ct)
            C[(size_t)(32 * wave + 16 * ii + 4 * g + j) * N + n0 + 16 * ct + r16] = iacc[ii][ct][j];
    }
    return;
  } else {
    float v[2][8][4];
    float swc[8];
#pragma unroll
    for (int ct = 0; ct < 8; ++ct) swc[ct] = SC == kSBlk ? 1.f : p.sw[n0 + 16 * ct + r16];
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      r4f4 sav = (r4f4){1.f, 1.f, 1.f, 1.f};
      if constexpr (SC == kSCoarse) sav = *(const r4f4*)(SA + 32 * wave + 16 * ii + 4 * g);
#pragma unroll
      for (int ct = 0; ct < 8; ++ct)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (SC == kSCoarse) v[ii][ct][j] = (float)iacc[ii][ct][j] * (sav[j] * swc[ct]);
          else if constexpr (SC == kSABlk) v[ii][ct][j] = facc[ii][ct][j] * swc[ct];
          else v[ii][ct][j] = facc[ii][ct][j];
        }
    }
    if (p.SKG > 1) {
      float* dst = p.ws + (size_t)ky * 256 * N;
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int ct = 0; ct < 8; ++ct) dst[(size_t)(32 * wave + 16 * ii + 4 * g + j) * N + n0 + 16 * ct + r16] = v[ii][ct][j];
      return;
    }
    if constexpr (OUT == kOutF16) {
      unsigned short* C = (unsigned short*)p.c;
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int ct = 0; ct < 8; ++ct)
            C[(size_t)(32 * wave + 16 * ii + 4 * g + j) * N + n0 + 16 * ct + r16] =
                __builtin_bit_cast(unsigned short, (_Float16)v[ii][ct][j]);
      return;
    } else {
      // FWHT-128 over the group's columns, stages lg = 0..6 in order (the lower index keeps a + b, the upper
      // takes a - b): bits 0-3 are lane bits 0-3, bits 4-6 the column tile ct
      unsigned short* C = (unsigned short*)p.c;
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float x[8];
#pragma unroll
          for (int ct = 0; ct < 8; ++ct) x[ct] = v[ii][ct][j];
#pragma unroll
          for (int mask = 1; mask <= 8; mask <<= 1) {
            const bool upper = (lane & mask) != 0;
#pragma unroll
            for (int ct = 0; ct < 8; ++ct) {
              const float o = r4_xor_lane(x[ct], mask);
              x[ct] = upper ? o - x[ct] : x[ct] + o;
            }
          }
#pragma unroll
          for (int b = 1; b <= 4; b <<= 1)
#pragma unroll
            for (int ct = 0; ct < 8; ++ct)
              if ((ct & b) == 0) {
                const float a0 = x[ct], b0 = x[ct | b];
                x[ct] = a0 + b0;
                x[ct | b] = a0 - b0;
              }
          const int r = 32 * wave + 16 * ii + 4 * g + j;
#pragma unroll
          for (int ct = 0; ct < 8; ++ct) {
            const int n = n0 + 16 * ct + r16;
            C[(size_t)r * N + n] = r4_bf16_rn((x[ct] * p.svh[n]) * p.out_scale);
          }
        }
    }
  }
}

template <int KB, int SC, int OUT, bool DENSE>
__global__ __launch_bounds__(512, 1) void ti8_gemm_kernel(TI8Args p) {
  __shared__ __attribute__((aligned(16))) unsigned char bst[2][4][128][16];   // [stage][k-tile][column slot][16 B]
  __shared__ int flag;
  if (!DENSE || p.G == 0) {
    const int ktw = (p.K >> 4) / p.SKG;
    ti8_piece<KB, SC, OUT, DENSE>(p, bst, &flag, blockIdx.x, blockIdx.y, blockIdx.y * ktw, ktw >> 2, -1);
    return;
  }
  // stream-K: this workgroup's units [u0, u1), a unit = (group, 128-k block) = 2 steps
  const int c = blockIdx.x, nb = p.K >> 7;
  const int u0 = (int)((long long)c * p.U / p.G), u1 = (int)((long long)(c + 1) * p.U / p.G);
  const int first = u0 / nb;
  for (int g = first; g * nb < u1; ++g) {
    const int b0 = max(u0, g * nb) - g * nb, b1 = min(u1, (g + 1) * nb) - g * nb;
    const bool whole = b0 == 0 && b1 == nb;
    ti8_piece<KB, SC, OUT, DENSE>(p, bst, &flag, g, 0, 8 * b0, 2 * (b1 - b0), whole ? -1 : 2 * c + (g == first ? 0 : 1));
    __syncthreads();   // the next piece restages the LDS
  }
}

// The second pass of a split dense launch: the SKG slices of ws added in slice order (as integers for the
// int32 test entry), then stored as f16 (or int32).
template <int OUT>
__global__ __launch_bounds__(256) void ti8_finish_kernel(const void* __restrict__ ws, void* __restrict__ c, int M,
                                                         int N, int SKG) {
  const long long id = (long long)blockIdx.x * 256 + threadIdx.x;
  if (id >= (long long)M * N) return;
  const size_t sy = (size_t)M * N;
  if constexpr (OUT == kOutI32) {
    int acc = 0;
    for (int y = 0; y < SKG; ++y) acc += ((const int*)ws)[y * sy + id];
    ((int*)c)[id] = acc;
  } else {
    float acc = ((const float*)ws)[id];
    for (int y = 1; y < SKG; ++y) acc += ((const float*)ws)[y * sy + id];
    ((unsigned short*)c)[id] = __builtin_bit_cast(unsigned short, (_Float16)acc);
  }
}

std::string ti8_check(int M, int K, int N, int n_split, int KB, int skw, int skg) {
  using r4d::str;
  if (M != 256) return "M must be 256";
  if (K <= 0 || N <= 0 || K % 128 || N % 128) return "K and N must be positive multiples of 128";
  if (n_split < 0 || n_split > N || n_split % 128) return "n_split must be in 0..N and a multiple of 128";
  if (KB != 4 && KB != 5) return "KB " + str(KB) + " is not instantiated (4, 5)";
  if (skw != 2 && skw != 4 && skw != 8) return "skw must be 2, 4 or 8";
  if (skg != 1 && skg != 2 && skg != 4 && skg != 8) return "skg must be 1, 2, 4 or 8";
  if ((K / 128) % (skw * skg)) return "(K / 128) must be divisible by skw * skg";
  if ((long long)256 * K >= (1LL << 32)) return "256 K must be below 2^32 bytes";
  // a split launch's fp32 slices go through the prefill GEMM's finish, which addresses them with 32-bit offsets
  if (skg > 1 && (long long)skg * 256 * N * 4 > (1LL << 31))
    return "the fp32 slices skg * 256 * N * 4 bytes must fit 2 GiB (32-bit offsets of the split finish): lower skg";
  return "";
}

template <int KB, int SC, int OUT, bool DENSE>
void ti8_launch(const TI8Args& a, int N, int SKG, hipStream_t st) {
  if (a.G > 0) hipLaunchKernelGGL((ti8_gemm_kernel<KB, SC, OUT, DENSE>), dim3(a.G), dim3(512), 0, st, a);
  else hipLaunchKernelGGL((ti8_gemm_kernel<KB, SC, OUT, DENSE>), dim3(N / 128, SKG), dim3(512), 0, st, a);
}

void ti8_run(bool p128, int64_t a8_0, int64_t sa_0, int64_t a8_1, int64_t sa_1, int n_split, int64_t w, int64_t sw,
             int64_t svh, int64_t c, int64_t ws, int64_t tickets, int M, int K, int N, int KB, int skw, int skg,
             float out_scale, int64_t stream, const char* entry) {
  (void)tickets;
  r4d::require(entry, ti8_check(M, K, N, n_split, KB, skw, skg));
  if (!a8_0 || !sa_0 || !w || !sw || !svh || !c) r4d::fail(entry, "null A8, SA, W, SW, svh or C");
  if (a8_1 && !sa_1) r4d::fail(entry, "a8_1 without sa_1");
  if (!a8_1 && n_split != N) r4d::fail(entry, "a one-part launch (a8_1 = 0) needs n_split = N");
  if (skg > 1 && !ws) r4d::fail(entry, "skg > 1 needs ws");
  TI8Args a{};
  a.a8[0] = (const signed char*)a8_0;
  a.a8[1] = (const signed char*)a8_1;
  a.sa[0] = (const float*)sa_0;
  a.sa[1] = a8_1 ? (const float*)sa_1 : (const float*)sa_0;
  a.n_split = n_split;
  a.w = (const void*)w;
  a.sw = (const float*)sw;
  a.svh = (const float*)svh;
  a.c = (void*)c;
  a.ws = (float*)ws;
  a.K = K;
  a.N = N;
  a.SKG = skg;
  a.out_scale = out_scale;
  hipStream_t st = (hipStream_t)stream;
  if (KB == 4) {
    if (p128) ti8_launch<4, kSBlk, kOutBf16, false>(a, N, skg, st);
    else ti8_launch<4, kSCoarse, kOutBf16, false>(a, N, skg, st);
  } else {
    if (p128) ti8_launch<5, kSBlk, kOutBf16, false>(a, N, skg, st);
    else ti8_launch<5, kSCoarse, kOutBf16, false>(a, N, skg, st);
  }
  if (skg > 1) r4d::launch_split_finish(a.ws, a.svh, a.c, M, N, skg, 1, out_scale, st);
  r4d::launch_ok(entry);
}

void ti8_table(bool col, int64_t w, int64_t sw, int K, int N, int KB, int64_t stream, const char* entry) {
  if (K <= 0 || N <= 0 || K % 128 || N % 128) r4d::fail(entry, "K and N must be positive multiples of 128");
  if (KB != 4 && KB != 5) r4d::fail(entry, "KB must be 4 or 5");
  if (!w || !sw) r4d::fail(entry, "null buffer");
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid(N / 32, col ? 1 : K / 128);
  auto W = (const unsigned*)w;
  auto S = (float*)sw;
  if (KB == 4) {
    if (col) hipLaunchKernelGGL((ti8_wscale_kernel<4, true>), grid, dim3(64), 0, st, W, S, K, N);
    else hipLaunchKernelGGL((ti8_wscale_kernel<4, false>), grid, dim3(64), 0, st, W, S, K, N);
  } else {
    if (col) hipLaunchKernelGGL((ti8_wscale_kernel<5, true>), grid, dim3(64), 0, st, W, S, K, N);
    else hipLaunchKernelGGL((ti8_wscale_kernel<5, false>), grid, dim3(64), 0, st, W, S, K, N);
  }
  r4d::launch_ok(entry);
}

void ti8_dump(bool col, int64_t w, int64_t sw, int64_t w8, int64_t wp, int K, int N, int KB, int64_t stream,
              const char* entry) {
  if (K <= 0 || N <= 0 || K % 128 || N % 128) r4d::fail(entry, "K and N must be positive multiples of 128");
  if (KB != 4 && KB != 5) r4d::fail(entry, "KB must be 4 or 5");
  if (!w || !sw || !w8) r4d::fail(entry, "null buffer");
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid(N / 32, K / 64);
  auto W = (const unsigned*)w;
  auto S = (const float*)sw;
  auto B = (unsigned char*)w8;
  auto P = (signed char*)wp;
  if (KB == 4) {
    if (col) hipLaunchKernelGGL((ti8_dump_kernel<4, true>), grid, dim3(64), 0, st, W, S, B, P, K, N);
    else hipLaunchKernelGGL((ti8_dump_kernel<4, false>), grid, dim3(64), 0, st, W, S, B, P, K, N);
  } else {
    if (col) hipLaunchKernelGGL((ti8_dump_kernel<5, true>), grid, dim3(64), 0, st, W, S, B, P, K, N);
    else hipLaunchKernelGGL((ti8_dump_kernel<5, false>), grid, dim3(64), 0, st, W, S, B, P, K, N);
  }
  r4d::launch_ok(entry);
}

// ---- the dense int8 GEMM (W8 block layout weights) --------------------------------------------------------
std::string dense_check(int M, int K, int N, int SKG) {
  if (M != 256) return "M must be 256 (the prefill chunk)";
  if (K <= 0 || N <= 0 || K % 128 || N % 128) return "K and N must be positive multiples of 128";
  if ((long long)N * K >= (1LL << 32)) return "N K must be below 2^32 bytes";
  if (SKG < 0 || SKG > 64 || (SKG > 0 && (K / 128) % SKG)) return "SKG must be 0 (stream-K) or 1..64 dividing K / 128";
  return "";
}

void dense_run(int64_t a8, int64_t sa, int64_t w8, int64_t sw, int64_t c, int64_t ws, int64_t tickets, int M, int K,
               int N, int SKG, int scale_mode, bool raw_i32, int64_t stream, const char* entry) {
  r4d::require(entry, dense_check(M, K, N, SKG));
  if (scale_mode < 0 || scale_mode > 2) r4d::fail(entry, "scale_mode must be 0 (row / column), 1 (per-128 "
                                                         "activation, column weight) or 2 (per-128 both)");
  if (!a8 || !w8 || !c || (!raw_i32 && (!sa || !sw))) r4d::fail(entry, "null buffer");
  if (SKG > 1 && !ws) r4d::fail(entry, "a split launch (SKG > 1) needs ws");
  if (SKG == 0 && (!ws || !tickets)) r4d::fail(entry, "a stream-K launch (SKG = 0) needs ws and tickets");
  TI8Args a{};
  a.a8[0] = (const signed char*)a8;
  a.sa[0] = a.sa[1] = (const float*)sa;
  a.n_split = N;
  a.w = (const void*)w8;
  a.sw = (const float*)sw;
  a.c = (void*)c;
  a.ws = (float*)ws;
  a.K = K;
  a.N = N;
  a.SKG = SKG == 0 ? 1 : SKG;
  a.out_scale = 1.f;
  if (SKG == 0) {
    a.U = (N / 128) * (K / 128);
    a.G = a.U < kStreamG ? a.U : kStreamG;
    a.tickets = (unsigned*)tickets;
  }
  hipStream_t st = (hipStream_t)stream;
  if (raw_i32) ti8_launch<4, kSCoarse, kOutI32, true>(a, N, SKG, st);
  else if (scale_mode == 0) ti8_launch<4, kSCoarse, kOutF16, true>(a, N, SKG, st);
  else if (scale_mode == 1) ti8_launch<4, kSABlk, kOutF16, true>(a, N, SKG, st);
  else ti8_launch<4, kSBlk, kOutF16, true>(a, N, SKG, st);
  if (SKG > 1) {
    const long long n = (long long)M * N;
    if (raw_i32)
      hipLaunchKernelGGL(ti8_finish_kernel<kOutI32>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                         (const void*)ws, (void*)c, M, N, SKG);
    else
      hipLaunchKernelGGL(ti8_finish_kernel<kOutF16>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                         (const void*)ws, (void*)c, M, N, SKG);
  }
  r4d::launch_ok(entry);
}

}  // namespace

extern "C" {

const char* r4d_gemm_i8_dense_check(int M, int K, int N, int SKG) { return r4d::check_result(dense_check(M, K, N, SKG)); }
size_t r4d_gemm_i8_dense_ws_bytes(int M, int N, int SKG) {
  if (SKG == 0) return (size_t)kStreamG * 2 * kSlot * 4;   // stream-K: two partial-piece slots per workgroup
  return SKG > 1 ? (size_t)SKG * M * N * 4 : 0;
}
// The dense int8 GEMM: a8 in the A8 layout (r4d_trellis_i8_quant_act / _row), w8 in the W8 block layout
// (r4d_i8_pack_w), C f16 [256][N]. scale_mode 0: sa [256], sw [N]; 1: sa [K/128][256], sw [N]; 2: sa
// [K/128][256], sw [K/128][N]. SKG > 1: K split into SKG slices (ws, a second pass adds them); SKG = 0:
// stream-K over 256 workgroups (ws ws_bytes(M, N, 0), tickets u32 [N/128] zero before the first call and
// self-resetting; int32 sums are exact in any order, the per-128 modes add pieces in a fixed order).
void r4d_gemm_i8_dense(int64_t a8, int64_t sa, int64_t w8, int64_t sw, int64_t c, int64_t ws, int64_t tickets, int M,
                       int K, int N, int SKG, int scale_mode, int64_t stream) {
  dense_run(a8, sa, w8, sw, c, ws, tickets, M, K, N, SKG, scale_mode, false, stream, "gemm_i8_dense");
}
// Test entry: the exact int32 sums C[m][n] = sum_k A[m][k] W[n][k] (int32 [256][N]) through the same kernel and
// split.
void r4d_gemm_i8_dense_raw(int64_t a8, int64_t w8, int64_t c, int64_t ws, int64_t tickets, int M, int K, int N,
                           int SKG, int64_t stream) {
  dense_run(a8, 0, w8, 0, c, ws, tickets, M, K, N, SKG, 0, true, stream, "gemm_i8_dense_raw");
}
// This build's K split for the dense int8 GEMM: the fewest slices (of at least 1024 k) that reach 128
// workgroups -- the split that measured fastest at both config-4 shapes (1 at 5120 x 17408, 4 at 17408 x 5120).
int r4d_mi355x_i8_skg(int K, int N) {
  const int G = N / 128, nkb = K / 128;
  int best = 1;
  for (int d = 1; d <= 8; d *= 2) {         // the split counts r4d_gemm_trellis_nt_i8_check allows
    if (nkb % d || nkb / d < 8) continue;
    best = d;
    if ((long long)G * d >= 128) break;
  }
  return best;
}

// This build's launch form for the dense int8 GEMM by scale mode: the per-128 modes run stream-K (SKG = 0; measured
// 8-11 % faster than the best split at both config-4 shapes), row / column scales the split above.
int r4d_mi355x_i8_dense_skg(int K, int N, int scale_mode) {
  if (K <= 0 || N <= 0 || K % 128 || N % 128) return 1;
  return scale_mode != 0 ? 0 : r4d_mi355x_i8_skg(K, N);
}

// r4d.h:490 (K / 128) N floats
size_t r4d_trellis_i8_wscale_count(int K, int N) { return (size_t)(K / 128) * (size_t)N; }
// r4d.h:491
void r4d_trellis_i8_wscale(int64_t w, int64_t sw, int K, int N, int KB, int64_t stream) {
  ti8_table(false, w, sw, K, N, KB, stream, "trellis_i8_wscale");
}
// r4d.h:492
void r4d_trellis_i8_dump_w(int64_t w, int64_t sw, int64_t w8, int64_t wp, int K, int N, int KB, int64_t stream) {
  ti8_dump(false, w, sw, w8, wp, K, N, KB, stream, "trellis_i8_dump_w");
}
// r4d.h:495-497; skw is the reference's per-workgroup K split: checked for legality, not used
void r4d_gemm_trellis_nt_i8(int64_t a8_0, int64_t sa_0, int64_t a8_1, int64_t sa_1, int n_split, int64_t w,
                            int64_t sw, int64_t svh, int64_t c, int64_t ws, int64_t tickets, int M, int K, int N,
                            int KB, int skw, int skg, float out_scale, int64_t stream) {
  ti8_run(true, a8_0, sa_0, a8_1, sa_1, n_split, w, sw, svh, c, ws, tickets, M, K, N, KB, skw, skg, out_scale, stream,
          "gemm_trellis_nt_i8");
}
// r4d.h:498
const char* r4d_gemm_trellis_nt_i8_check(int M, int K, int N, int n_split, int KB, int skw, int skg) {
  return r4d::check_result(ti8_check(M, K, N, n_split, KB, skw, skg));
}
// r4d.h:499 SKG M N fp32
size_t r4d_gemm_trellis_nt_i8_ws_bytes(int M, int N, int SKG) { return (size_t)SKG * M * N * 4; }
// r4d.h:514
size_t r4d_trellis_i8_wscale_col_count(int K, int N) {
  (void)K;
  return (size_t)N;
}
// r4d.h:515
void r4d_trellis_i8_wscale_col(int64_t w, int64_t swc, int K, int N, int KB, int64_t stream) {
  ti8_table(true, w, swc, K, N, KB, stream, "trellis_i8_wscale_col");
}
// r4d.h:516
void r4d_trellis_i8_dump_w_col(int64_t w, int64_t swc, int64_t w8, int64_t wp, int K, int N, int KB, int64_t stream) {
  ti8_dump(true, w, swc, w8, wp, K, N, KB, stream, "trellis_i8_dump_w_col");
}
// r4d.h:519-521
void r4d_gemm_trellis_nt_i8c(int64_t a8_0, int64_t sa_0, int64_t a8_1, int64_t sa_1, int n_split, int64_t w,
                             int64_t swc, int64_t svh, int64_t c, int64_t ws, int64_t tickets, int M, int K, int N,
                             int KB, int skw, int skg, float out_scale, int64_t stream) {
  ti8_run(false, a8_0, sa_0, a8_1, sa_1, n_split, w, swc, svh, c, ws, tickets, M, K, N, KB, skw, skg, out_scale,
          stream, "gemm_trellis_nt_i8c");
}

}  // extern "C"
