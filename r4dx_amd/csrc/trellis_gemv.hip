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
// the whole batch, so the MFMA cost per weight is independent of M up to 16. SKG workgroups split K;
// inside a workgroup, SK waves split each pair's slice (SK = 4, the split form) or one wave takes it
// whole (SK = 1). Partial sums go to ws [SKG][M][N] and the last workgroup of a 128-column group
// (ticket) sums them in a fixed order and finishes: FWHT-128 in fp32 in the reference's stage order,
// * svh, * out_scale, one bf16 rounding. A row's bits depend on (K, N, KB, SKG, SK) only -- never on M,
// on the pairs per workgroup or on the other rows -- so decode rows equal verify rows for every M <= 64.
#include "r4d_dev.h"
#include "r4d_host.h"
#include "r4d_mi355x.h"

namespace {

template <int KB>
struct Words {
  unsigned w[KB + 1];   // [0] history, [1..KB] own words
};

#define R4_RSRC_FLAGS 0x00020000
typedef __amdgpu_buffer_rsrc_t r4_rsrc;
__device__ __forceinline__ r4_rsrc r4_make_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)bytes, R4_RSRC_FLAGS);
}

// Byte offsets, inside a (pair, k-tile) block, of the lane's own words (KB c .. KB c + KB - 1 of tile t)
// and history word (KB c - 1 mod 8 KB); block q of a step sits q * 64 KB bytes further.
template <int KB>
struct LaneWords {
  unsigned own, hist;
  __device__ __forceinline__ LaneWords(int q, int t, int c) {
    const unsigned tile = (unsigned)(q * 16 * KB + t * 8 * KB);
    own = (tile + KB * c) * 4u;
    hist = (tile + (KB * c - 1 + 8 * KB) % (8 * KB)) * 4u;
  }
};

// Cache policy of the weight loads: nontemporal (each word is read once per launch; measured ~2 % faster
// per step than the default policy).
constexpr int kWeightPolicy = 2;

// One step's words of this lane from the slice buffer at step byte offset so (out of range -> 0).
template <int KB, bool HIST = true>
__device__ __forceinline__ void load_words(Words<KB>& s, r4_rsrc r, const LaneWords<KB>& lw, unsigned so) {
  // one wide load per lane where the KB words allow it (buffer loads need dword alignment only): KB 4 one dwordx4,
  // KB 5 a dwordx4 and a dword, KB 3 a dwordx3 -- not KB dword loads, each of which would touch every line of the step
  if constexpr (KB == 4 || KB == 5) {
    const r4u4 v = __builtin_bit_cast(r4u4, __builtin_amdgcn_raw_buffer_load_b128(r, lw.own + so, 0, kWeightPolicy));
    s.w[1] = v[0]; s.w[2] = v[1]; s.w[3] = v[2]; s.w[4] = v[3];
    if constexpr (KB == 5) s.w[5] = __builtin_amdgcn_raw_buffer_load_b32(r, lw.own + so + 16, 0, kWeightPolicy);
  } else if constexpr (KB == 3) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b96(r, lw.own + so, 0, kWeightPolicy);
    s.w[1] = v[0]; s.w[2] = v[1]; s.w[3] = v[2];
  } else {
#pragma unroll
    for (int i = 0; i < KB; ++i) s.w[1 + i] = __builtin_amdgcn_raw_buffer_load_b32(r, lw.own + so + 4 * i, 0, kWeightPolicy);
  }
  if constexpr (HIST) s.w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, lw.hist + so, 0, kWeightPolicy);
}

// A row's two fragments (h = 0, 1) of one k-tile from the row buffer at byte offset off:
// k 16kt + {0..3, 8..11} and {4..7, 12..15}.
__device__ __forceinline__ void load_a(r4h8 (&af)[2], r4_rsrc r, unsigned off) {
  const r4u4 lo = __builtin_bit_cast(r4u4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
  const r4u4 hi = __builtin_bit_cast(r4u4, __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, 0));
  const r4u4 f0 = {lo[0], lo[1], hi[0], hi[1]}, f1 = {lo[2], lo[3], hi[2], hi[3]};
  af[0] = __builtin_bit_cast(r4h8, f0);
  af[1] = __builtin_bit_cast(r4h8, f1);
}

// Same, for the plain pointer form (the reconstruct kernel).
template <int KB>
__device__ __forceinline__ void load_words_ptr(Words<KB>& s, const unsigned* __restrict__ blk, int t, int c) {
  const unsigned* tile = blk + t * 8 * KB;
#pragma unroll
  for (int i = 0; i <= KB; ++i) s.w[i] = tile[r4_lane_word<KB>(c, i)];
}

// Kernel geometry: a workgroup is NPW tile pairs x SK waves (64 NPW SK threads); the SK waves of a pair
// split the workgroup's K slice into SK contiguous parts, added in k order; SKG workgroups split K.
// The split form (SK = 4, NPW = 1 or 2) finishes every 128-column group in the last of its
// SKG 4 / NPW contributors through ws and tickets; the whole-group form (NPW = 4, SK = 1) covers a group
// and, at SKG = 1, finishes it in the workgroup (no ws). Many short workgroups let the dispatcher
// balance the VALU-bound decode over the CUs (measured better on gfx950 than a persistent grid).
// Weights are prefetched PF steps ahead (a step is 4 k-tiles = one dwordx4 per lane) and issued before
// A is staged in LDS.
constexpr int kRedParts = 8;         // the final slice sum is 8 interleaved runs, added in order
constexpr int kRedRows = 4;          // rows of the final slice sum per pass (8 measured slower at M = 8: LDS)

// n / d for the staging loops' row split (d = M <= 64, n below 2^20): one high multiply by the launch-uniform
// floor(2^32 / d) + 1, exact whenever n d < 2^32 (the error term n e / (d 2^32), 0 < e <= d, stays below 1 / d);
// d = 1 (whose multiplier would need 33 bits) is marked by 0 and returns n.
// The multipliers for d = 0..64 as a constant table (d = 0 unused): a scalar load of the launch's M instead of a 64-bit
// division formed with VALU ops in every wave.
struct R4DivMagic {
  unsigned m[65];
  constexpr R4DivMagic() : m() {
    for (unsigned d = 1; d <= 64; ++d) m[d] = d == 1u ? 0u : (unsigned)(0x100000000ull / d) + 1u;
  }
};
__constant__ constexpr R4DivMagic kR4DivMagic{};
__device__ __forceinline__ unsigned r4_div_magic(unsigned d) { return kR4DivMagic.m[d]; }
__device__ __forceinline__ int r4_div_by(int n, unsigned magic) {
  return magic ? (int)__umulhi((unsigned)n, magic) : n;
}

// XF > 0: A0 is the raw input x [M][K] (XF 1: f16, 2: bf16) and the workgroup stages its own slice of the
// transformed A = f16(FWHT128(fp32(x) * suh) * xscale) (suh of the group's column part) straight into LDS --
// the arithmetic of r4dx_trellis_input_*, so A is bit-identical to the unfused path's.
template <int KB, int MT, int NPW, int SK, bool ALDS, int XF, bool WQ = false>
__global__ __launch_bounds__(64 * NPW * SK) void tq_gemv_kernel(
    const R4AParts ap,
    const unsigned* __restrict__ W, const float* __restrict__ svh, void* __restrict__ Cv,
    float* __restrict__ ws, unsigned* __restrict__ tickets, int M, int K, int N, int SKG, int full,
    float out_scale, const R4SParts sp, float xscale,
    unsigned long long* __restrict__ clk, const float* __restrict__ wsc, int wq_gsh) {
  // steps in flight; 2 where each ring slot also carries MT row tiles of A from global memory (4 slots of 4 row
  // tiles would not fit the VGPRs and spill)
  constexpr int PF = (!ALDS && MT >= 4) ? 2 : 4;
  constexpr int NT = 64 * NPW * SK;
  constexpr int NW = NPW * SK;                 // waves
  constexpr int BLK = 16 * KB;                 // words per (pair, k-tile) block
  extern __shared__ r4u4 lds_raw[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // the _raw entry's clock probe (r4d.h:376-383): workgroup (0, 0)'s thread 0 records the shader clock and
  // the 100 MHz wall clock at entry and at the end of its own work (its sums combined, before any output)
  const bool probe = clk != nullptr && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0;
  if (probe) {
    clk[0] = __builtin_amdgcn_s_memtime();
    clk[1] = __builtin_amdgcn_s_memrealtime();
  }
  const int pl = wave % NPW, ks = wave / NPW;
  const int ky = blockIdx.y;
  const int pair = blockIdx.x * NPW + pl;
  const int group = (blockIdx.x * NPW) >> 2;
  const int KT = K >> 4, ktw = r4_div_by(KT, r4_div_magic((unsigned)SKG)), kt0 = ky * ktw;   // SKG <= 64, KT < 2^20
  const unsigned short* __restrict__ A0 = ap.a[0];
  const unsigned short* __restrict__ A = r4_part_a(ap, group * 128);
  const int q = lane >> 4, t = (lane >> 3) & 1, c = lane & 7, mrow = lane & 15;

  // Steps (4 k-tiles each) of the slice, split into SK contiguous parts of at most nsw steps.
  const int steps_all = (ktw + 3) >> 2;
  const int nsw = (steps_all + SK - 1) / SK;
  const int st_beg = ks * nsw;
  const int nst = max(0, min(nsw, steps_all - st_beg));
  const int ktl_pad = SK * nsw * 4;            // k-tiles the LDS copy of A covers (zero past ktw)
  const unsigned mmag = r4_div_magic((unsigned)M);

  // LDS: the A slice (ALDS) + its zero block while the k loop runs; after it (every wave past the barrier that ends
  // the loop), the same bytes hold [SK - 1 partial accumulators per pair] [M x 128 sums] [8 x 4 x 128 reduce runs]
  // [flag]. The launch asks for the larger of the two.
  r4u4* alds = lds_raw;
  float* part_acc = (float*)lds_raw;                                 // [(SK-1) * NPW][8 MT][64]
  float* red = part_acc + (size_t)(SK - 1) * NPW * 8 * MT * 64;      // [M][128]
  float* runs = red + (size_t)M * 128;                               // [8][4][128]
  const int red_rows = min(kRedRows, M);      // rows per finish pass (the LDS holds no more)
  int* flag = (int*)(runs + (size_t)kRedParts * red_rows * 128);

  const unsigned* __restrict__ wpair = W + ((size_t)pair * KT + kt0) * BLK;
  const r4_rsrc wr = r4_make_rsrc(wpair, (unsigned)ktw * BLK * 4u);
  const LaneWords<KB> lw(q, t, c);
  constexpr unsigned kStepBytes = 4 * BLK * 4;
  // A: LDS byte address of this lane's fragment pair at step 0 and its per-step stride (rows >= M
  // read the zero block with stride 0); or, from global memory, a buffer over A with the row offset.
  unsigned a_off[MT], a_stride[MT];
  const r4_rsrc ar = r4_make_rsrc(A, (unsigned)((size_t)M * K * 2));
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int r = i * 16 + mrow;
    if constexpr (ALDS) {
      a_off[i] = r < M ? (unsigned)(((st_beg * 4 + q) * M + r) * 32) : (unsigned)(ktl_pad * M * 32);
      a_stride[i] = r < M ? (unsigned)(4 * M * 32) : 0u;
    } else {
      a_off[i] = r < M ? (unsigned)((size_t)r * K * 2 + (size_t)(kt0 + st_beg * 4 + q) * 32) : 0x80000000u;
      a_stride[i] = 4 * 32;
    }
  }

  struct St {
    Words<KB> w;
    r4h8 a[ALDS ? 1 : MT][2];
  };
  // Step s of this wave (clamped to its last step, so a prefetch past the end re-reads a cached
  // line instead of another wave's weights).
  auto load = [&](St& s, int sidx) {
    const int sc = min(sidx, nst - 1);
    load_words<KB, XF == 0>(s.w, wr, lw, (unsigned)(st_beg + sc) * kStepBytes);
    if constexpr (!ALDS) {
      const bool ok = (st_beg + sc) * 4 + q < ktw;
#pragma unroll
      for (int i = 0; i < MT; ++i) load_a(s.a[i], ar, ok ? a_off[i] + (unsigned)sc * a_stride[i] : 0x80000000u);
    }
  };
  r4f4 acc[MT][2];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i][0] = acc[i][1] = (r4f4){0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const St& s, int sidx) {
    r4h8 af[MT][2];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      if constexpr (ALDS) {
        const r4u4* p = (const r4u4*)((const char*)alds + a_off[i] + (unsigned)sidx * a_stride[i]);
        af[i][0] = __builtin_bit_cast(r4h8, p[0]);
        af[i][1] = __builtin_bit_cast(r4h8, p[1]);
      } else {
        af[i][0] = s.a[i][0];
        af[i][1] = s.a[i][1];
      }
    }
    unsigned d[2][2][4];
    if constexpr (XF == 0) {
      r4_decode<KB>(s.w.w, d);
      if constexpr (WQ) {
        // the _wq measurement: this lane's k-tile and two columns under their group scales
        const int kt = kt0 + (st_beg + sidx) * 4 + q;
        float sc[2] = {1.0f, 1.0f};
        if (kt < KT) {
          const size_t row = (size_t)(kt >> wq_gsh) * N + (size_t)pair * 32 + 16 * t + c;
          sc[0] = wsc[row];
          sc[1] = wsc[row + 8];
        }
        r4_wq_apply(d, sc);
      }
    } else {
      // the fused-transform form takes the history word from lane c - 1 through the LDS crossbar (ds_bpermute,
      // no VALU): measured 3 % faster there, while in the plain form the load is faster
      unsigned wl[KB + 1];
      wl[0] = (unsigned)__builtin_amdgcn_ds_bpermute(((lane & ~7) | ((lane + 7) & 7)) << 2, (int)s.w.w[KB]);
#pragma unroll
      for (int i = 1; i <= KB; ++i) wl[i] = s.w.w[i];
      r4_decode<KB>(wl, d);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const r4h8 b0 = r4_frag(d[0][h]), b1 = r4_frag(d[1][h]);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        acc[i][0] = r4_mfma16(af[i][h], b0, acc[i][0]);
        acc[i][1] = r4_mfma16(af[i][h], b1, acc[i][1]);
      }
    }
  };

  // Fused transform: one wave per (128-block, row) of the slice; lane l takes k = 128 b + 2 l, 2 l + 1 (one
  // dword of x, two floats of suh). The x and suh of this wave's first kXfPre blocks are requested before
  // the weight stream and the rest after it: loads retire in order, so a block requested after the
  // weights waits for them.
  constexpr int kXfPre = 6;
  const int xf_nblk = (ktl_pad + 7) >> 3;
  const float* __restrict__ suh_p = sp.s[r4_part_idx(ap, group * 128)];
  struct XfIn {
    unsigned x2;   // x[2l], x[2l + 1] (f16 or bf16 bits)
    r4f2 s2;       // suh[2l], suh[2l + 1]
  };
  // unconditional buffer loads (a unit past the slice reads past both buffers and gets 0): no branch around a load,
  // so the waits before a unit's use count only what is needed
  const r4_rsrc xr = r4_make_rsrc(A0, (unsigned)((size_t)M * K * 2));
  const r4_rsrc shr = r4_make_rsrc(suh_p, (unsigned)((size_t)K * 4));
  auto xf_load = [&](int u) {
    XfIn v;
    const int b = r4_div_by(u, mmag), r = u - b * M;
    const bool ok = u < xf_nblk * M && 8 * b < ktw;
    const unsigned kb = (unsigned)(16 * kt0 + 128 * b + 2 * lane);
    v.x2 = __builtin_amdgcn_raw_buffer_load_b32(xr, ok ? ((unsigned)r * (unsigned)K + kb) * 2u : 0xFFFFFFF0u, 0, 0);
    v.s2 = __builtin_bit_cast(r4f2, __builtin_amdgcn_raw_buffer_load_b64(shr, ok ? kb * 4u : 0xFFFFFFF0u, 0, 0));
    return v;
  };
  XfIn xpre[XF > 0 ? kXfPre : 1];
  if constexpr (XF > 0) {
#pragma unroll
    for (int j = 0; j < kXfPre; ++j) xpre[j] = xf_load(wave + NW * j);
  }
  // The weight stream starts while A is staged, so its latency overlaps the staging. In the plain staged form the
  // first pass's A loads go out just before it: loads retire in order, so the staging then waits for A only, not for
  // the PF steps of weights behind it.
  St ring[PF];
  // unconditional (a wave without steps reads past its buffer, which returns 0), so no branch joins the loads and the
  // staging's waits count the A loads only
  auto load_ring = [&]() {
#pragma unroll
    for (int i = 0; i < PF; ++i) load(ring[i], i);
  };
  if constexpr (!(ALDS && XF == 0)) load_ring();
  if constexpr (ALDS && XF > 0) {
    // A = f16(FWHT128(fp32(x) * suh) * xscale) (r4_fwht128_wave_pairs: the same fp32 operations per element
    // as r4dx_trellis_input_*), each lane's two adjacent k written as one dword to its fragment slot --
    // element k16 of k-tile ktl sits at half (k16 >> 3) + 2 ((k16 >> 2) & 1) of the 32-byte (ktl, row)
    // chunk (h = 0: k 0-3, 8-11; h = 1: k 4-7, 12-15); then the zero block.
    unsigned* ah = (unsigned*)alds;
    auto xf_stage = [&](int u, const XfIn& v) {
      const int b = r4_div_by(u, mmag), r = u - b * M;
      if (u >= xf_nblk * M) return;
      unsigned hv = 0u;
      if (8 * b < ktw) {
        const float x0 = XF == 2 ? r4_bf16_to_f32((unsigned short)(v.x2 & 0xFFFFu)) : r4_f16_to_f32((unsigned short)(v.x2 & 0xFFFFu));
        const float x1 = XF == 2 ? r4_bf16_to_f32((unsigned short)(v.x2 >> 16)) : r4_f16_to_f32((unsigned short)(v.x2 >> 16));
        float v0 = x0 * v.s2[0];
        float v1 = x1 * v.s2[1];
        r4_fwht128_wave_pairs(v0, v1, lane);
        hv = (unsigned)r4_f16_rn(v0 * xscale) | ((unsigned)r4_f16_rn(v1 * xscale) << 16);
      }
      const int kl = 128 * b + 2 * lane, ktl = kl >> 4, k16 = kl & 15;
      if (ktl < ktl_pad) ah[(size_t)(ktl * M + r) * 8 + (((k16 >> 3) & 1) + 2 * ((k16 >> 2) & 1)) * 2 + ((k16 & 3) >> 1)] = hv;
    };
#pragma unroll
    for (int j = 0; j < kXfPre; ++j) xf_stage(wave + NW * j, xpre[j]);
#pragma unroll 1
    for (int u0 = wave + NW * kXfPre; u0 < xf_nblk * M; u0 += NW * kXfPre) {   // the rest, kXfPre units per round trip
      XfIn v[kXfPre];
#pragma unroll
      for (int j = 0; j < kXfPre; ++j) v[j] = xf_load(u0 + NW * j);
#pragma unroll
      for (int j = 0; j < kXfPre; ++j) xf_stage(u0 + NW * j, v[j]);
    }
    if (threadIdx.x < 8) ah[(size_t)ktl_pad * M * 8 + threadIdx.x] = 0u;
    __syncthreads();
  } else if constexpr (ALDS) {
    // chunk (ktl, row, j): k 16 (kt0 + ktl) + 8j .. + 8 of A[row] -> halves of fragments h = 0, 1;
    // k-tiles past the slice are zero, and so is the 32-byte block after the copy (rows >= M read it).
    // kStageU chunks per thread per pass, all loads issued before any is written: one memory round trip
    // per pass, not one per chunk (at M = 8 and up a workgroup stages several chunks per thread)
    constexpr int kStageU = 4;
    const int chunks = ktl_pad * M * 2;
    // chunk i's byte offset in A, or one past the buffer (a zero chunk): the loads are unconditional buffer loads, so
    // the kStageU of a pass go out back to back (a load under a branch waits for its data at the branch's end)
    auto chunk_off = [&](int i) -> unsigned {
      const int j = i & 1, rm = i >> 1, ktl = r4_div_by(rm, mmag), r = rm - ktl * M;
      return (i < chunks && ktl < ktw) ? (unsigned)(((size_t)r * K + 16 * (kt0 + ktl) + 8 * j) * 2) : 0xFFFFFFF0u;
    };
    auto chunk_load = [&](int i) -> r4u4 {
      return __builtin_bit_cast(r4u4, __builtin_amdgcn_raw_buffer_load_b128(ar, chunk_off(i), 0, 0));
    };
    if (chunks + 2 <= NT) {   // one chunk per thread at most (M = 1, 2): no unrolled address arithmetic
      const int i = threadIdx.x;
      const int j = i & 1, rm = i >> 1;
      const r4u4 v = chunk_load(i);
      __builtin_amdgcn_sched_barrier(0);   // the A load goes out before the weight loads
      load_ring();
      if (i < chunks + 2) {
        r4u2* dst = (r4u2*)(alds + (size_t)rm * 2);
        dst[j] = (r4u2){v[0], v[1]};
        dst[2 + j] = (r4u2){v[2], v[3]};
      }
    } else {
      // every thread runs the first pass (chunks + 2 > NT here): its loads, then the weight stream, unconditionally, so
      // the waits before the writes count the A loads only
      // branch-free writes: a chunk past the copy is zero (its load read past the buffer) and lands in the zero block
      auto put_pass = [&](int i0, const r4u4 (&v)[kStageU]) {
#pragma unroll
        for (int u = 0; u < kStageU; ++u) {
          const int i = i0 + u * NT;
          const int j = i & 1, rm = min(i >> 1, chunks >> 1);
          r4u2* dst = (r4u2*)(alds + (size_t)rm * 2);
          dst[j] = (r4u2){v[u][0], v[u][1]};        // h = 0, elements 4j .. 4j + 3
          dst[2 + j] = (r4u2){v[u][2], v[u][3]};    // h = 1
        }
      };
      {
        r4u4 v[kStageU];
#pragma unroll
        for (int u = 0; u < kStageU; ++u) v[u] = chunk_load((int)threadIdx.x + u * NT);
        __builtin_amdgcn_sched_barrier(0);
        load_ring();
        put_pass((int)threadIdx.x, v);
      }
      for (int i0 = (int)threadIdx.x + kStageU * NT; i0 < chunks + 2; i0 += kStageU * NT) {
        r4u4 v[kStageU];
#pragma unroll
        for (int u = 0; u < kStageU; ++u) v[u] = chunk_load(i0 + u * NT);
        put_pass(i0, v);
      }
    }
    __syncthreads();
  }
  if (nst > 0) {
    int st = 0;
    for (; st + PF <= nst; st += PF) {
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        compute(ring[i], st + i);
        load(ring[i], st + i + PF);
        __builtin_amdgcn_sched_barrier(0);   // one step at a time: no decode hoisted across the reload
      }
    }
#pragma unroll
    for (int i = 0; i < PF - 1; ++i)
      if (st + i < nst) compute(ring[i], st + i);
  }

  // The A slice is dead once every wave has left the loop: the combine, the sums and the reduce runs reuse its bytes.
  if constexpr (ALDS) __syncthreads();
  // Combine the SK waves of each pair in k order (ks = 0, 1, ...) into wave ks = 0.
  if constexpr (SK > 1) {
    if (ks > 0) {
      float* dst = part_acc + ((size_t)((ks - 1) * NPW + pl) * 8 * MT) * 64;
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
          for (int j = 0; j < 4; ++j) dst[((i * 2 + f) * 4 + j) * 64 + lane] = acc[i][f][j];
    }
    __syncthreads();
    if (ks == 0) {
#pragma unroll
      for (int s = 1; s < SK; ++s) {
        const float* src = part_acc + ((size_t)((s - 1) * NPW + pl) * 8 * MT) * 64;
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int f = 0; f < 2; ++f)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][f][j] += src[((i * 2 + f) * 4 + j) * 64 + lane];
      }
    }
  }

  if (probe) {
    clk[2] = __builtin_amdgcn_s_memtime();
    clk[3] = __builtin_amdgcn_s_memrealtime();
  }

  // Lane l of wave (pl, ks = 0) holds rows 16 i + 4 (l >> 4) + j of column slot nb = l & 15 of
  // fragment cs: true column 32 pair + 16 (nb >> 3) + (nb & 7) + 8 cs.
  const int nb = lane & 15, rq = lane >> 4;
  const int gcol0 = (pair & 3) * 32 + 16 * (nb >> 3) + (nb & 7);   // inside the group
  float* Cf = (float*)Cv;
  unsigned short* Cb = (unsigned short*)Cv;
  const int n0 = group * 128;
  const bool in_block = NPW == 4 && SKG == 1;   // the workgroup holds its whole group

  if (SKG == 1 && !full) {
    if (ks == 0) {
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
    }
    return;
  }
  if (in_block) {
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
    if (ks == 0) {
      float* wsy = ws + (size_t)ky * M * N;
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 16 * i + 4 * rq + j;
          if (r < M) {
            r4_store_coherent(&wsy[(size_t)r * N + n0 + gcol0], acc[i][0][j]);
            r4_store_coherent(&wsy[(size_t)r * N + n0 + gcol0 + 8], acc[i][1][j]);
          }
        }
    }
    if (!r4_ticket_last(&tickets[group * R4_TICKET_WORDS], (unsigned)(SKG * (4 / NPW)), flag)) return;
    // Sum the SKG slices: run p (0..7) adds slices p, p + 8, ... in order; the 8 runs are then added
    // in order 0..7 -- the same arithmetic for every element whatever M is. kRedRows rows at a time
    // (bounded LDS); the finished sums land in red[r][128] for the epilogue.
    // SKG <= 64, so one batch of 8 loads (slices p, p + 8, ..., p + 56) covers a run. The loads are
    // coherent (sc1) buffer loads over ws: a slice past SKG or an item past the end reads past the buffer
    // and returns 0, so every thread issues all loads of its kFinItems items at once, with no branches.
    const unsigned sy4 = (unsigned)M * (unsigned)N * 4u;
    const r4_rsrc wsr = r4_make_rsrc(ws, (unsigned)SKG * sy4);
    if (SKG <= kRedParts) {
      // At most one slice per run (every planned split): each thread sums whole elements -- run p is 0.f + slice p,
      // the runs are added in order and the empty ones (p >= SKG) add +0.f, which the one addition below stands for
      // (adding +0.f again changes nothing) -- with its SKG loads issued at once: the same bits as the general form
      // below, without its loads of absent slices and its second pass through LDS.
      constexpr int kFinE = 2;   // elements per thread per pass
      for (int e0 = (int)threadIdx.x; e0 < M * 128; e0 += kFinE * NT) {
        float tv[kFinE][kRedParts];
#pragma unroll
        for (int it = 0; it < kFinE; ++it) {
          const int e = e0 + it * NT;
          const unsigned off = e < M * 128 ? ((unsigned)(e >> 7) * (unsigned)N + (unsigned)(n0 + (e & 127))) * 4u : 0xFFFFFFF0u;
#pragma unroll
          for (int p = 0; p < kRedParts; ++p)
            if (p < SKG)
              tv[it][p] = __builtin_bit_cast(
                  float, __builtin_amdgcn_raw_buffer_load_b32(wsr, off == 0xFFFFFFF0u ? off : off + (unsigned)p * sy4, 0, 16));
        }
#pragma unroll
        for (int it = 0; it < kFinE; ++it) {
          const int e = e0 + it * NT;
          float v = 0.f + tv[it][0];
#pragma unroll
          for (int p = 1; p < kRedParts; ++p)
            if (p < SKG) v += 0.f + tv[it][p];
          if (SKG < kRedParts) v += 0.f;
          if (e < M * 128) {
            if (full) red[e] = v;
            else Cf[(size_t)(e >> 7) * N + n0 + (e & 127)] = v;
          }
        }
      }
      __syncthreads();
      if (!full) return;
    } else {
    constexpr int kFinItems = 4;
    for (int r0 = 0; r0 < M; r0 += red_rows) {
      const int rows = min(red_rows, M - r0);
      const int items = kRedParts * rows * 128;
      for (int b0 = 0; b0 < items; b0 += kFinItems * NT) {
        float tv[kFinItems][8];
#pragma unroll
        for (int it = 0; it < kFinItems; ++it) {
          const int idx = b0 + it * NT + (int)threadIdx.x;
          const int p = idx / (rows * 128), e = idx - p * rows * 128;
          const unsigned off = idx < items ? (unsigned)p * sy4 + ((unsigned)(r0 + (e >> 7)) * (unsigned)N + (unsigned)(n0 + (e & 127))) * 4u
                                           : 0xFFFFFFF0u;
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const unsigned ou = off + (unsigned)u * (unsigned)kRedParts * sy4;
            const unsigned o = (off == 0xFFFFFFF0u || ou < off) ? 0xFFFFFFF0u : ou;   // wrap-safe
            tv[it][u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wsr, o, 0, 16));
          }
        }
#pragma unroll
        for (int it = 0; it < kFinItems; ++it) {
          const int idx = b0 + it * NT + (int)threadIdx.x;
          if (idx < items) {
            const int p = idx / (rows * 128), e = idx - p * rows * 128;
            float v = 0.f;
#pragma unroll
            for (int u = 0; u < 8; ++u) v += tv[it][u];
            runs[(size_t)p * red_rows * 128 + e] = v;
          }
        }
      }
      __syncthreads();
      for (int e = threadIdx.x; e < rows * 128; e += NT) {
        float v = runs[e];
#pragma unroll
        for (int p = 1; p < kRedParts; ++p) v += runs[(size_t)p * red_rows * 128 + e];
        if (full) red[(size_t)r0 * 128 + e] = v;
        else Cf[(size_t)(r0 + (e >> 7)) * N + n0 + (e & 127)] = v;
      }
      __syncthreads();
    }
    if (!full) return;
    }
  }
  // The epilogue: one wave per row, the group's 128 sums as (lane, lane + 64).
  const float sv0 = svh[n0 + lane], sv1 = svh[n0 + lane + 64];
  for (int r = wave; r < M; r += NW) {
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
  load_words_ptr<KB>(s, W + ((size_t)pair * KT + kt) * (16 * KB), t, c);
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

// The _wq entries' scale table [K / 16 >> gsh][N] (r4d.h:433-436): s = max|Q| / 127 (fp32 division; 1 for an
// all-zero group) over each column's 16 2^gsh values of a group of 2^gsh k-tiles, from the GEMM's own decode. One
// wave per (tile pair, block of max(4, 2^gsh) k-tiles); a lane takes the amax of its 16 values per column, the
// lanes of one group meet by shuffles.
template <int KB>
__global__ __launch_bounds__(256) void tq_wscale_kernel(const unsigned* __restrict__ W, float* __restrict__ table,
                                                        int K, int N, int gsh) {
  const int lane = threadIdx.x & 63;
  const int KT = K >> 4, ktb = max(4, 1 << gsh), nblk = KT / ktb;
  const long long id = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (id >= (long long)(N >> 5) * nblk) return;
  const int pair = (int)(id / nblk), blk = (int)(id - (long long)pair * nblk);
  const int q = lane >> 4, t = (lane >> 3) & 1, c = lane & 7;
  float m[2] = {0.f, 0.f};
  for (int st = 0; st < ktb / 4; ++st) {
    const int kt = blk * ktb + st * 4 + q;
    Words<KB> w;
    load_words_ptr<KB>(w, W + ((size_t)pair * KT + kt) * (16 * KB), t, c);
    unsigned d[2][2][4];
    r4_decode<KB>(w.w, d);
#pragma unroll
    for (int cs = 0; cs < 2; ++cs)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const unsigned v = d[cs][h][j];
          m[cs] = __builtin_fmaxf(m[cs], __builtin_fmaxf(__builtin_fabsf(r4_f16_to_f32((unsigned short)(v & 0xFFFFu))),
                                                         __builtin_fabsf(r4_f16_to_f32((unsigned short)(v >> 16)))));
        }
  }
  // a group spans k-tile lanes q ^ 1 (gsh 1) or all four (gsh >= 2)
#pragma unroll
  for (int cs = 0; cs < 2; ++cs) {
    m[cs] = __builtin_fmaxf(m[cs], __shfl_xor(m[cs], 16, 64));
    if (gsh >= 2) m[cs] = __builtin_fmaxf(m[cs], __shfl_xor(m[cs], 32, 64));
  }
  if ((q & ((1 << min(gsh, 2)) - 1)) != 0) return;
  const int g = (blk * ktb + q) >> gsh;
#pragma unroll
  for (int cs = 0; cs < 2; ++cs)
    table[(size_t)g * N + pair * 32 + 16 * t + 8 * cs + c] = m[cs] > 0.f ? m[cs] / 127.0f : 1.0f;
}

// Dynamic LDS of one launch.
size_t gemv_ktl_pad(int SK, int ktw) { return (size_t)SK * ((((ktw + 3) >> 2) + SK - 1) / SK) * 4; }
// The A slice (ALDS) and, after the k loop, in the same bytes: the partial accumulators, the sums, the reduce runs and
// the flag.
size_t gemv_lds(int MT, int NPW, int SK, bool alds, int ktw, int M) {
  const size_t a = alds ? gemv_ktl_pad(SK, ktw) * M * 32 + 32 : 0;
  const size_t tail = (size_t)(SK - 1) * NPW * 8 * MT * 64 * 4 +
                      (size_t)(M + kRedParts * (M < kRedRows ? M : kRedRows)) * 128 * 4 + 16;
  return a > tail ? a : tail;
}
constexpr size_t kAldsMax = 48 * 1024;   // A slices up to this many bytes are staged in LDS

constexpr size_t kXfAldsMax = 96 * 1024;   // the fused transform stages the slice in LDS up to this size

// The launch form launch_gemv_np picks: the whole-group form (4 pairs x 1 wave) for the SK = 1 order or an unsplit
// launch without ws, else the split form (1 pair at M = 1, 2 at M >= 2, each over 4 waves); MT row tiles of 16.
struct GemvForm {
  int NPW, SK, MT;
};
// xf (the fused input transform): at M = 1 a workgroup of a launch with N >= 8192 holds two pairs, which halves the
// transform work repeated per pair (every workgroup transforms its whole K slice). Measured per launch at M = 1
// (µs, one pair / two pairs per workgroup): 5120x8192 12.0 / 11.5, 5120x16384 18.8 / 17.4, 5120x34816 34.1 / 33.2,
// but 6144x5120 10.9 / 11.8 and 17408x5120 19.5 / 20.8 (fewer workgroups on the 160 pairs of N = 5120).
GemvForm gemv_form(int M, int N, int SKG, bool have_ws, bool sk1, bool xf = false) {
  GemvForm f;
  f.MT = M <= 16 ? 1 : M <= 32 ? 2 : 4;
  if (sk1 || (SKG == 1 && !have_ws)) { f.NPW = 4; f.SK = 1; }
  else { f.NPW = M == 1 && !(xf && N >= 8192) ? 1 : 2; f.SK = 4; }
  return f;
}
// The LDS bytes of a launch of that form (alds: A staged in LDS, forced by the fused transform).
size_t gemv_form_lds(int M, int K, int N, int SKG, bool have_ws, bool sk1, bool xf) {
  const GemvForm f = gemv_form(M, N, SKG, have_ws, sk1, xf);
  const int ktw = K / 16 / SKG;
  const bool alds = xf || gemv_ktl_pad(f.SK, ktw) * M * 32 <= kAldsMax;
  return gemv_lds(f.MT, f.NPW, f.SK, alds, ktw, M);
}

template <int KB, int MT, int NPW, int SK, bool ALDS, int XF, bool WQ = false>
void launch_gemv(const r4d_gemv_args& a) {
  dim3 grid(a.N / 32 / NPW, a.SKG), block(64 * NPW * SK);
  const int ktw = a.K / 16 / a.SKG;
  const size_t smem = gemv_lds(MT, NPW, SK, ALDS, ktw, a.M);
  if (smem > 160 * 1024) r4d::fail("gemm_trellis_nt_m64", "LDS request above 160 KiB");
  static std::atomic<unsigned long long> lds_set{0};
  if (smem > 64 * 1024)
    r4d::allow_lds((const void*)tq_gemv_kernel<KB, MT, NPW, SK, ALDS, XF, WQ>, lds_set, "gemm_trellis_nt_m64");
  const R4AParts ap = r4_parts((const void*)a.a0, (const void*)a.a1, a.n_split, (const void*)a.a2, a.n_end1,
                               (const void*)a.a3, a.n_end2);
  R4SParts sp;
  sp.s[0] = (const float*)a.suh0;
  sp.s[1] = (const float*)(a.suh1 ? a.suh1 : a.suh0);
  sp.s[2] = a.suh2 ? (const float*)a.suh2 : sp.s[1];
  sp.s[3] = a.suh3 ? (const float*)a.suh3 : sp.s[2];
  hipLaunchKernelGGL((tq_gemv_kernel<KB, MT, NPW, SK, ALDS, XF, WQ>), grid, block, smem, (hipStream_t)a.stream, ap,
                     (const unsigned*)a.w, (const float*)a.svh, (void*)a.c, (float*)a.ws,
                     (unsigned*)a.tickets, a.M, a.K, a.N, a.SKG, a.full, a.out_scale, sp, a.xscale,
                     (unsigned long long*)a.clk,
                     (const float*)a.wsc, a.wq_gsh);
}

template <int KB, int MT, int NPW, int SK>
void launch_gemv_a(const r4d_gemv_args& a) {
  const int ktw = a.K / 16 / a.SKG;
  const size_t abytes = gemv_ktl_pad(SK, ktw) * a.M * 32;
  if (a.xf) {
    if (abytes > kXfAldsMax) r4d::fail("trellis_gemv_xf", "the A slice does not fit LDS: raise SKG");
    if (a.xf == 2) launch_gemv<KB, MT, NPW, SK, true, 2>(a);
    else launch_gemv<KB, MT, NPW, SK, true, 1>(a);
  } else if (a.wsc) {
    if constexpr (KB == 4 || KB == 5) {
      if (abytes <= kAldsMax) launch_gemv<KB, MT, NPW, SK, true, 0, true>(a);
      else launch_gemv<KB, MT, NPW, SK, false, 0, true>(a);
    } else {
      r4d::fail("gemm_trellis_nt_m64_wq", "KB must be 4 or 5");
    }
  } else if (abytes <= kAldsMax) {
    launch_gemv<KB, MT, NPW, SK, true, 0>(a);
  } else {
    launch_gemv<KB, MT, NPW, SK, false, 0>(a);
  }
}

// The whole-group form (one wave per pair over the slice) at SK = 1 or for an unsplit launch without ws;
// else the split form: each pair's slice split over 4 waves, one pair per workgroup at M = 1 and two at
// M >= 2 (measured best; the pairs of a workgroup are independent, so the form does not change a bit,
// and fewer workgroups take fewer tickets on the group's counter).
template <int KB, int MT>
void launch_gemv_np(const r4d_gemv_args& a) {
  const GemvForm f = gemv_form(a.M, a.N, a.SKG, a.ws != 0 && a.tickets != 0, a.sk1 != 0, a.xf != 0);
  if (f.SK == 1) launch_gemv_a<KB, MT, 4, 1>(a);
  else if (f.NPW == 1) launch_gemv_a<KB, MT, 1, 4>(a);
  else launch_gemv_a<KB, MT, 2, 4>(a);
}

template <int KB>
void launch_gemv_kb(const r4d_gemv_args& a) {
  const int mt = gemv_form(a.M, a.N, a.SKG, true, false).MT;
  if (mt <= 1) launch_gemv_np<KB, 1>(a);
  else if (mt <= 2) launch_gemv_np<KB, 2>(a);
  else launch_gemv_np<KB, 4>(a);
}

}  // namespace

// ---- host entries ------------------------------------------------------------------------------
void r4d::gemv_run(r4d_gemv_args& a, const char* entry) {
  if (!a.a0 || !a.w || !a.c) r4d::fail(entry, "null A, W or C");
  if (const char* m = r4d_gemm_trellis_nt_m64_check(a.M, a.K, a.N, a.n_split, a.KB, a.SKG, a.full,
                                                    a.svh != 0, a.ws != 0 && a.tickets != 0))
    r4d::fail(entry, m);
  if (a.KB == 4) launch_gemv_kb<4>(a);
  else if (a.KB == 5) launch_gemv_kb<5>(a);
  else launch_gemv_kb<3>(a);
  r4d::launch_ok(entry);
}

// Grid-stride zero fill of `words` u32 words and `tail` (0..3) trailing bytes.
__global__ __launch_bounds__(256) void r4_clear_kernel(unsigned* __restrict__ p, size_t words, int tail) {
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < words; i += stride) p[i] = 0u;
  if (blockIdx.x == 0 && (int)threadIdx.x < tail) ((unsigned char*)(p + words))[threadIdx.x] = 0;
}

namespace r4d {
void launch_clear(void* p, size_t bytes, hipStream_t st, const char* entry) {
  if (bytes == 0) return;
  const size_t words = bytes / 4;
  size_t blocks = (words + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 1024) blocks = 1024;
  hipLaunchKernelGGL(r4_clear_kernel, dim3((unsigned)blocks), dim3(256), 0, st, (unsigned*)p, words, (int)(bytes & 3));
  launch_ok(entry);
}
}  // namespace r4d

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
  else if ((size_t)SKG * (size_t)M * (size_t)N * 4u > ((size_t)1 << 31))
    e = "the split partials SKG * M * N * 4 bytes must fit 2 GiB (32-bit offsets of the finish): lower SKG";
  return r4d::check_result(e);
}


void r4d_gemm_trellis_nt_m64(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t svh, int64_t c,
                             int64_t ws, int64_t tickets, int M, int K, int N, int KB, int WV, int SK,
                             int MT, int NP, int SKG, int U, int NT, float out_scale, int64_t stream) {
  (void)WV; (void)MT; (void)NP; (void)U; (void)NT;
  r4d_gemv_args a{a0, a1, n_split, w, svh, c, ws, tickets, M, K, N, KB, SKG, 1, out_scale, stream};
  a.sk1 = SK == 1 || SK == 2;
  r4d::gemv_run(a, "gemm_trellis_nt_m64");
}

void r4d_gemm_trellis_nt_m64_raw(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t c, int64_t ws,
                                 int64_t tickets, int M, int K, int N, int KB, int WV, int SK, int MT,
                                 int NP, int SKG, int U, int NT, int64_t clk, int64_t stream) {
  (void)WV; (void)MT; (void)NP; (void)U; (void)NT;
  r4d_gemv_args a{a0, a1, n_split, w, 0, c, ws, tickets, M, K, N, KB, SKG, 0, 1.f, stream};
  a.sk1 = SK == 1 || SK == 2;
  a.clk = clk;
  r4d::gemv_run(a, "gemm_trellis_nt_m64_raw");
}

// r4d.h:425-450: the fake-quant measurement entries -- r4d_gemm_trellis_nt_m64 / _raw with every decoded weight
// rounded to int8 under its (column, 2^gsh k-tile group) scale before the MFMA; the legality is the entry's own,
// plus KB 4 or 5, gsh 1..3 with 16 << gsh dividing K, and a non-null table.
static void wq_check(int K, int KB, int64_t wscale, int gsh, const char* entry) {
  if (!wscale) r4d::fail(entry, "the _wq entry needs a scale table (r4d_trellis_wscale_f32)");
  if (gsh < 1 || gsh > 3 || K % (16 << gsh)) r4d::fail(entry, "gsh must be 1, 2 or 3 with 16 << gsh dividing K");
  if (KB != 4 && KB != 5) r4d::fail(entry, "KB must be 4 or 5");
}
void r4d_gemm_trellis_nt_m64_wq(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t svh, int64_t c, int64_t ws,
                                int64_t tickets, int M, int K, int N, int KB, int WV, int SK, int MT, int NP, int SKG,
                                int U, int NT, float out_scale, int64_t wscale, int gsh, int64_t stream) {
  (void)WV; (void)MT; (void)NP; (void)U; (void)NT;
  wq_check(K, KB, wscale, gsh, "gemm_trellis_nt_m64_wq");
  r4d_gemv_args a{a0, a1, n_split, w, svh, c, ws, tickets, M, K, N, KB, SKG, 1, out_scale, stream};
  a.sk1 = SK == 1 || SK == 2;
  a.wsc = wscale;
  a.wq_gsh = gsh;
  r4d::gemv_run(a, "gemm_trellis_nt_m64_wq");
}
void r4d_gemm_trellis_nt_m64_raw_wq(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t c, int64_t ws,
                                    int64_t tickets, int M, int K, int N, int KB, int WV, int SK, int MT, int NP,
                                    int SKG, int U, int NT, int64_t wscale, int gsh, int64_t stream) {
  (void)WV; (void)MT; (void)NP; (void)U; (void)NT;
  wq_check(K, KB, wscale, gsh, "gemm_trellis_nt_m64_raw_wq");
  r4d_gemv_args a{a0, a1, n_split, w, 0, c, ws, tickets, M, K, N, KB, SKG, 0, 1.f, stream};
  a.sk1 = SK == 1 || SK == 2;
  a.wsc = wscale;
  a.wq_gsh = gsh;
  r4d::gemv_run(a, "gemm_trellis_nt_m64_raw_wq");
}
// r4d.h:433-436, 441-442
size_t r4d_trellis_wscale_count(int K, int N, int gsh) {
  if (K <= 0 || N <= 0 || gsh < 1 || gsh > 3) return 0;
  return (size_t)((K / 16) >> gsh) * (size_t)N;
}
void r4d_trellis_wscale_f32(int64_t w, int64_t scale, int K, int N, int KB, int gsh, int64_t stream) {
  const char* e = "trellis_wscale_f32";
  if (!w || !scale) r4d::fail(e, "null w or scale");
  if (KB != 4 && KB != 5) r4d::fail(e, "KB must be 4 or 5");
  if (N <= 0 || N % 32) r4d::fail(e, "N must be a positive multiple of 32");
  if (gsh < 1 || gsh > 3 || K <= 0 || K % (16 << gsh) || (K / 16) % 4) r4d::fail(e, "gsh 1..3, 16 << gsh and 64 dividing K");
  const int ktb = (1 << gsh) > 4 ? (1 << gsh) : 4;
  const long long waves = (long long)(N / 32) * ((K / 16) / ktb);
  dim3 grid((unsigned)((waves + 3) / 4)), block(256);
  if (KB == 4) hipLaunchKernelGGL(tq_wscale_kernel<4>, grid, block, 0, (hipStream_t)stream, (const unsigned*)w, (float*)scale, K, N, gsh);
  else hipLaunchKernelGGL(tq_wscale_kernel<5>, grid, block, 0, (hipStream_t)stream, (const unsigned*)w, (float*)scale, K, N, gsh);
  r4d::launch_ok(e);
}

// No reference counterpart: r4d_gemm_trellis_nt_m64 over up to four input parts -- the projections that share
// one input (q | k | v, qkv | z) laid out as one linear whose column ranges read their own transformed input
// (a[p] for columns [n0[p], n0[p + 1])), one launch instead of one per projection. Columns compute exactly as in
// the one-part launch of that range at the same SKG.
const char* r4dx_gemm_trellis_nt_m64_parts_check(int parts, const int* n0, int M, int K, int N, int KB, int SKG,
                                                 int have_ws) {
  const std::string e = r4d::parts_rule(parts, n0, N);
  if (!e.empty()) return r4d::check_result(e);
  return r4d_gemm_trellis_nt_m64_check(M, K, N, parts > 1 ? n0[1] : N, KB, SKG, 1, 1, have_ws);
}

void r4dx_gemm_trellis_nt_m64_parts(const int64_t* a, const int* n0, int parts, int64_t w, int64_t svh, int64_t c,
                                    int64_t ws, int64_t tickets, int M, int K, int N, int KB, int SKG,
                                    float out_scale, int64_t stream) {
  const char* e = "gemm_trellis_nt_m64_parts";
  if (!a || !n0) r4d::fail(e, "null part arrays");
  if (const char* m = r4dx_gemm_trellis_nt_m64_parts_check(parts, n0, M, K, N, KB, SKG, ws != 0 && tickets != 0))
    r4d::fail(e, m);
  for (int p = 0; p < parts; ++p)
    if (!a[p]) r4d::fail(e, "null part input");
  r4d_gemv_args g{a[0], parts > 1 ? a[1] : 0, parts > 1 ? n0[1] : N, w, svh, c, ws, tickets, M, K, N, KB, SKG, 1,
                  out_scale, stream};
  if (parts > 2) { g.a2 = a[2]; g.n_end1 = n0[2]; }
  if (parts > 3) { g.a3 = a[3]; g.n_end2 = n0[3]; }
  r4d::gemv_run(g, e);
}

// No reference counterpart: the input transform of r4dx_trellis_input_f16 / _bf16 fused into the GEMV.
const char* r4dx_trellis_gemv_xf_check(int M, int K, int N, int n_split, int KB, int SKG, int have_ws) {
  if (const char* m = r4d_gemm_trellis_nt_m64_check(M, K, N, n_split, KB, SKG, 1, 1, have_ws)) return m;
  std::string e;
  if ((K / 128) % SKG) e = "the fused transform needs whole 128-blocks per slice: (K / 128) % SKG == 0";
  else {
    const GemvForm f = gemv_form(M, N, SKG, have_ws != 0, false, true);
    if (gemv_ktl_pad(f.SK, K / 16 / SKG) * M * 32 > kXfAldsMax) e = "the A slice does not fit LDS: raise SKG";
    else if (gemv_form_lds(M, K, N, SKG, have_ws != 0, false, true) > 160 * 1024)
      e = "the A slice, the split partials and the finish buffers exceed 160 KiB of LDS: lower M or raise SKG";
  }
  return r4d::check_result(e);
}

void r4dx_trellis_gemv_xf(int64_t x, int x_is_bf16, int64_t suh0, int64_t suh1, int n_split, int prescale_log2,
                          int64_t w, int64_t svh, int64_t c, int64_t ws, int64_t tickets, int M, int K, int N, int KB,
                          int SKG, float out_scale, int64_t stream) {
  const char* entry = "trellis_gemv_xf";
  if (!x || !suh0 || !w || !c) r4d::fail(entry, "null x, suh, W or C");
  if (!suh1 && n_split != N) r4d::fail(entry, "a one-part launch (suh1 = 0) needs n_split = N");
  if (prescale_log2 < -24 || prescale_log2 > 24) r4d::fail(entry, "|prescale_log2| must be <= 24");
  if (const char* m = r4dx_trellis_gemv_xf_check(M, K, N, n_split, KB, SKG, ws != 0 && tickets != 0))
    r4d::fail(entry, m);
  r4d_gemv_args a{x, 0, n_split, w, svh, c, ws, tickets, M, K, N, KB, SKG, 1, out_scale, stream};
  a.suh0 = suh0;
  a.suh1 = suh1;
  a.xf = x_is_bf16 ? 2 : 1;
  // float(2^s / sqrt(128)), rounded once from double (trellis_ref.hpp:146-148)
  a.xscale = (float)(__builtin_ldexp(1.0, prescale_log2) / __builtin_sqrt(128.0));
  if (a.KB == 4) launch_gemv_kb<4>(a);
  else if (a.KB == 5) launch_gemv_kb<5>(a);
  else launch_gemv_kb<3>(a);
  r4d::launch_ok(entry);
}

// No reference counterpart: r4dx_trellis_gemv_xf over up to four column parts, each with its own suh -- the input
// transform of r4dx_trellis_input_* (nout = parts) fused into r4dx_gemm_trellis_nt_m64_parts: projections that read
// one input x (q | k | v, gdn qkv | z) stored as one linear run as ONE launch. Columns [n0[p], n0[p + 1]) use suh[p];
// every column equals the two-launch form (the transform, then the parts launch at the same SKG) bit for bit.
const char* r4dx_trellis_gemv_xf_parts_check(int parts, const int* n0, int M, int K, int N, int KB, int SKG,
                                             int have_ws) {
  const std::string e = r4d::parts_rule(parts, n0, N);
  if (!e.empty()) return r4d::check_result(e);
  return r4dx_trellis_gemv_xf_check(M, K, N, parts > 1 ? n0[1] : N, KB, SKG, have_ws);
}

void r4dx_trellis_gemv_xf_parts(int64_t x, int x_is_bf16, const int64_t* suh, const int* n0, int parts,
                                int prescale_log2, int64_t w, int64_t svh, int64_t c, int64_t ws, int64_t tickets,
                                int M, int K, int N, int KB, int SKG, float out_scale, int64_t stream) {
  const char* entry = "trellis_gemv_xf_parts";
  if (!suh || !n0) r4d::fail(entry, "null part arrays");
  if (!x || !w || !c || !svh) r4d::fail(entry, "null x, W, svh or C");
  if (prescale_log2 < -24 || prescale_log2 > 24) r4d::fail(entry, "|prescale_log2| must be <= 24");
  if (const char* m = r4dx_trellis_gemv_xf_parts_check(parts, n0, M, K, N, KB, SKG, ws != 0 && tickets != 0))
    r4d::fail(entry, m);
  for (int p = 0; p < parts; ++p)
    if (!suh[p]) r4d::fail(entry, "null part suh");
  r4d_gemv_args a{x, parts > 1 ? x : 0, parts > 1 ? n0[1] : N, w, svh, c, ws, tickets, M, K, N, KB, SKG, 1, out_scale,
                  stream};
  if (parts > 2) { a.a2 = x; a.n_end1 = n0[2]; }
  if (parts > 3) { a.a3 = x; a.n_end2 = n0[3]; }
  a.suh0 = suh[0];
  a.suh1 = parts > 1 ? suh[1] : 0;
  a.suh2 = parts > 2 ? suh[2] : 0;
  a.suh3 = parts > 3 ? suh[3] : 0;
  a.xf = x_is_bf16 ? 2 : 1;
  a.xscale = (float)(__builtin_ldexp(1.0, prescale_log2) / __builtin_sqrt(128.0));
  if (a.KB == 4) launch_gemv_kb<4>(a);
  else if (a.KB == 5) launch_gemv_kb<5>(a);
  else launch_gemv_kb<3>(a);
  r4d::launch_ok(entry);
}

int r4d_gemm_trellis_nt_m64_has_rate(int KB) { return KB == 3 || KB == 4 || KB == 5; }
int r4d_gemm_trellis_nt_m64_max_m(void) { return 64; }
size_t r4d_gemm_trellis_nt_m64_ws_bytes(int M, int N, int SKG) {
  return (size_t)SKG * (size_t)M * (size_t)N * sizeof(float);
}
// One 128-byte line per 128-column group (the counter in its first word): the contributors of different groups
// then never meet on one cache line's atomics.
size_t r4d_gemm_trellis_nt_m64_tickets_bytes(int N) {
  return (size_t)(N > 0 ? N / 128 : 0) * R4_TICKET_WORDS * sizeof(unsigned);
}

void r4d_gemm_trellis_nt_m64_zero_tickets(int64_t tickets, size_t bytes, int64_t stream) {
  if (bytes == 0) return;
  if (tickets == 0) r4d::fail("gemm_trellis_nt_m64_zero_tickets", "null buffer");
  if (tickets & 3) r4d::fail("gemm_trellis_nt_m64_zero_tickets", "tickets must be 4-byte aligned");
  r4d::launch_clear((void*)tickets, bytes, (hipStream_t)stream, "gemm_trellis_nt_m64_zero_tickets");
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

// This build's split choice for the GEMV, measured on MI355X over the 27B shapes and their same-input merges
// (KB 4, M = 1 and 8): among the powers of two 2..8 dividing K/16 (the engine's tuning rows hold no other SKG:
// TrellisRowFits, src/model/linear.cpp:243-255) that leave each of a slice's 4 waves at least 16 k-tiles, the
// ones that launch at least 6 waves per CU are preferred, and of those the one closest to 32 k-tiles per wave
// (log distance; ties to the larger SKG); with none, the largest. E.g. K = 5120: SKG 2 from N = 6144 on
// (16384 columns: 18.2 us against 20.1 at SKG 4), 4 for N = 1024; K = 6144, N = 5120: 4.
// Depends on the shape only, so every M <= 16 gets the same row bits.
int r4d_mi355x_trellis_gemv_skg(int K, int N, int KB) {
  (void)KB;
  const int KT = K / 16;
  if (KT <= 0 || N <= 0) return 1;
  int cus = 256, dev = 0;
  if (hipGetDevice(&dev) == hipSuccess) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) cus = n;
  }
  const long long want = 6LL * cus;
  int best = 0, fallback = 1;
  double best_d = 1e30;
  for (int d = 2; d <= 8 && d <= KT; d *= 2) {
    if (KT % d) continue;
    const double per_wave = (double)KT / d / 4.0;
    if (per_wave < 16.0) continue;
    fallback = d;
    if ((long long)(N / 32) * 4 * d < want) continue;
    const double dist = per_wave > 32.0 ? per_wave / 32.0 : 32.0 / per_wave;
    if (dist <= best_d) {
      best = d;
      best_d = dist;
    }
  }
  // Workgroups per CU at the pick (the M = 1 form: one per pair and slice). Below 1.25 most of the chip idles;
  // between x.25 and x.75 under 4, a quarter to three quarters of the CUs run one more workgroup than the rest.
  // The next split then spreads the work more evenly, as long as each wave keeps >= 10 k-tiles. Measured, SKG
  // before -> after at M = 1 / M = 8 (us): 6144x5120 4 -> 8: 9.7 -> 9.1 / 13.0 -> 11.8; 5120x6144 2 -> 4:
  // 10.5 -> 9.4 / 12.3 -> 12.0; 5120x10240 2 -> 4: 13.6 -> 12.3 / 18.4 -> 15.6; 5120x1024 4 -> 8: 5.9 -> 5.6 /
  // 8.6 -> 7.7; 5120x5120 4 -> 8: 9.2 -> 8.6 / 12.1 -> 11.9.
  int pick = best ? best : fallback;
  while (pick < 8 && KT % (2 * pick) == 0 && KT / (2 * pick) >= 40) {
    const double per_cu = (double)(N / 32) * pick / cus;
    const double frac = per_cu - (long long)per_cu;
    if (!(per_cu < 1.25 || (per_cu < 4.0 && frac >= 0.25 && frac <= 0.75))) break;
    pick *= 2;
  }
  return pick;
}

}  // extern "C"

