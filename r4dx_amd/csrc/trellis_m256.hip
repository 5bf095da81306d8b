// trellis_m256.hip -- the trellis linear for a 256- (or 128-) row prefill chunk in one launch on gfx950:
// r4d_gemm_trellis_nt_m256, _check, _ws_bytes (the C ABI of the reference's third_party/libr4d/r4d.h:
// 395-423) and this build's _raw fp32 entry.
//
// C[m][n] = bf16((FWHT128(A_p(n) @ Q)[m][n] * svh[n]) * out_scale), A f16 [M][K] (M = 128 or 256).
//
// DESIGN (MI355X): MFMA-bound. A workgroup is 8 waves = all M rows x one 128-column group x one K slice: 4 producer
// waves load the step's A rows and decode one tile pair each (the GEMV's decode, r4d_dev.h) into a double-buffered
// LDS stage, 4 math waves run v_mfma_f32_16x16x32_f16 over it (details at the kernel). Each weight is decoded once for
// all M rows. Unsplit, the epilogue applies the FWHT-128 in the accumulator layout (stages in the reference's order),
// then svh, out_scale, one bf16 rounding. Split K (chosen only where it shortens the critical path: the partial sums
// are M x N fp32 per slice) writes each slice to ws and a second launch, tq_m256_finish, adds the slices in order
// and finishes. Unit counts that are not a multiple of the compute units run in the balanced form (one workgroup per
// CU over an even share of the steps, a cut unit's accumulators handed on exactly; see the kernel).
#include "r4d_dev.h"
#include "r4d_host.h"
#include "r4d_mi355x.h"

namespace {

typedef __amdgpu_buffer_rsrc_t r4_rsrc;
__device__ __forceinline__ r4_rsrc mk_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)bytes, 0x00020000);
}

// A workgroup is 8 waves over all M rows x one 128-column group x one K slice, in 64-k steps through a
// double-buffered LDS stage:
//   * 4 producer waves: producer p loads rows [p M/4, (p+1) M/4) of the step's A (coalesced: 8 lanes per
//     128-byte row segment) and the words of tile pair p, decodes them, and writes both into the stage;
//   * 4 math waves: math wave (rh, ch) owns rows [rh M/2, +M/2) x columns [64 ch, +64) of the group =
//     RT = M / 32 row tiles x 4 column tiles of v_mfma_f32_16x16x32_f16, reading A and B from LDS.
// A and B are stored in the M <= 64 kernel's MFMA operand order, so that every output element sees the
// same MFMAs with the same operands in the same order and the results agree bit for bit: the 16-byte
// chunk 4 h + g of a step holds fragment half h of k-tile g (element e <-> k = 8 (e >> 2) + 4 h + (e & 3)),
// and MFMA half kh reads chunks 4 kh + 0..3. A is [row][8 chunks], written as 8-byte quads (a lane's
// natural 8 k split into its h = 0 and h = 1 quads); B is [chunk][column], the decode's d[cs][h] as is.
// Chunk c of row r sits at slot c ^ m2_swz(r), so the 16 rows a fragment read touches use 16 distinct
// bank groups. (Natural-order A chunks with 16-byte writes measured ~3 % faster, but pair k differently
// inside an MFMA; reading them back as two 8-byte halves costs 25 % in read conflicts.)
constexpr int kM2Waves = 8;
// j = (r >> 1) & 7 with bit 2 flipped by bit 0: still 16 distinct slots for a fragment read's 16 rows, and
// the 8-byte quad writes of 8 consecutive rows (4 chunks per row and half h) use both 64-byte chunk groups
__device__ __forceinline__ int m2_swz(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int m2_slot(int r, int c) { return (r * 8 + (c ^ m2_swz(r))) * 16; }
// B is [chunk][column] instead: a decode lane writes columns 32 p + 16 t + 8 cs + c, so column bit 3 is
// flipped on odd 16-column tiles to keep the t = 0 and t = 1 lanes of one write on different banks; a
// fragment read (16 consecutive columns of one chunk) stays a permutation of 16 bank slots.
__device__ __forceinline__ int m2_bslot(int n, int c) { return c * 2048 + ((n ^ (((n >> 4) & 1) << 3)) * 16); }

// The work of a launch is U = (N / 128) * SKG units -- unit u = group * SKG + y is K slice y of column group u / SKG
// -- of nst steps each, taken in unit order. Data-parallel (P = 0): workgroup (group, y) takes one unit. Balanced
// (P > 0 workgroups, used when U exceeds the CUs and is not a multiple of them): workgroup c takes the steps
// an even share (T / P, one more for the first T % P) of the T = U nst, P <= U so that a range spans at most the end of one unit, whole units
// and the start of one more. A unit cut by a range boundary stays one fold from 0.f in k order: the workgroup that
// holds its start runs that part FIRST and publishes the fp32 accumulators (fix[c], M x 128; then flags[4 c] = 1),
// the workgroup that holds the rest runs it LAST, starting from those accumulators (so every element is the same
// sum, bit for bit). Workgroups are dispatched in index order and the publisher's part is its first work, so the
// wait cannot deadlock; it is bounded anyway, and a wait that runs out poisons its results with NaN.
constexpr int kSegWhole = 0, kSegPublish = 1, kSegContinue = 2;
constexpr int kFlagStride = 4;            // words between two workgroups' flags
// Workgroup c's flag is word kFlagStride c + 1 of the ticket buffer: never word 32 g, the counter of 128-column group g
// that the M <= 64 kernel's split hand-over takes tickets on, so a flag left set can never be read as a ticket count.
__device__ __forceinline__ unsigned* m2_flag(unsigned* flags, unsigned c) { return flags + (size_t)c * kFlagStride + 1; }

// A workgroup's share: steps [beg, end) of the launch's units in order (unit u = group * SKG + y, nst steps each).
struct M2Share {
  int ub, sb, ue, se, whole0, nseg;
};
__device__ __forceinline__ M2Share m2_share(int N, int SKG, int nst, int P) {
  // T = (N / 128) * SKG * nst <= (N / 128) * K / 64 steps fits 32 bits; workgroup c gets T / P steps, one more for the
  // first T % P workgroups
  int beg, end;
  if (P > 0) {
    const unsigned T = (unsigned)(N / 128) * (unsigned)SKG * (unsigned)nst, q = T / (unsigned)P, r = T % (unsigned)P;
    const unsigned c = blockIdx.x;
    beg = (int)(c * q + (c < r ? c : r));
    end = beg + (int)q + (c < r ? 1 : 0);
  } else {
    beg = (blockIdx.x * SKG + blockIdx.y) * nst;
    end = beg + nst;
  }
  M2Share sh;
  sh.ub = beg / nst; sh.sb = beg - sh.ub * nst; sh.ue = end / nst; sh.se = end - sh.ue * nst;
  sh.whole0 = sh.sb ? sh.ub + 1 : sh.ub;
  sh.nseg = (sh.se ? 1 : 0) + (sh.ue - sh.whole0) + (sh.sb ? 1 : 0);
  return sh;
}
// Segment si in run order: the start of unit ue (published), the whole units, the rest of unit ub (continued).
struct M2Seg {
  int u, s0, s1, kind;
};
__device__ __forceinline__ M2Seg m2_seg(const M2Share& sh, int si, int nst) {
  M2Seg g;
  if (sh.se && si == 0) { g.u = sh.ue; g.s0 = 0; g.s1 = sh.se; g.kind = kSegPublish; }
  else if (sh.sb && si == sh.nseg - 1) { g.u = sh.ub; g.s0 = sh.sb; g.s1 = nst; g.kind = kSegContinue; }
  else { g.u = sh.whole0 + si - (sh.se ? 1 : 0); g.s0 = 0; g.s1 = nst; g.kind = kSegWhole; }
  return g;
}

// SK4: the M <= 64 kernel's 4-wave order (its SK 4, 8 and 16): each K slice's steps are cut into 4 contiguous parts of
// ceil(steps / 4) steps, each part summed from 0.f, the parts added in order ((p0 + p1) + p2) + p3 (an empty part adds
// +0.f); the slice then always goes through ws (or raw C) and tq_m256_finish, as that kernel's split hand-over does.
// Data-parallel only (P = 0), and with RT = 4: the finished parts' sum takes a second accumulator set.
template <int KB, int RT, bool WQ = false, bool SK4 = false>
__global__ __launch_bounds__(64 * kM2Waves, 1) void tq_m256_kernel(
    const R4AParts ap, const unsigned* __restrict__ W, const float* __restrict__ svh, void* __restrict__ Cv,
    float* __restrict__ ws, int M, int K, int N, int SKG, int full, float out_scale,
    const float* __restrict__ wsc, int wq_gsh, float* __restrict__ fix, unsigned* __restrict__ flags, int P) {
  constexpr int BLK = 16 * KB;                    // words per (pair, k-tile) block
  constexpr unsigned kStepBytes = 4 * BLK * 4;    // one pair's words per step
  constexpr int MR = 32 * RT;                     // rows of the launch (128 or 256)
  constexpr int kA = MR * 128, kStage = kA + 128 * 128;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int KT = K >> 4, ktw = KT / SKG;
  const int nst = ktw >> 2;                       // steps per unit

  const M2Share sh = m2_share(N, SKG, nst, P);

  // The segment preamble both roles run (the same barriers): segment geometry, then, for a continuation, one thread
  // waits for the previous workgroup's flag (and clears it for the next launch) and tells the workgroup whether it
  // came in time.
#define M2_SEGMENT_BEGIN                                                                                   \
    const M2Seg sg = m2_seg(sh, si, nst);                                                                  \
    int Kv = K, Nv = N;                                                                                    \
    asm volatile("" : "+s"(Kv), "+s"(Nv));                                                                 \
    const int kind = sg.kind;                                                                              \
    const int group = sg.u / SKG, ky = sg.u - group * SKG;                                                 \
    const int kt0 = ky * ktw + 4 * sg.s0;                                                                  \
    const int ns = sg.s1 - sg.s0;                                                                          \
    const int n0 = group * 128;                                                                            \
    const unsigned short* __restrict__ A = r4_part_a(ap, n0);                                              \
    __syncthreads();                                                                                       \
    bool poisoned = false;                                                                                 \
    if (kind == kSegContinue) {                                                                            \
      if (threadIdx.x == 0) {                                                                              \
        unsigned* f = m2_flag(flags, blockIdx.x - 1);                                                        \
        int spin = 0;                                                                                      \
        while (__hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u && spin < (1 << 24)) { \
          __builtin_amdgcn_s_sleep(8);                                                                     \
          ++spin;                                                                                          \
        }                                                                                                  \
        __hip_atomic_store(f, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);                             \
        *(volatile int*)lds = spin < (1 << 24) ? 0 : 1;                                                    \
      }                                                                                                    \
      __syncthreads();                                                                                     \
      poisoned = *(volatile int*)lds != 0;                                                                 \
      __syncthreads();                                                                                     \
    }                                                                                                      \
    (void)poisoned; (void)A; (void)Kv; (void)Nv; (void)kt0;

  if (wave >= 4) {
   for (int si = 0; si < sh.nseg; ++si) {
    M2_SEGMENT_BEGIN
    {
      // ---- producer p
      const int p = wave - 4;
      const int q = lane >> 4, t = (lane >> 3) & 1, c = lane & 7;
      const int pair = group * 4 + p;
      const r4_rsrc wr = mk_rsrc(W + ((size_t)pair * KT + kt0) * BLK, (unsigned)ns * kStepBytes);
      const unsigned tile = (unsigned)(q * 16 * KB + t * 8 * KB);
      const unsigned own = (tile + KB * c) * 4u, hist = (tile + (KB * c - 1 + 8 * KB) % (8 * KB)) * 4u;
      constexpr int RA = MR / 4, AU = RA / 8;     // rows per producer; 16-byte loads per lane per step
      const r4_rsrc ar = mk_rsrc(A, (unsigned)((size_t)MR * Kv * 2));
      // load u covers rows {a, a+1, a+2, a+3, a+8, .., a+11}, a = 4 (u & 1) + 16 (u >> 1), lane group i = lane >> 3
      // taking row a + (i & 1) + 8 ((i >> 1) & 1) + 2 (i >> 2): each 32-lane half of a quad write then holds rows
      // whose swizzles differ in bit 2 (two disjoint 64-byte chunk groups), so the writes are free of bank conflicts
      const int li = lane >> 3, ac = lane & 7;
      const int ar0 = p * RA + (li & 1) + 8 * ((li >> 1) & 1) + 2 * (li >> 2);
      auto arow = [&](int uu) { return ar0 + 4 * (uu & 1) + 16 * (uu >> 1); };
      const unsigned aoff = (unsigned)(((size_t)ar0 * Kv + (size_t)kt0 * 16 + ac * 8) * 2);

      struct St {
        unsigned w[KB + 1];
        r4u4 a[AU];
      };
      auto load = [&](St& s, int st) {
        const int sc = min(st, ns - 1);
        const unsigned so = (unsigned)sc * kStepBytes;
        // one wide load per lane (dword alignment suffices): KB 4 a dwordx4, KB 5 a dwordx4 and a dword, KB 3 a dwordx3
        if constexpr (KB == 4 || KB == 5) {
          const r4u4 v = __builtin_bit_cast(r4u4, __builtin_amdgcn_raw_buffer_load_b128(wr, own + so, 0, 0));
          s.w[1] = v[0]; s.w[2] = v[1]; s.w[3] = v[2]; s.w[4] = v[3];
          if constexpr (KB == 5) s.w[5] = __builtin_amdgcn_raw_buffer_load_b32(wr, own + so + 16, 0, 0);
        } else {
          const auto v = __builtin_amdgcn_raw_buffer_load_b96(wr, own + so, 0, 0);
          s.w[1] = v[0]; s.w[2] = v[1]; s.w[3] = v[2];
        }
        s.w[0] = __builtin_amdgcn_raw_buffer_load_b32(wr, hist + so, 0, 0);
#pragma unroll
        for (int uu = 0; uu < AU; ++uu)
          s.a[uu] = __builtin_bit_cast(r4u4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 ar, aoff + (unsigned)((arow(uu) - ar0) * Kv * 2) + (unsigned)sc * 128u, 0, 0));
      };
      auto put = [&](const St& s, int st) {
        unsigned char* stg = lds + (st & 1) * kStage;
        // chunk 4 h + g of a row = fragment half h of k-tile g (k 4h..4h+3, 8+4h..8+4h+3), the M <= 64
        // kernel's MFMA operand order: the lane's 8 natural k (ac even: k 0-7, odd: 8-15 of k-tile ac >> 1)
        // split into its h = 0 and h = 1 quads
#pragma unroll
        for (int uu = 0; uu < AU; ++uu) {
          unsigned char* row = stg + (ac & 1) * 8;
          *(r4u2*)(row + m2_slot(arow(uu), ac >> 1)) = (r4u2){s.a[uu][0], s.a[uu][1]};
          *(r4u2*)(row + m2_slot(arow(uu), 4 + (ac >> 1))) = (r4u2){s.a[uu][2], s.a[uu][3]};
        }
        unsigned d[2][2][4];
        r4_decode<KB>(s.w, d);
        if constexpr (WQ) {
          // the _wq measurement: the producer rounds its tile pair's weights before publishing them, so every
          // row group's MFMA sees the same values the M <= 64 _wq kernel feeds its MFMA
          // (a put past the last step carries the clamped last step's words: use its k-tile, inside the table)
          const int kt = kt0 + min(st, ns - 1) * 4 + q;
          const size_t row = (size_t)(kt >> wq_gsh) * Nv + (size_t)pair * 32 + 16 * t + c;
          const float sc[2] = {wsc[row], wsc[row + 8]};
          r4_wq_apply(d, sc);
        }
#pragma unroll
        for (int cs = 0; cs < 2; ++cs) {
          const int n = 32 * p + 16 * t + 8 * cs + c;
#pragma unroll
          for (int h = 0; h < 2; ++h)
            *(r4u4*)(stg + kA + m2_bslot(n, 4 * h + q)) = (r4u4){d[cs][h][0], d[cs][h][1], d[cs][h][2], d[cs][h][3]};
        }
      };
      constexpr int PF = 2;
      St ring[PF];
#pragma unroll
      for (int i = 0; i < PF; ++i) load(ring[i], i);
      // stage 0 <- step 0; then, after barrier st, stage (st + 1) & 1 <- step st + 1. In the steady loop a
      // put past the last step writes the (clamped) last step into the stage nobody reads any more, so the
      // loop carries no branch; the remainder of ns % PF steps runs in the tail.
      put(ring[0], 0);
      load(ring[0], PF);
      int st = 0;
      for (; st + PF <= ns; st += PF) {
#pragma unroll
        for (int i = 0; i < PF; ++i) {
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          __builtin_amdgcn_s_barrier();
          put(ring[(i + 1) % PF], st + i + 1);
          load(ring[(i + 1) % PF], st + i + 1 + PF);
        }
      }
      static_assert(PF == 2, "the tail below names the two ring slots");
      for (; st < ns; ++st) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        // ring slots are named by constants only: a runtime index would move the whole ring to scratch memory
        if (st + 1 < ns) {
          if (((st + 1) & 1) == 0) put(ring[0], st + 1);
          else put(ring[1], st + 1);
        }
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      // the math waves' closing barriers: the publish handoff, or the epilogue's two exchange rounds
      if (kind == kSegPublish) {
        __syncthreads();
      } else if (SKG == 1 && full && !SK4) {
#pragma unroll 1
        for (int r = 0; r < 2 * 2; ++r) __syncthreads();
      }
    }
   }
    return;
  }

  for (int si = 0; si < sh.nseg; ++si) {
    M2_SEGMENT_BEGIN
    // ---- math wave (rh, ch)
    // the lane index passes through an empty asm at every segment, so the fragment addresses derived from it are
    // formed per segment instead of being hoisted out of the segment loop (live through the epilogue, they would
    // push the accumulators out of the register file)
    int lane_s = lane;
    asm volatile("" : "+v"(lane_s));
    const int rh = wave >> 1, ch = wave & 1;
    const int r16 = lane_s & 15, g = lane_s >> 4;
    r4f4 acc[RT][4];
    r4f4 tot[SK4 ? RT : 1][4];                     // SK4: the sum of the finished parts
    const int nsw = SK4 ? (ns + 3) / 4 : 0;        // SK4: steps per part
    int next_part = nsw, folds = 0;
    // SK4, at a part boundary: tot = p0, then tot + p1, ...; the next part starts from 0.f
    auto fold = [&]() {
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
          if constexpr (SK4) {
#pragma unroll
            for (int j = 0; j < 4; ++j) tot[i][ct][j] = folds == 0 ? acc[i][ct][j] : tot[i][ct][j] + acc[i][ct][j];
          }
          acc[i][ct] = (r4f4){0.f, 0.f, 0.f, 0.f};
        }
      ++folds;
    };
    // a published slot is [wave][i][ct][lane_s] r4f4: one coalesced 1 KiB run per (wave, i, ct)
    if (kind == kSegContinue) {
      // coherent (sc1) 16-byte loads: one per (i, ct), lane_s-contiguous, offsets constant past the lane_s's own
      const r4_rsrc fr = mk_rsrc(fix + (size_t)(blockIdx.x - 1) * MR * 128, (unsigned)(MR * 128 * 4));
      const float pv = poisoned ? __builtin_nanf("") : 0.f;
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
          const r4f4 v = __builtin_bit_cast(
              r4f4, __builtin_amdgcn_raw_buffer_load_b128(fr, (unsigned)lane_s * 16u, ((wave * RT + i) * 4 + ct) * 1024, 16));
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][ct][j] = v[j] + pv;
        }
    } else {
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) acc[i][ct] = (r4f4){0.f, 0.f, 0.f, 0.f};
    }
    const int arow = rh * (MR / 2) + r16, bcol = 64 * ch + r16;
    // Software pipeline by half steps (kh = 0, 1 = the step's two 32-k halves): the fragments of the next
    // half are read while the current half's MFMAs run, and the barrier sits between the halves, so neither
    // the LDS latency nor the barrier wait idles the MFMA pipe. The last step is peeled (no barrier after it:
    // the producers meet ns barriers too).
    auto read_half = [&](r4h8 (&af)[RT], r4h8 (&bf)[4], int st, int kh) {
      const unsigned char* stg = lds + (st & 1) * kStage;
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) bf[ct] = *(const r4h8*)(stg + kA + m2_bslot(bcol + 16 * ct, 4 * kh + g));
#pragma unroll
      for (int i = 0; i < RT; ++i) af[i] = *(const r4h8*)(stg + m2_slot(arow + 16 * i, 4 * kh + g));
    };
    auto mfma_half = [&](const r4h8 (&af)[RT], const r4h8 (&bf)[4]) {
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) acc[i][ct] = r4_mfma16(af[i], bf[ct], acc[i][ct]);
    };
    r4h8 af0[RT], bf0[4], af1[RT], bf1[4];
    __builtin_amdgcn_s_barrier();          // B_0: stage 0 landed
    read_half(af0, bf0, 0, 0);
    for (int st = 0; st + 1 < ns; ++st) {
      read_half(af1, bf1, st, 1);
      mfma_half(af0, bf0);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // this wave's reads of stage st done
      __builtin_amdgcn_s_barrier();                        // B_(st+1): stage st + 1 landed
      read_half(af0, bf0, st + 1, 0);
      mfma_half(af1, bf1);
      if constexpr (SK4) {
        if (st + 1 == next_part) {   // step st closed a part (uniform: a scalar branch)
          fold();
          next_part += nsw;
        }
      }
    }
    read_half(af1, bf1, ns - 1, 1);
    mfma_half(af0, bf0);
    mfma_half(af1, bf1);
    if constexpr (SK4) {
      // the last part added to the others; fewer than 4 non-empty parts: the empty ones' +0.f (once is all of them)
      const bool empty = (ns + nsw - 1) / nsw < 4;
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float v = folds > 0 ? tot[i][ct][j] + acc[i][ct][j] : acc[i][ct][j];
            if (empty) v = v + 0.f;
            acc[i][ct][j] = v;
          }
    }

    if (kind == kSegPublish) {
      // coherent (sc1, write-through) 16-byte stores in the layout the continuation reads
      const r4_rsrc fr = mk_rsrc(fix + (size_t)blockIdx.x * MR * 128, (unsigned)(MR * 128 * 4));
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(r4u4, acc[i][ct]), fr, (unsigned)lane_s * 16u,
                                                 ((wave * RT + i) * 4 + ct) * 1024, 16);
      // every store acknowledged before the barrier, then one thread raises the flag
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __syncthreads();
      if (threadIdx.x == 0)
        __hip_atomic_store(m2_flag(flags, blockIdx.x), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      continue;
    }

    // lane_s holds, for row tile i and column tile ct, rows rh M/2 + 16 i + 4 g + j, column 64 ch + 16 ct + r16; the
    // stores go through a buffer resource: the lane_s's own offset, the row (16 i + j) as a scalar offset, the column
    // tile as an immediate
    const int row0 = rh * (MR / 2);
    const unsigned lane_off = (unsigned)((row0 + 4 * g) * Nv + n0 + 64 * ch + r16);   // elements
    // the row stride as a VGPR: the 32 row offsets are formed at the stores (VALU) instead of living in SGPRs.
    // (__float_as_uint, not __builtin_bit_cast, on a vector element: this compiler's bit_cast of acc[i][ct][j]
    // reads element 0 whatever j is.)
    unsigned nvv = (unsigned)Nv;
    asm volatile("" : "+v"(nvv));
    if (SK4 || SKG > 1 || !full) {
      float* dst = SKG > 1 || (SK4 && full) ? ws + (size_t)ky * M * Nv : (float*)Cv;
      const r4_rsrc dr = mk_rsrc(dst, (unsigned)((size_t)M * Nv * 4));
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int ct = 0; ct < 4; ++ct)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][ct][j]), dr,
                                                  (lane_off + (unsigned)(16 * i + j) * nvv) * 4u + ct * 64, 0, 0);
      continue;
    }
    // FWHT-128 over the group's columns, stages lg = 0..6 in order on column bit lg (the lower index keeps
    // a + b, the upper takes a - b): bits 0-3 are lane bits 0-3, bits 4-5 the column tile, bit 6 the
    // column half ch, exchanged with the partner wave (rh, ch ^ 1) through LDS in two rounds of RT / 2 row
    // tiles (every wave of the workgroup meets both barriers of a round); a round's tiles take their stages 0-5
    // just before its exchange, so the other round's accumulators need no temporaries meanwhile.
    auto stages_0_5 = [&](int i) {
      auto lane_stage = [&](int mask) {
        const bool upper = (lane_s & mask) != 0;
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float o = r4_xor_lane(acc[i][ct][j], mask);
            acc[i][ct][j] = upper ? o - acc[i][ct][j] : acc[i][ct][j] + o;
          }
      };
      lane_stage(1);
      lane_stage(2);
      lane_stage(4);
      lane_stage(8);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float a0 = acc[i][0][j], b0 = acc[i][1][j], a1 = acc[i][2][j], b1 = acc[i][3][j];   // bit 4: ct ^ 1
        acc[i][0][j] = a0 + b0; acc[i][1][j] = a0 - b0; acc[i][2][j] = a1 + b1; acc[i][3][j] = a1 - b1;
        a0 = acc[i][0][j]; b0 = acc[i][2][j]; a1 = acc[i][1][j]; b1 = acc[i][3][j];           // bit 5: ct ^ 2
        acc[i][0][j] = a0 + b0; acc[i][2][j] = a0 - b0; acc[i][1][j] = a1 + b1; acc[i][3][j] = a1 - b1;
      }
      __builtin_amdgcn_sched_barrier(0);   // one row tile's stages at a time (bounded temporaries)
    };
    constexpr int RR = RT / 2;                     // row tiles per exchange round
    // exchange area [wave 0..3][RR][ct][lane]: this wave's run and its partner's, each one base plus constants
    r4f4* const xw = (r4f4*)lds + (size_t)wave * RR * 4 * 64 + lane_s;
    const r4f4* const xr = (const r4f4*)lds + (size_t)(wave ^ 1) * RR * 4 * 64 + lane_s;
    const r4_rsrc cr = mk_rsrc(Cv, (unsigned)((size_t)M * Nv * 2));
#pragma unroll
    for (int rd = 0; rd < 2; ++rd) {
#pragma unroll
      for (int ii = 0; ii < RR; ++ii) stages_0_5(rd * RR + ii);
      __syncthreads();                             // the stages (or the previous round) are no longer read
#pragma unroll
      for (int ii = 0; ii < RR; ++ii)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) xw[(ii * 4 + ct) * 64] = acc[rd * RR + ii][ct];
      __syncthreads();
      float sv[4];
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) sv[ct] = svh[n0 + 64 * ch + 16 * ct + r16];
#pragma unroll
      for (int ii = 0; ii < RR; ++ii) {
        const int i = rd * RR + ii;
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
          const r4f4 o = xr[(ii * 4 + ct) * 64];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float v = ch ? o[j] - acc[i][ct][j] : acc[i][ct][j] + o[j];
            __builtin_amdgcn_raw_buffer_store_b16(r4_bf16_rn_sel((v * sv[ct]) * out_scale), cr,
                                                  (lane_off + (unsigned)(16 * i + j) * nvv) * 2u + ct * 32, 0, 0);
          }
        }
      }
    }
  }
}
#undef M2_SEGMENT_BEGIN

// The split form's second pass: a workgroup per (128-column group, 16 rows) sums the SKG slices of ws in
// slice order into LDS, then one wave per row applies the group's FWHT-128 (r4_fwht128_wave, the reference's
// stage order), svh, out_scale and the bf16 rounding -- or, raw, stores the fp32 sums. Up to 8 slices (one per
// run): a thread takes 4 adjacent columns of 2 rows and requests all 8 slices of them at once as 16-byte
// loads (a slice past SKG reads past the buffer and returns 0, which is exactly what an empty run adds), so
// one memory round trip covers the workgroup; more slices take the general loop (a thread per column).
constexpr int kFinRows = 16;
__global__ __launch_bounds__(256) void tq_m256_finish(const float* __restrict__ ws, const float* __restrict__ svh,
                                                      void* __restrict__ Cv, int M, int N, int SKG, int full,
                                                      float out_scale) {
  __shared__ float sums[kFinRows][128];
  const int group = blockIdx.x, r0 = blockIdx.y * kFinRows;
  const int n0 = group * 128;
  const size_t sy = (size_t)M * N;
  // the M <= 64 kernel's slice order: run p (0..7) = 0.f + slices p, p + 8, ... in order, then the 8 runs
  // added in order 0..7
  if (SKG <= 8) {
    const int cq = threadIdx.x & 31, rr = threadIdx.x >> 5;      // columns 4 cq .. 4 cq + 3, rows rr, rr + 8
    const unsigned sy4 = (unsigned)sy * 4u;
    const r4_rsrc wr = mk_rsrc(ws, (unsigned)SKG * sy4);
    r4f4 t[8][2];
#pragma unroll
    for (int p = 0; p < 8; ++p)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const unsigned off = (unsigned)p * sy4 + (unsigned)((r0 + rr + 8 * u) * N + n0 + 4 * cq) * 4u;
        t[p][u] = __builtin_bit_cast(r4f4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0));
      }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float acc = 0.f + t[0][u][e];
#pragma unroll
        for (int p = 1; p < 8; ++p) acc = acc + (0.f + t[p][u][e]);
        v[e] = acc;
      }
      const int r = rr + 8 * u;
      if (!full) {
        *(r4f4*)((float*)Cv + (size_t)(r0 + r) * N + n0 + 4 * cq) = (r4f4){v[0], v[1], v[2], v[3]};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) sums[r][4 * cq + e] = v[e];
      }
    }
    if (!full) return;
  } else {
    const int col = threadIdx.x & 127, rh = threadIdx.x >> 7;   // rows rh + 2 u
    float v[kFinRows / 2];
#pragma unroll 1
    for (int p = 0; p < 8; ++p) {
      float run[kFinRows / 2];
#pragma unroll
      for (int u = 0; u < kFinRows / 2; ++u) run[u] = 0.f;
      for (int y = p; y < SKG; y += 8) {
        float t[kFinRows / 2];
#pragma unroll
        for (int u = 0; u < kFinRows / 2; ++u) t[u] = ws[(size_t)y * sy + (size_t)(r0 + rh + 2 * u) * N + n0 + col];
#pragma unroll
        for (int u = 0; u < kFinRows / 2; ++u) run[u] += t[u];
      }
#pragma unroll
      for (int u = 0; u < kFinRows / 2; ++u) v[u] = p == 0 ? run[u] : v[u] + run[u];
    }
    if (!full) {
      float* Cf = (float*)Cv;
#pragma unroll
      for (int u = 0; u < kFinRows / 2; ++u) Cf[(size_t)(r0 + rh + 2 * u) * N + n0 + col] = v[u];
      return;
    }
#pragma unroll
    for (int u = 0; u < kFinRows / 2; ++u) sums[rh + 2 * u][col] = v[u];
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  unsigned short* Cb = (unsigned short*)Cv;
  const float sv0 = svh[n0 + lane], sv1 = svh[n0 + lane + 64];
  for (int r = wave; r < kFinRows; r += 4) {
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
  // the kernel's stores and the split finish address one slice, and all SKG slices, with 32-bit buffer offsets
  if ((long long)SKG * M * N * 4 > (1LL << 31))
    return "the fp32 slices SKG * M * N * 4 bytes must fit 2 GiB (32-bit offsets of the split finish): lower SKG";
  return "";
}

// The device's compute units (cached per device).
int m256_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    cache[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cache[dev];
}
// Workgroups of the balanced form for a launch of U units (0: data-parallel): used when U exceeds the compute units and
// is not a multiple of them, and ws (for the published accumulators) and the tickets (for the flags) are there.
int m256_balanced_p(int M, int N, int SKG, bool have_ws, bool have_tickets) {
  (void)M;
  const int G = N / 128, U = G * SKG, cus = m256_cus();
  if (!have_ws || !have_tickets || U <= cus || U % cus == 0) return 0;
  if ((long long)cus * kFlagStride + 1 > (long long)G * R4_TICKET_WORDS) return 0;   // the flags fit the ticket buffer
  return cus;
}

template <int KB, int RT, bool WQ, bool SK4 = false>
void m256_launch_rt(const R4AParts& ap, const unsigned* w,
                    const float* svh, void* c, float* ws, unsigned* tickets, int M, int K, int N, int SKG, int full,
                    float out_scale, const float* wsc, int wq_gsh, hipStream_t st) {
  constexpr unsigned lds = 2 * (32 * RT * 128 + 128 * 128);
  static std::atomic<unsigned long long> lds_set{0};
  r4d::allow_lds((const void*)tq_m256_kernel<KB, RT, WQ, SK4>, lds_set, "gemm_trellis_nt_m256");
  const int P = SK4 ? 0 : m256_balanced_p(M, N, SKG, ws != nullptr, tickets != nullptr);
  // the published accumulators follow the SKG slices in ws (SKG = 1: no slices, they start at ws)
  float* fix = ws ? ws + (SKG > 1 ? (size_t)SKG * M * N : 0) : nullptr;
  const dim3 grid = P > 0 ? dim3(P) : dim3(N / 128, SKG);
  hipLaunchKernelGGL((tq_m256_kernel<KB, RT, WQ, SK4>), grid, dim3(64 * kM2Waves), lds, st, ap,
                     w, svh, c, ws, M, K, N, SKG, full, out_scale, wsc, wq_gsh, fix, tickets, P);
}
// The SK4 order, one launch per 128-row half (the 128-row form holds the second accumulator set): half h reads its
// parts' rows from 128 h, writes C's rows from 128 h (bf16, or fp32 raw) and, through ws, its own [SKG][128][N]
// slices -- ws holds both halves' slices in SKG M N floats -- each finished by its own second pass.
template <int KB, bool WQ>
void m256_launch_sk4(int M, const R4AParts& ap, const unsigned* w, const float* svh, void* c, float* ws, int K, int N,
                     int SKG, int full, float out_scale, const float* wsc, int wq_gsh, hipStream_t st) {
  for (int h = 0; h < M / 128; ++h) {
    R4AParts aph = ap;
    for (int p = 0; p < 4; ++p) aph.a[p] = ap.a[p] + (size_t)h * 128 * K;
    void* ch = (char*)c + (size_t)h * 128 * N * (full ? 2 : 4);
    float* wsh = ws ? ws + (size_t)h * SKG * 128 * N : nullptr;
    m256_launch_rt<KB, 4, WQ, true>(aph, w, svh, ch, wsh, nullptr, 128, K, N, SKG, full, out_scale, wsc, wq_gsh, st);
    if (SKG > 1 || full) r4d::launch_split_finish(wsh, svh, ch, 128, N, SKG, full, out_scale, st);
  }
}

template <int KB>
void m256_launch(int M, const R4AParts& ap, const unsigned* w,
                 const float* svh, void* c, float* ws, unsigned* tickets, int K, int N, int SKG, int full,
                 float out_scale, const float* wsc, int wq_gsh, hipStream_t st, bool sk4) {
  if (sk4) {
    if (wsc) {
      if constexpr (KB == 4 || KB == 5) m256_launch_sk4<KB, true>(M, ap, w, svh, c, ws, K, N, SKG, full, out_scale, wsc, wq_gsh, st);
    } else {
      m256_launch_sk4<KB, false>(M, ap, w, svh, c, ws, K, N, SKG, full, out_scale, nullptr, 0, st);
    }
    return;
  }
  if (wsc) {
    if constexpr (KB == 4 || KB == 5) {
      if (M == 256) m256_launch_rt<KB, 8, true>(ap, w, svh, c, ws, tickets, M, K, N, SKG, full, out_scale, wsc, wq_gsh, st);
      else m256_launch_rt<KB, 4, true>(ap, w, svh, c, ws, tickets, M, K, N, SKG, full, out_scale, wsc, wq_gsh, st);
    }
    return;
  }
  if (M == 256) m256_launch_rt<KB, 8, false>(ap, w, svh, c, ws, tickets, M, K, N, SKG, full, out_scale, nullptr, 0, st);
  else m256_launch_rt<KB, 4, false>(ap, w, svh, c, ws, tickets, M, K, N, SKG, full, out_scale, nullptr, 0, st);
}

// sk_split: the caller asked for the M <= 64 kernel's 4-wave order (SK 4, 8, 16), which that kernel runs when SKG > 1
// or ws and tickets are given (else its one-wave form).
void m256_run_parts(const R4AParts& ap, int64_t w, int64_t svh, int64_t c, int64_t ws, int64_t tickets, int M,
                    int K, int N, int KB, int SKG, int full, float out_scale, int64_t stream, const char* entry,
                    int64_t wscale = 0, int wq_gsh = 0, bool sk_split = false) {
  r4d::require(entry, m256_check(M, K, N, ap.n_end[0] > N ? N : ap.n_end[0], KB, SKG));
  if (!ap.a[0] || !w || !c) r4d::fail(entry, "null A, W or C");
  if (full && !svh) r4d::fail(entry, "svh must be non-null");
  if (SKG > 1 && !ws) r4d::fail(entry, "SKG > 1 needs ws");
  const bool sk4 = sk_split && (SKG > 1 || (ws && tickets));
  auto Wp = (const unsigned*)w;
  auto S = (const float*)svh;
  auto WS = (float*)ws;
  auto T = (unsigned*)tickets;
  hipStream_t st = (hipStream_t)stream;
  auto WSC = (const float*)wscale;
  if (KB == 4) m256_launch<4>(M, ap, Wp, S, (void*)c, WS, T, K, N, SKG, full, out_scale, WSC, wq_gsh, st, sk4);
  else if (KB == 5) m256_launch<5>(M, ap, Wp, S, (void*)c, WS, T, K, N, SKG, full, out_scale, WSC, wq_gsh, st, sk4);
  else m256_launch<3>(M, ap, Wp, S, (void*)c, WS, T, K, N, SKG, full, out_scale, WSC, wq_gsh, st, sk4);
  if (SKG > 1 && !sk4) r4d::launch_split_finish(WS, S, (void*)c, M, N, SKG, full, out_scale, st);
  r4d::launch_ok(entry);
}

void m256_run(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t svh, int64_t c, int64_t ws,
              int64_t tickets, int M, int K, int N, int KB, int SKG, int full, float out_scale, int64_t stream,
              const char* entry, int64_t wscale = 0, int wq_gsh = 0, bool sk_split = false) {
  r4d::require(entry, m256_check(M, K, N, n_split, KB, SKG));
  m256_run_parts(r4_parts((const void*)a0, (const void*)a1, n_split), w, svh, c, ws, tickets, M, K, N, KB, SKG, full,
                 out_scale, stream, entry, wscale, wq_gsh, sk_split);
}

}  // namespace

void r4d::launch_split_finish(const float* ws, const float* svh, void* c, int M, int N, int SKG, int full,
                              float out_scale, hipStream_t st) {
  hipLaunchKernelGGL(tq_m256_finish, dim3(N / 128, M / kFinRows), dim3(256), 0, st, ws, svh, c, M, N, SKG, full, out_scale);
}

// SK names the M <= 64 row this launch reproduces: 1 or 2 (0 means 1) is r4d_gemm_trellis_nt_m64's one-wave-per-pair
// order; 4, 8 and 16 its 4-wave split order (which that kernel runs when SKG > 1 or ws and tickets are given, else its
// one-wave form -- and so does this one).
static bool m256_sk_ok(int SK) { return SK == 0 || SK == 1 || SK == 2 || SK == 4 || SK == 8 || SK == 16; }
static bool m256_sk_split(int SK) { return SK == 4 || SK == 8 || SK == 16; }
static const char* const sk_msg =
    "SK must be 1, 2, 4, 8 or 16 (0 means 1): 1 and 2 reproduce r4d_gemm_trellis_nt_m64's one-wave-per-pair order, "
    "4, 8 and 16 its 4-wave split order";

extern "C" {

// r4d.h:416-419. Every element equals, bit for bit, what r4d_gemm_trellis_nt_m64 gives it at M = 64 with
// SK = 1 (or 2: the same order) and the same SKG (the same MFMA operands in the same order per K slice, the same
// slice order and epilogue). SK must be 0, 1 or 2 (0 means 1); NP, U and skw are the reference's geometry knobs:
// accepted, unused.
void r4d_gemm_trellis_nt_m256(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t svh, int64_t c,
                              int64_t ws, int64_t tickets, int M, int K, int N, int KB, int SK, int NP,
                              int SKG, int U, float out_scale, int64_t stream, int skw) {
  (void)NP; (void)U; (void)skw;
  if (!m256_sk_ok(SK)) r4d::fail("gemm_trellis_nt_m256", sk_msg);
  m256_run(a0, a1, n_split, w, svh, c, ws, tickets, M, K, N, KB, SKG, 1, out_scale, stream,
           "gemm_trellis_nt_m256", 0, 0, m256_sk_split(SK));
}

const char* r4d_gemm_trellis_nt_m256_check(int M, int K, int N, int n_split, int KB, int SK, int NP, int SKG,
                                           int U, int skw) {
  (void)NP; (void)U; (void)skw;
  if (!m256_sk_ok(SK)) return r4d::check_result(sk_msg);
  return r4d::check_result(m256_check(M, K, N, n_split, KB, SKG));
}

// SKG fp32 slices [SKG][M][N], and after them (SKG > 1) room for the balanced form's published accumulators: M x 128
// fp32 per workgroup, at most one workgroup per compute unit (at SKG = 1 they fit in the M x N floats).
size_t r4d_gemm_trellis_nt_m256_ws_bytes(int M, int N, int SKG) {
  if (M <= 0 || N <= 0 || SKG <= 0) return 0;
  const size_t slices = (size_t)SKG * (size_t)M * (size_t)N * sizeof(float);
  if (SKG == 1) return slices;
  const size_t units = (size_t)(N / 128) * (size_t)SKG, cus = (size_t)m256_cus();
  return slices + (units < cus ? units : cus) * (size_t)M * 128 * sizeof(float);
}

// No reference counterpart: r4d_gemm_trellis_nt_m256 over up to four input parts (the prefill form of
// r4dx_gemm_trellis_nt_m64_parts): columns [n0[p], n0[p + 1]) read a[p]. Every column equals the one-part launch
// of its range at the same SKG.
const char* r4dx_gemm_trellis_nt_m256_parts_check(int parts, const int* n0, int M, int K, int N, int KB, int SKG) {
  std::string e = r4d::parts_rule(parts, n0, N);
  if (e.empty()) e = m256_check(M, K, N, parts > 1 ? n0[1] : N, KB, SKG);
  return r4d::check_result(e);
}
void r4dx_gemm_trellis_nt_m256_parts(const int64_t* a, const int* n0, int parts, int64_t w, int64_t svh, int64_t c,
                                     int64_t ws, int64_t tickets, int M, int K, int N, int KB, int SKG,
                                     float out_scale, int64_t stream) {
  const char* e = "gemm_trellis_nt_m256_parts";
  if (!a || !n0) r4d::fail(e, "null part arrays");
  if (const char* m = r4dx_gemm_trellis_nt_m256_parts_check(parts, n0, M, K, N, KB, SKG)) r4d::fail(e, m);
  for (int p = 0; p < parts; ++p)
    if (!a[p]) r4d::fail(e, "null part input");
  const R4AParts ap = r4_parts((const void*)a[0], parts > 1 ? (const void*)a[1] : nullptr, parts > 1 ? n0[1] : N,
                               parts > 2 ? (const void*)a[2] : nullptr, parts > 2 ? n0[2] : 0,
                               parts > 3 ? (const void*)a[3] : nullptr, parts > 3 ? n0[3] : 0);
  m256_run_parts(ap, w, svh, c, ws, tickets, M, K, N, KB, SKG, 1, out_scale, stream, e);
}

void r4d_gemm_trellis_nt_m256_raw(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t c, int64_t ws,
                                  int64_t tickets, int M, int K, int N, int KB, int SKG, int64_t stream) {
  m256_run(a0, a1, n_split, w, 0, c, ws, tickets, M, K, N, KB, SKG, 0, 1.f, stream, "gemm_trellis_nt_m256_raw");
}

// r4d.h:451-454: r4d_gemm_trellis_nt_m256 with the weight fake-quant of the _wq entries (the scale table of
// r4d_trellis_wscale_f32, 2^gsh k-tiles per group; a null table throws). Bit-identical, per element, to
// r4d_gemm_trellis_nt_m64_wq at M = 64, SK = 1 (or 2) and the same SKG.
void r4d_gemm_trellis_nt_m256_wq(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t svh, int64_t c,
                                 int64_t ws, int64_t tickets, int M, int K, int N, int KB, int SK, int NP,
                                 int SKG, int U, float out_scale, int64_t stream, int skw, int64_t wscale,
                                 int gsh) {
  (void)NP; (void)U; (void)skw;
  const char* e = "gemm_trellis_nt_m256_wq";
  if (!m256_sk_ok(SK)) r4d::fail(e, sk_msg);
  if (!wscale) r4d::fail(e, "the _wq entry needs a scale table (r4d_trellis_wscale_f32)");
  if (gsh < 1 || gsh > 3 || K % (16 << gsh)) r4d::fail(e, "gsh must be 1, 2 or 3 with 16 << gsh dividing K");
  if (KB != 4 && KB != 5) r4d::fail(e, "KB must be 4 or 5");
  m256_run(a0, a1, n_split, w, svh, c, ws, tickets, M, K, N, KB, SKG, 1, out_scale, stream, e, wscale, gsh,
           m256_sk_split(SK));
}

// This build's K split for the prefill GEMM: the steps per CU decide the critical path (one workgroup resident per
// CU: the two LDS stages take 96 KiB; the balanced form evens out unit counts that are not a multiple of the CUs), so
// SKG minimises those steps plus the cost of the second pass (SKG x M x N fp32 written and read back). SKG is a power of two
// up to 8: the engine's tuning rows hold no other (TrellisRowFits, src/model/linear.cpp:243-255), and the M = 64
// band's row carries this SKG (PlanTrellisM256 reads it there, linear.cpp:696-701).
int r4d_mi355x_trellis_m256_skg(int K, int N, int KB) {
  (void)KB;
  const int KT = K / 16, G = N / 128;
  if (KT <= 0 || G <= 0) return 1;
  const int cus = m256_cus();
  int best = 1;
  double best_cost = 1e30;
  for (int d = 1; d <= 8; d *= 2) {
    if (KT % (4 * d)) continue;
    const long long units = (long long)G * d;
    const int steps = KT / (4 * d);
    // steps on the critical path: one unit per compute unit at most, else the balanced form's share (a whole number
    // of rounds when the units are a multiple of the compute units)
    const bool balanced = units > cus && units % cus != 0;
    const double path = balanced ? (double)((units * steps + cus - 1) / cus) : (double)((units + cus - 1) / cus) * steps;
    // fitted to SKG sweeps of the layer's M = 256 launch shapes (TP 1 and 2; one workgroup per CU; weights streamed
    // from HBM, > 1 GB of copies): a step ~1.05 us in the data-parallel form and ~1.4 us per step of a share in the
    // balanced form (all CUs busy; 1.4 reproduces every sweep's best SKG, e.g. 17408 x 5120: SKG 4 82.1 us, SKG 8
    // balanced 80.5 us; 6144 x 5120: 37.6 / 44.0 us; 8704 x 5120: 47.3 / 53.3 us; 5120 x 34816: SKG 1 balanced
    // 132 us, SKG 2 145 us); a split costs ~2 us (the finish launch) plus ~0.06 us per workgroup-slice (its partials
    // written and read back)
    const double cost = path * (balanced ? 1.4 : 1.05) + (d > 1 ? 2.0 + 0.06 * G * d : 0.0);
    if (cost < best_cost) {
      best_cost = cost;
      best = d;
    }
  }
  return best;
}

}  // extern "C"
