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
// coalesced dwordx4 per lane per 64-k block (lane l: tile 2p + ((l & 31) >> 4), lh = l >> 5, r = l & 15),
// w4_pf blocks in flight in a statically indexed ring; the loads are nontemporal (each weight byte is
// read once).
//
// Dequant per dword (8 nibbles, nibble i at k = 16 s + 4 lh + {0, 8, 1, 9, 2, 10, 3, 11}[i]): masks
// 0x000F000F and 0x00F000F0 of the dword and of the dword >> 8 pick the nibble pairs (0, 4), (1, 5),
// (2, 6), (3, 7); one and-xor each gives the f16 bits of 1024 + q (the ^ 8 folded into the xor constant)
// for a low nibble and of 1024 + 16 q for a high one; one packed f16 add of -(1024 + z), resp.
// -(1024 + 16 z), gives q - z, resp. 16 (q - z), exactly. Pairs (0, 4), (2, 6) are k +0, +2, +1, +3
// ("U", unscaled) and (1, 5), (3, 7) are k +8, +10, +9, +11 ("S", scaled by 16). A 64-k block is four
// MFMAs of eight elements per lane: U of dwords (0, 1), U of (2, 3), S of (0, 1), S of (2, 3) -- each
// inside one group of 32. The two chains are combined as (U + S / 16) * scale: the 1 / 16 undoes the
// factor 16 exactly (a power of two). The A fragment of an MFMA is two runs of four k in that order,
// staged in LDS with one row of zeros per (block, MFMA, k-half) for the lanes whose row is absent.
//
// Two MFMA forms. M <= 8: v_mfma_f32_16x16x32_f16 with rows (2 m + tile): lane (n, kq) holds the B data
// of tile kq & 1, k-half kq >> 1, and A row rho is nonzero only where rho & 1 == kq & 1, so output row
// 2 m + t is row m of tile t -- one 16x16x32 covers both tiles at half the MFMA cycles of a 32x32x16.
// M > 8: v_mfma_f32_32x32x16_f16 (lane = column l & 31, k-half l >> 5), MT row tiles of 32.
//
// A is staged per chunk of KC 64-k blocks (all of K when it fits the LDS budget); a chunk change is a
// block barrier. N = 248 320 gives 7 760 waves of work, so no split of K is needed.
#include "r4d_dev.h"
#include "r4d_host.h"
#include "r4d_mi355x.h"

#include <map>
#include <mutex>

namespace {

typedef __amdgpu_buffer_rsrc_t r4_rsrc;
__device__ __forceinline__ r4_rsrc mk_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)bytes, 0x00020000);
}

constexpr int kWaves = 8;          // 8 waves = 256 output columns per workgroup
// weight steps in flight per wave: 6 in the 16x16x32 form at G = 64 (measured faster there), else 4
__host__ __device__ constexpr int w4_pf(int G, bool small) { return G == 64 && small ? 6 : 4; }
constexpr int kNT = 2;             // cache policy of the weight loads: nontemporal (read once, streamed)
constexpr int kLdsBudget = 40 * 1024;   // A chunk bytes per workgroup (four workgroups per CU)

// 64-k blocks per A chunk for M rows (M + 1 staged): a multiple of pf, at most KB64 rounded up to one.
__host__ __device__ inline int w4_chunk(int M, int KB64, int pf) {
  int kc = kLdsBudget / (128 * (M + 1));
  kc -= kc % pf;
  const int all = (KB64 + pf - 1) / pf * pf;
  return kc < all ? kc : all;
}

// B operand of MFMA c (0: U of dwords 0,1; 1: U of 2,3; 2: S of 0,1; 3: S of 2,3) from the dequantized
// halves: u[s] = (k +0,+2 ; +1,+3), v[s] = (k +8,+10 ; +9,+11).
struct W4B {
  r4u2 u[4], v[4];
};
__device__ __forceinline__ void w4_dequant(const r4u4 w, const unsigned (&nz)[4], const unsigned (&nz16)[4], W4B& o) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const unsigned x = w[s], y = x >> 8;
    const unsigned p0 = (x & 0x000F000Fu) ^ 0x64086408u, p1 = (x & 0x00F000F0u) ^ 0x64806480u;
    const unsigned p2 = (y & 0x000F000Fu) ^ 0x64086408u, p3 = (y & 0x00F000F0u) ^ 0x64806480u;
    const r4h2 z = __builtin_bit_cast(r4h2, nz[s]), z16 = __builtin_bit_cast(r4h2, nz16[s]);
    o.u[s][0] = __builtin_bit_cast(unsigned, __builtin_bit_cast(r4h2, p0) + z);
    o.u[s][1] = __builtin_bit_cast(unsigned, __builtin_bit_cast(r4h2, p2) + z);
    o.v[s][0] = __builtin_bit_cast(unsigned, __builtin_bit_cast(r4h2, p1) + z16);
    o.v[s][1] = __builtin_bit_cast(unsigned, __builtin_bit_cast(r4h2, p3) + z16);
  }
}
__device__ __forceinline__ r4h8 w4_bop(const W4B& b, int c) {
  const r4u2 lo = c == 0 ? b.u[0] : c == 1 ? b.u[2] : c == 2 ? b.v[0] : b.v[2];
  const r4u2 hi = c == 0 ? b.u[1] : c == 1 ? b.u[3] : c == 2 ? b.v[1] : b.v[3];
  return __builtin_bit_cast(r4h8, (r4u4){lo[0], lo[1], hi[0], hi[1]});
}
// k offset (in the 64-k block, before 4 lh) of the first run of MFMA c's A fragment; the second run is +16
__host__ __device__ constexpr int w4_run_k(int c) { return c == 0 ? 0 : c == 1 ? 32 : c == 2 ? 8 : 40; }

// (f16 -(1024 + z), f16 -(1024 + 16 z)) pairs of one Wsz word: -(1024 + 16 z) = 16 (-(1024 + z)) + 15360,
// exact in f16 (integers below 2048)
__device__ __forceinline__ void w4_zeros(unsigned szw, unsigned& nz, unsigned& nz16) {
  nz = __builtin_amdgcn_perm(szw, szw, 0x03020302u);
  nz16 = __builtin_bit_cast(unsigned, __builtin_elementwise_fma(__builtin_bit_cast(r4h2, nz),
                                                                (r4h2){(_Float16)16.0f, (_Float16)16.0f},
                                                                (r4h2){(_Float16)15360.0f, (_Float16)15360.0f}));
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

// The fused argmax of the logits entry: each workgroup reduces its columns to one key per row, folds it
// into slot (workgroup mod kAmSlots) of the row with an atomic max, and takes the launch's ticket; the last
// workgroup reduces the slots, writes (index, value) per row and clears the slots it read.
constexpr int kAmSlots = 64;
struct AmFused {
  unsigned long long* slots;   // [kAmSlots][64 rows] u64, zero between launches
  unsigned* ticket;            // one ticket line
  int* out_idx;
  float* out_val;              // may be null
};

// Epilogue of the fused argmax: the logits are stored coherently (agent scope, so the last workgroup reads
// the winner's own bits whichever XCD wrote them); a wave reduces its lanes' keys per row across the lanes
// that share the row, the workgroup across its waves in LDS, and one thread per row folds that into the
// row's slot. Dead waves (no tile) and columns >= N contribute nothing.
// The per-wave keys and the ticket flag reuse the A chunk's LDS (w4_am_lds bytes of it): a static array would
// take the M = 8 workgroup past 40 KiB and the CU from four workgroups to three.
template <bool SMALL>
constexpr int w4_am_rows() { return SMALL ? 8 : 64; }
__host__ __device__ constexpr size_t w4_am_lds(bool small) { return (size_t)kWaves * (small ? 8 : 64) * 8 + 16; }

template <bool SMALL, int MT, typename Acc>
__device__ __forceinline__ void w4_store_argmax(const Acc (&acc)[SMALL ? 1 : MT], float* __restrict__ C, int M,
                                                int N, int t0, bool live, const AmFused& af, void* lds) {
  constexpr int RS = w4_am_rows<SMALL>();
  auto red = reinterpret_cast<unsigned long long (*)[RS]>(lds);
  int* flag = reinterpret_cast<int*>(red + kWaves);
  __syncthreads();   // every wave is past its last read of the A chunk
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, lh = lane >> 5;
  if constexpr (SMALL) {
    // lane: column 16 (t0 + (e & 1)) + (lane & 15), row 2 (lane >> 4) + (e >> 1)
    unsigned long long k[2] = {0ull, 0ull};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 2 * (lane >> 4) + (e >> 1), n = 16 * (t0 + (e & 1)) + (lane & 15);
      if (live && m < M && n < N) {
        __hip_atomic_store(&C[(size_t)m * N + n], acc[0][e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        k[e >> 1] = am_max(k[e >> 1], am_key(acc[0][e], (unsigned)n));
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const unsigned lo = __shfl_xor((unsigned)k[j], o, 64), hi = __shfl_xor((unsigned)(k[j] >> 32), o, 64);
        k[j] = am_max(k[j], ((unsigned long long)hi << 32) | lo);
      }
      if ((lane & 15) == 0) red[w][2 * (lane >> 4) + j] = k[j];
    }
  } else {
    // lane: column 16 t0 + (lane & 31), row i 32 + (e / 4) 8 + lh 4 + e % 4
    const int n = 16 * t0 + (lane & 31);
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = i * 32 + (e >> 2) * 8 + lh * 4 + (e & 3);
        unsigned long long k = 0ull;
        if (live && m < M && n < N) {
          __hip_atomic_store(&C[(size_t)m * N + n], acc[i][e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          k = am_key(acc[i][e], (unsigned)n);
        }
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) {
          const unsigned lo = __shfl_xor((unsigned)k, o, 64), hi = __shfl_xor((unsigned)(k >> 32), o, 64);
          k = am_max(k, ((unsigned long long)hi << 32) | lo);
        }
        if ((lane & 31) == 0) red[w][m] = k;
      }
  }
  __syncthreads();
  if ((int)threadIdx.x < M) {
    unsigned long long k = 0ull;
#pragma unroll
    for (int v = 0; v < kWaves; ++v) k = am_max(k, red[v][threadIdx.x]);
    __hip_atomic_fetch_max(&af.slots[(blockIdx.x % kAmSlots) * 64 + threadIdx.x], k, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!r4_ticket_last(af.ticket, gridDim.x, flag)) return;
  // the last workgroup: thread t reads slot t / 8 of rows 8 j + t % 8 (all loads issued before any use),
  // clears them, and the slots reduce across lanes (8 per wave) and waves
  unsigned long long k[8];
  const int sl = threadIdx.x >> 3, r8 = threadIdx.x & 7;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    k[j] = 8 * j + r8 < M ? __hip_atomic_load(&af.slots[sl * 64 + 8 * j + r8], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                          : 0ull;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (8 * j + r8 < M) __hip_atomic_store(&af.slots[sl * 64 + 8 * j + r8], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();   // every wave is past its reads of red
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (8 * j >= M) break;
#pragma unroll
    for (int o = 8; o < 64; o <<= 1) {
      const unsigned lo = __shfl_xor((unsigned)k[j], o, 64), hi = __shfl_xor((unsigned)(k[j] >> 32), o, 64);
      k[j] = am_max(k[j], ((unsigned long long)hi << 32) | lo);
    }
    if (lane < 8) red[w][8 * j + lane] = k[j];
  }
  __syncthreads();
  if ((int)threadIdx.x < M) {
    const int row = threadIdx.x;
    unsigned long long kr = 0ull;
#pragma unroll
    for (int v = 0; v < kWaves; ++v) kr = am_max(kr, red[v][row]);
    int idx;
    float val;
    am_decode(kr, &idx, &val);
    af.out_idx[row] = idx;
    // the key holds the winner's bits except the sign of a zero: read a zero winner's own bits back
    if (af.out_val)
      af.out_val[row] = kr >= am_key(-__builtin_inff(), 0u) && val == 0.0f
                            ? __hip_atomic_load(&C[(size_t)row * N + idx], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                            : val;
  }
}

// SMALL: the 16x16x32 form (M <= 8). MT: row tiles of 32 in the 32x32x16 form.
// AM (with OUTF): the fused per-row argmax of the logits (AmFused).
template <int G, bool SMALL, int MT, bool OUTF, bool AM>
__global__ __launch_bounds__(64 * kWaves) void w4_kernel(const unsigned short* __restrict__ A,
                                                          const unsigned* __restrict__ Wq,
                                                          const unsigned* __restrict__ Wsz,
                                                          void* __restrict__ Cv, int M, int K, int N, AmFused af) {
  static_assert(!AM || OUTF, "the fused argmax reads fp32 logits");
  extern __shared__ r4u4 alds[];   // chunk fragments [kb][c][lh][M] of 8 halves, then a zero block
  const int lane = threadIdx.x & 63;
  const int KB64 = K >> 6, groups = K / G;
  const int tiles = N >> 4;
  constexpr int kPF = w4_pf(G, SMALL);
  const int KC = w4_chunk(M, KB64, kPF);
  const int M1 = M + 1;                        // staged rows: row M is zero
  int t0 = (blockIdx.x * kWaves + (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * 2;
  const bool live = t0 < tiles;
  if (!live) t0 = tiles - 1;                   // a spare wave streams the last tile and stores nothing
  const int tl = t0 + ((lane & 31) >> 4), lh = lane >> 5, r = lane & 15;

  const r4_rsrc wr = mk_rsrc(Wq, (unsigned)((size_t)N * K / 2));
  const unsigned wlane = (unsigned)((((size_t)tl * KB64) * 2 + lh) * 16 + r) * 16u;
  const r4_rsrc sr = mk_rsrc(Wsz, (unsigned)((size_t)N * groups * 4));
  // the lane's own tile (its zero point) and, in the SMALL form, both tiles' scales at column r
  const unsigned sown = (unsigned)(((size_t)tl * groups * 16) + r) * 4u;
  const unsigned st0 = (unsigned)(((size_t)t0 * groups * 16) + r) * 4u;
  const unsigned st1 = (unsigned)(((size_t)(t0 + 1) * groups * 16) + r) * 4u;
  constexpr int NG = 64 / G;                  // groups per 64-k block
  constexpr int NS = SMALL ? 2 : 1;           // scale words per group
  const bool own1 = ((lane >> 4) & 1) != 0;   // SMALL: the lane's own tile is t0 + 1

  // A fragment byte offsets in the chunk (without the kb, c term) per row tile
  constexpr int NA = SMALL ? 1 : MT;
  unsigned a_lane[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    int m, h;
    bool ok;
    if constexpr (SMALL) {
      const int rho = lane & 15, kq = lane >> 4;
      m = rho >> 1; h = kq >> 1; ok = (rho & 1) == (kq & 1) && m < M;
    } else {
      m = i * 32 + (lane & 31); h = lh; ok = m < M;
    }
    a_lane[i] = (unsigned)((h * M1 + (ok ? m : M)) * 16);
  }
  const unsigned kb_stride = 8u * (unsigned)M1 * 16u;   // bytes per 64-k block in the chunk
  auto afrag = [&](int i, int kbl, int c) -> r4h8 {
    const unsigned off = (unsigned)kbl * kb_stride + (unsigned)c * 2u * M1 * 16u + a_lane[i];
    return __builtin_bit_cast(r4h8, *(const r4u4*)((const char*)alds + off));
  };
  // stage 64-k blocks [kb0, kb0 + KC) of A: fragment ((kbl * 4 + c) * 2 + h) * M1 + m holds
  // A[m][64 kb + run_k(c) + 4 h + {0, 2, 1, 3, 16, 18, 17, 19}] (row M: zeros)
  auto stage = [&](int kb0) {
    const int n = min(KC, KB64 - kb0) * 8 * M1;
    for (int i = threadIdx.x; i < n; i += 64 * kWaves) {
      const int m = i % M1, rest = i / M1, h = rest & 1, c = (rest >> 1) & 3, kbl = rest >> 3;
      r4u4 v = {0u, 0u, 0u, 0u};
      if (m < M) {
        const unsigned short* src = A + (size_t)m * K + 64 * (kb0 + kbl) + w4_run_k(c) + 4 * h;
        const r4u2 lo = *(const r4u2*)src, hi = *(const r4u2*)(src + 16);
        v[0] = __builtin_amdgcn_perm(lo[1], lo[0], 0x05040100u);
        v[1] = __builtin_amdgcn_perm(lo[1], lo[0], 0x07060302u);
        v[2] = __builtin_amdgcn_perm(hi[1], hi[0], 0x05040100u);
        v[3] = __builtin_amdgcn_perm(hi[1], hi[0], 0x07060302u);
      }
      alds[i] = v;
    }
  };

  using Acc = typename std::conditional<SMALL, r4f4, r4f16>::type;
  Acc acc[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) acc[i] = Acc{};

  // COOP (the 16x16x32 form at G = 32): the wave's 64 scale words of a block -- (tile t0 + (lane >> 5), group
  // (lane >> 4) & 1, column lane & 15) -- one load per lane instead of four, each handed to the lanes that use it at
  // compute time (ds_bpermute). Measured: g32 M = 1 / 8 146 -> 144 / 155 -> 151 us; at G = 64 (two loads replaced)
  // 5 % slower, so G = 64 keeps its own loads.
  constexpr bool COOP = SMALL && G == 32;
  const unsigned coop_base = (unsigned)((((size_t)(t0 + (lane >> 5)) * groups + (NG == 2 ? (lane >> 4) & 1 : 0)) * 16 +
                                         (lane & 15)) * 4u);
  struct St {
    r4u4 w;
    unsigned sz[COOP ? 1 : NG * NS];
  };
  auto load = [&](St& s, int kb) {
    const int kc = kb < KB64 ? kb : KB64 - 1;
    s.w = __builtin_bit_cast(r4u4, __builtin_amdgcn_raw_buffer_load_b128(wr, wlane + (unsigned)kc * 512u, 0, kNT));
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const unsigned go = (unsigned)(NG * kc + g) * 64u;
      if constexpr (COOP) {
        if (g == 0) s.sz[0] = __builtin_amdgcn_raw_buffer_load_b32(sr, coop_base + (unsigned)(NG * kc) * 64u, 0, kNT);
      } else if constexpr (SMALL) {
        s.sz[2 * g] = __builtin_amdgcn_raw_buffer_load_b32(sr, st0 + go, 0, kNT);
        s.sz[2 * g + 1] = __builtin_amdgcn_raw_buffer_load_b32(sr, st1 + go, 0, kNT);
      } else {
        s.sz[g] = __builtin_amdgcn_raw_buffer_load_b32(sr, sown + go, 0, kNT);
      }
    }
  };
  auto compute = [&](const St& s0, int kbl) {
    // the block's scale words of the lane's column: word 2 g + t for group g, tile t0 + t (COOP: from the lanes that
    // loaded them)
    unsigned szl[NG * NS];
    if constexpr (COOP) {
#pragma unroll
      for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int t = 0; t < 2; ++t)
          szl[2 * g + t] = (unsigned)__builtin_amdgcn_ds_bpermute(((t << 5) | (g << 4) | (lane & 15)) << 2, (int)s0.sz[0]);
    }
    struct SzView {
      const unsigned* p;
      __device__ unsigned operator[](int i) const { return p[i]; }
    };
    const struct { SzView sz; } s{SzView{COOP ? szl : s0.sz}};
    unsigned nz[4], nz16[4];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const unsigned own = SMALL ? (own1 ? s.sz[2 * g + 1] : s.sz[2 * g]) : s.sz[g];
      unsigned a, b;
      w4_zeros(own, a, b);
#pragma unroll
      for (int q = 0; q < 4 / NG; ++q) { nz[g * (4 / NG) + q] = a; nz16[g * (4 / NG) + q] = b; }
    }
    W4B bq;
    w4_dequant(s0.w, nz, nz16, bq);
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      // group g: G = 64 -> U chain (c 0, 1), S chain (c 2, 3); G = 32 -> g 0: c 0 / 2, g 1: c 1 / 3
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        Acc tu, ts;
        if constexpr (SMALL) {
          tu = __builtin_amdgcn_mfma_f32_16x16x32_f16(afrag(i, kbl, G == 64 ? 0 : g), w4_bop(bq, G == 64 ? 0 : g), Acc{}, 0, 0, 0);
          ts = __builtin_amdgcn_mfma_f32_16x16x32_f16(afrag(i, kbl, G == 64 ? 2 : 2 + g), w4_bop(bq, G == 64 ? 2 : 2 + g), Acc{}, 0, 0, 0);
          if constexpr (G == 64) {
            tu = __builtin_amdgcn_mfma_f32_16x16x32_f16(afrag(i, kbl, 1), w4_bop(bq, 1), tu, 0, 0, 0);
            ts = __builtin_amdgcn_mfma_f32_16x16x32_f16(afrag(i, kbl, 3), w4_bop(bq, 3), ts, 0, 0, 0);
          }
          // output rows 4 (lane >> 4) + e = 2 m + t: tile t = e & 1 (rows m >= M have zero A and stay 0)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float sc = r4_f16_to_f32((unsigned short)(s.sz[2 * g + (e & 1)] & 0xFFFFu));
            acc[i][e] = __builtin_fmaf(__builtin_fmaf(ts[e], 0.0625f, tu[e]), sc, acc[i][e]);
          }
        } else {
          tu = __builtin_amdgcn_mfma_f32_32x32x16_f16(afrag(i, kbl, G == 64 ? 0 : g), w4_bop(bq, G == 64 ? 0 : g), Acc{}, 0, 0, 0);
          ts = __builtin_amdgcn_mfma_f32_32x32x16_f16(afrag(i, kbl, G == 64 ? 2 : 2 + g), w4_bop(bq, G == 64 ? 2 : 2 + g), Acc{}, 0, 0, 0);
          if constexpr (G == 64) {
            tu = __builtin_amdgcn_mfma_f32_32x32x16_f16(afrag(i, kbl, 1), w4_bop(bq, 1), tu, 0, 0, 0);
            ts = __builtin_amdgcn_mfma_f32_32x32x16_f16(afrag(i, kbl, 3), w4_bop(bq, 3), ts, 0, 0, 0);
          }
          const float sc = r4_f16_to_f32((unsigned short)(s.sz[g] & 0xFFFFu));
          // only the rows this launch has: row = (e / 4) * 8 + lh * 4 + e % 4
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (i * 32 + (e >> 2) * 8 < M) acc[i][e] = __builtin_fmaf(__builtin_fmaf(ts[e], 0.0625f, tu[e]), sc, acc[i][e]);
        }
      }
    }
  };

  // The ring is indexed statically (the loop unrolled by kPF): a register copy of a slot whose load is
  // still in flight would wait for it and leave one load in flight. Chunk boundaries fall on multiples
  // of kPF (KC is one).
  St ring[kPF];
#pragma unroll
  for (int i = 0; i < kPF; ++i) load(ring[i], i);
  const int full = KB64 - KB64 % kPF;
  int kb_chunk = 0;
  stage(0);
  __syncthreads();
  for (int kb = 0; kb < full; kb += kPF) {
    if (kb - kb_chunk == KC) {
      __syncthreads();
      kb_chunk = kb;
      stage(kb);
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < kPF; ++i) {
      compute(ring[i], kb - kb_chunk + i);
      load(ring[i], kb + i + kPF);
    }
  }
  if (full < KB64) {
    if (full - kb_chunk == KC) {
      __syncthreads();
      kb_chunk = full;
      stage(full);
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < kPF; ++i)
      if (full + i < KB64) compute(ring[i], full - kb_chunk + i);
  }
  if constexpr (AM) {
    w4_store_argmax<SMALL, MT>(acc, (float*)Cv, M, N, t0, live, af, (void*)alds);
    return;
  }
  if (!live) return;

  if constexpr (SMALL) {
    // lane: column 16 t + (lane & 15), rows 4 (lane >> 4) + e = 2 m + t
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 2 * (lane >> 4) + (e >> 1), n = 16 * (t0 + (e & 1)) + (lane & 15);
      if (m < M && n < N) {
        if constexpr (OUTF) ((float*)Cv)[(size_t)m * N + n] = acc[0][e];
        else ((unsigned short*)Cv)[(size_t)m * N + n] = r4_bf16_rn(acc[0][e]);
      }
    }
  } else {
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
}

std::string w4_check(int group, int M, int K, int N) {
  if (group != 32 && group != 64) return "group " + r4d::str(group) + " is not instantiated (32, 64)";
  if (M < 1 || M > 64) return "M must be 1..64";
  if (N <= 0 || N % 16) return "N must be a positive multiple of 16";
  if (K <= 0 || K % 64) return "K must be a positive multiple of 64 (the packed 64-k block)";
  if ((size_t)N * K / 2 >= (1ull << 32) || (size_t)N * (K / group) * 4 >= (1ull << 32))
    return "N x K too large for 32-bit buffer offsets (4 GiB of packed weights)";
  return "";
}

template <int G, bool OUTF, bool AM>
void w4_launch(int64_t a, int64_t wq, int64_t wsz, int64_t c, int M, int K, int N, hipStream_t st, const AmFused& af) {
  const int tiles = N / 16;
  const int waves = (tiles + 1) / 2;
  dim3 grid((waves + kWaves - 1) / kWaves), block(64 * kWaves);
  size_t smem = (size_t)w4_chunk(M, K / 64, w4_pf(G, M <= 8)) * 8 * (M + 1) * 16;
  if (AM && smem < w4_am_lds(M <= 8)) smem = w4_am_lds(M <= 8);
  auto Ap = (const unsigned short*)a;
  auto Wp = (const unsigned*)wq;
  auto Sp = (const unsigned*)wsz;
  if (M <= 8) hipLaunchKernelGGL((w4_kernel<G, true, 1, OUTF, AM>), grid, block, smem, st, Ap, Wp, Sp, (void*)c, M, K, N, af);
  else if (M <= 32) hipLaunchKernelGGL((w4_kernel<G, false, 1, OUTF, AM>), grid, block, smem, st, Ap, Wp, Sp, (void*)c, M, K, N, af);
  else hipLaunchKernelGGL((w4_kernel<G, false, 2, OUTF, AM>), grid, block, smem, st, Ap, Wp, Sp, (void*)c, M, K, N, af);
}

void w4_run(int group, int64_t a, int64_t wq, int64_t wsz, int64_t c, int M, int K, int N, bool outf,
            int64_t stream, const char* entry) {
  r4d::require(entry, w4_check(group, M, K, N));
  if (!a || !wq || !wsz || !c) r4d::fail(entry, "null buffer");
  hipStream_t st = (hipStream_t)stream;
  const AmFused none{nullptr, nullptr, nullptr, nullptr};
  if (group == 32) {
    if (outf) w4_launch<32, true, false>(a, wq, wsz, c, M, K, N, st, none);
    else w4_launch<32, false, false>(a, wq, wsz, c, M, K, N, st, none);
  } else {
    if (outf) w4_launch<64, true, false>(a, wq, wsz, c, M, K, N, st, none);
    else w4_launch<64, false, false>(a, wq, wsz, c, M, K, N, st, none);
  }
  r4d::launch_ok(entry);
}

constexpr int kAmParts = 256;         // most workgroups per row (partial keys per row)
constexpr int kAmMaxRows = 64;
constexpr int kAmPerThread = 8;       // elements per thread and batch: all 8 loads issued before any compare
constexpr int kAmThreads = 256;

// Partial keys of one argmax: [kAmMaxRows][kAmParts] u64, then a ticket line (R4_TICKET_WORDS u32) per row. Each
// row's workgroups store their keys, take the row's ticket, and the last one reduces the row and resets the ticket.
// The fused argmax of the logits entry has a region of its own after these: kAmSlots x kAmMaxRows u64 slots and one
// ticket line (AmFused).
struct AmScratch {
  unsigned long long* keys;
  unsigned* tickets;
  unsigned long long* fused_slots;
  unsigned* fused_ticket;
};
constexpr size_t kAmScratchBytes =
    (size_t)kAmMaxRows * kAmParts * sizeof(unsigned long long) + (size_t)kAmMaxRows * R4_TICKET_WORDS * sizeof(unsigned) +
    (size_t)kAmSlots * kAmMaxRows * sizeof(unsigned long long) + R4_TICKET_WORDS * sizeof(unsigned);

// One launch: workgroup (b, row) reduces elements [b chunk, (b + 1) chunk) of its row to one key; the last of the
// row's nblk workgroups (ticket) reduces their keys in a fixed order and writes the result.
template <bool BF16>
__global__ __launch_bounds__(kAmThreads) void am_kernel(const void* __restrict__ x, long long row_stride,
                                                        long long vocab, long long chunk, int nblk, AmScratch sc,
                                                        int* __restrict__ out_idx, float* __restrict__ out_val,
                                                        long long out_stride) {
  const int row = blockIdx.y;
  const long long b = (long long)blockIdx.x * chunk, e = b + chunk < vocab ? b + chunk : vocab;
  const long long base = (long long)row * row_stride;
  unsigned long long k = 0;
  for (long long i0 = b + threadIdx.x; i0 < e; i0 += (long long)kAmThreads * kAmPerThread) {
    float v[kAmPerThread];
#pragma unroll
    for (int u = 0; u < kAmPerThread; ++u) {
      const long long i = i0 + (long long)u * kAmThreads;
      v[u] = __builtin_nanf("");
      if (i < e) v[u] = BF16 ? r4_bf16_to_f32(((const unsigned short*)x)[base + i]) : ((const float*)x)[base + i];
    }
#pragma unroll
    for (int u = 0; u < kAmPerThread; ++u) k = am_max(k, am_key(v[u], (unsigned)(i0 + (long long)u * kAmThreads)));
  }
  __shared__ unsigned long long red[kAmThreads / 64];
  __shared__ int flag;
  k = am_wave_max(k);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = k;
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned long long kb = am_max(am_max(red[0], red[1]), am_max(red[2], red[3]));
    __hip_atomic_store(&sc.keys[row * kAmParts + blockIdx.x], kb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!r4_ticket_last(&sc.tickets[row * R4_TICKET_WORDS], (unsigned)nblk, &flag)) return;
  if (threadIdx.x >= 64) return;
  unsigned long long kr = 0;
  for (int i = threadIdx.x; i < nblk; i += 64)
    kr = am_max(kr, __hip_atomic_load(&sc.keys[row * kAmParts + i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  kr = am_wave_max(kr);
  if (threadIdx.x == 0) {
    int idx;
    float val;
    am_decode(kr, &idx, &val);
    out_idx[row * out_stride] = idx;
    // the winner's own bits (a -0 stays -0); the seed's value when nothing beat it
    if (out_val)
      out_val[row * out_stride] = kr < am_key(-__builtin_inff(), 0u) ? val
                                  : BF16 ? r4_bf16_to_f32(((const unsigned short*)x)[base + idx])
                                         : ((const float*)x)[base + idx];
  }
}

// The scratch of one (device, stream): allocated and zeroed on that stream at its first argmax, kept for the process
// (the reference keeps its argmax partials per stream the same way, src/kernels/src/r4dx_kernels.hip:1715-1734),
// so argmax calls on different streams of one device -- an MTP head beside its model -- never share partials.
// A first call on a stream under graph capture cannot allocate and throws: run one argmax on that stream first.
AmScratch am_scratch(hipStream_t st, const char* entry) {
  static std::mutex mu;
  static std::map<std::pair<int, hipStream_t>, void*> by_stream;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) r4d::fail(entry, "no current device");
  std::lock_guard<std::mutex> lock(mu);
  auto it = by_stream.find({dev, st});
  if (it == by_stream.end()) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
      r4d::fail(entry, "the stream's first argmax is under graph capture, where its scratch cannot be allocated: "
                       "run one argmax on this stream before capturing");
    void* p = nullptr;
    if (hipMalloc(&p, kAmScratchBytes) != hipSuccess) r4d::fail(entry, "scratch allocation failed");
    // cleared on st itself: a null-stream memset is not ordered with a non-blocking stream's next kernel
    r4d::launch_clear(p, kAmScratchBytes, st, entry);
    it = by_stream.emplace(std::make_pair(dev, st), p).first;
  }
  AmScratch s;
  s.keys = (unsigned long long*)it->second;
  s.tickets = (unsigned*)(s.keys + (size_t)kAmMaxRows * kAmParts);
  s.fused_slots = (unsigned long long*)(s.tickets + (size_t)kAmMaxRows * R4_TICKET_WORDS);
  s.fused_ticket = (unsigned*)(s.fused_slots + (size_t)kAmSlots * kAmMaxRows);
  return s;
}

void am_run(bool bf16, int64_t x, int64_t row_stride, int64_t out_idx, int64_t out_val, int64_t out_stride,
            int64_t rows, int64_t vocab, int64_t stream, const char* entry) {
  if (rows < 1 || rows > kAmMaxRows) r4d::fail(entry, "rows must be 1..64");
  if (vocab < 1 || vocab > 0x7FFFFFFFLL) r4d::fail(entry, "vocab must be 1..2^31-1");
  if (!x || !out_idx) r4d::fail(entry, "null buffer");
  hipStream_t st = (hipStream_t)stream;
  const AmScratch sc = am_scratch(st, entry);
  // one batch of kAmPerThread elements per thread and workgroup where kAmParts workgroups allow it
  const long long per = (long long)kAmThreads * kAmPerThread;
  long long nblk = (vocab + per - 1) / per;
  if (nblk > kAmParts) nblk = kAmParts;
  const long long chunk = (vocab + nblk - 1) / nblk;
  nblk = (vocab + chunk - 1) / chunk;
  const dim3 grid((unsigned)nblk, (unsigned)rows);
  if (bf16) hipLaunchKernelGGL(am_kernel<true>, grid, dim3(kAmThreads), 0, st, (const void*)x, (long long)row_stride,
                               (long long)vocab, chunk, (int)nblk, sc, (int*)out_idx, (float*)out_val,
                               (long long)out_stride);
  else hipLaunchKernelGGL(am_kernel<false>, grid, dim3(kAmThreads), 0, st, (const void*)x, (long long)row_stride,
                          (long long)vocab, chunk, (int)nblk, sc, (int*)out_idx, (float*)out_val,
                          (long long)out_stride);
  r4d::launch_ok(entry);
}

void w4_argmax_run(int group, int64_t a, int64_t wq, int64_t wsz, int64_t c, int64_t out_idx, int64_t out_val, int M,
                   int K, int N, int64_t stream, const char* entry) {
  r4d::require(entry, w4_check(group, M, K, N));
  if (!a || !wq || !wsz || !c || !out_idx) r4d::fail(entry, "null buffer");
  hipStream_t st = (hipStream_t)stream;
  const AmScratch sc = am_scratch(st, entry);
  const AmFused af{sc.fused_slots, sc.fused_ticket, (int*)out_idx, (float*)out_val};
  if (group == 32) w4_launch<32, true, true>(a, wq, wsz, c, M, K, N, st, af);
  else w4_launch<64, true, true>(a, wq, wsz, c, M, K, N, st, af);
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

void r4d_gemm_w4a16_nt_m64_f32_argmax(int group, int64_t a, int64_t wq, int64_t wsz, int64_t c, int64_t out_idx,
                                      int64_t out_val, int M, int K, int N, int64_t stream) {
  w4_argmax_run(group, a, wq, wsz, c, out_idx, out_val, M, K, N, stream, "gemm_w4a16_nt_m64_f32_argmax");
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
