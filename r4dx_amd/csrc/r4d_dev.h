// r4d_dev.h -- device-side building blocks shared by every gfx950 kernel of libr4d_mi355x:
// vector types, f16/bf16 rounding, the trellis ("mul1") tile decode into CDNA4 MFMA fragments,
// the wave64 FWHT-128 and small wave utilities.
//
// THE FORMAT (reference: tests/kernels/trellis_ref.hpp:40-115, third_party/libr4d/r4d_trellis_dq.h:8-17).
// A 16 k x 16 n tile is a tail-biting ring of 256*KB bits in 8*KB uint32 words, stream bit 32w at bit
// 31 of word w. Position p owns bits [KB p, KB (p+1)); its 16-bit state is the 16 ring bits ending at
// KB (p+1). The weight is f16((1024 + bytesum(state * 0x83DCD12D mod 2^32)) * f16(0x1EEE) + f16(0xC931)),
// rounded once. Position p = 8t + j with t = 4c + m (c = 0..7, m = 0..3) sits at k = {2m, 2m+1, 2m+8,
// 2m+9}[j & 3] of column c + 8 (j >> 2).
//
// THE LANE MAP (this build's own, for wave64 and v_mfma_f32_16x16x32_f16). A wave reads 1 KiB of the
// pair grid in one coalesced global_load_dwordx4: at KB = 4 that is four consecutive (tile pair,
// k-tile) blocks of one pair. Lane l takes block q = l >> 4, tile t = (l >> 3) & 1 of the pair and
// words 4c..4c+3 (c = l & 7) of that tile's ring -- positions 32c..32c+31, i.e. ALL 16 k of columns c
// and c + 8 -- plus the word before (4c - 1 mod 32, the tail-biting history). It decodes 32 weights
// into four MFMA B fragments F[cs][h] (cs: column c or c + 8; h: the k half), each 8 f16 with element
// e <-> k = 8 (e >> 2) + 4 h + (e & 3) (the same k sets and order as the reference's FragK16, so the
// int8 path can read the reference's A8 layout unchanged). In a 16x16x32 MFMA the B lane l supplies
// column l & 15 and k-group l >> 4: column slot 8t + c is true pair column 16t + c + 8cs and k-group q
// is k-tile q of the step, so the A fragment of lane l must hold row (l & 15), k-tile q, half h in
// that same element order. Nothing else is permuted; the output columns are put back in the epilogue.
//
// THE VALUE PATH per state (s in the high or low half of a 32-bit window W):
//   s = W >> 16 or W & 0xFFFF                        (double-rate VALU on gfx950)
//   x = v_mul_lo_u32(s, 0x83DCD12D)                  (single rate on gfx950, measured)
//   two states -> v_sad_u8 / v_sad_hi_u8 seeded with 0x64006400: the exact f16 bits of 1024 + bytesum
//   one v_pk_fma_f16 with f16(0x1EEE), f16(0xC931): both weights, one rounding each.
// At KB = 4 one v_alignbit window holds the states of (m, j) and (m, j + 4) (the two columns), so 12
// alignbits cover the lane's 32 states. Measured on gfx950 (one full chip of waves): v_mul_lo_u32,
// v_alignbit, v_sad_u8 and v_pk_fma_f16 issue at ~34 T lane-ops/s, v_and / v_lshrrev / v_add_u32
// at ~58 T, so a state costs ~3.4 single-rate issue slots.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// The input parts of a trellis linear: columns [n_end[p - 1], n_end[p]) read a[p] (n_end[3] is past every
// column). One part: every n_end past N; the reference's two-part form: n_end[0] = n_split.
struct R4AParts {
  const unsigned short* a[4];
  int n_end[3];
};
inline R4AParts r4_parts(const void* a0, const void* a1, int n_split, const void* a2 = nullptr, int n_end1 = 0,
                         const void* a3 = nullptr, int n_end2 = 0) {
  R4AParts ap;
  ap.a[0] = (const unsigned short*)a0;
  ap.a[1] = a1 ? (const unsigned short*)a1 : ap.a[0];
  ap.a[2] = a2 ? (const unsigned short*)a2 : ap.a[1];
  ap.a[3] = a3 ? (const unsigned short*)a3 : ap.a[2];
  ap.n_end[0] = n_split;
  ap.n_end[1] = a2 ? n_end1 : 0x7FFFFFFF;
  ap.n_end[2] = a3 ? n_end2 : 0x7FFFFFFF;
  return ap;
}
// the part (0..3) of the 128-column group starting at column n0, and its input (uniform per workgroup: scalar
// compares)
__device__ __forceinline__ int r4_part_idx(const R4AParts& ap, int n0) {
  return n0 < ap.n_end[0] ? 0 : n0 < ap.n_end[1] ? 1 : n0 < ap.n_end[2] ? 2 : 3;
}
__device__ __forceinline__ const unsigned short* r4_part_a(const R4AParts& ap, int n0) {
  return n0 < ap.n_end[0] ? ap.a[0] : n0 < ap.n_end[1] ? ap.a[1] : n0 < ap.n_end[2] ? ap.a[2] : ap.a[3];
}
// The input-transform sign vectors (suh) of a fused-transform launch's parts, selected like R4AParts' inputs.
struct R4SParts {
  const float* s[4];
};

typedef _Float16 r4h8 __attribute__((ext_vector_type(8)));
typedef _Float16 r4h2 __attribute__((ext_vector_type(2)));
typedef float r4f4 __attribute__((ext_vector_type(4)));
typedef float r4f16 __attribute__((ext_vector_type(16)));
typedef unsigned r4u4 __attribute__((ext_vector_type(4)));
typedef unsigned r4u2 __attribute__((ext_vector_type(2)));
typedef float r4f2 __attribute__((ext_vector_type(2)));
typedef int r4i4 __attribute__((ext_vector_type(4)));

#define R4_WAVE 64

// ---- rounding --------------------------------------------------------------------------------
// fp32 -> bf16 bits, nearest even, NaN kept quiet (reference: src/core/include/r4dx/core/dtype.hpp:64-73).
__device__ __forceinline__ unsigned short r4_bf16_rn(float f) {
  const unsigned u = __builtin_bit_cast(unsigned, f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (unsigned short)((u >> 16) | 0x40u);
  return (unsigned short)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
// The same rounding as a select (no branch): in a fully unrolled epilogue an early return becomes divergent control
// flow per element.
__device__ __forceinline__ unsigned short r4_bf16_rn_sel(float f) {
  const unsigned u = __builtin_bit_cast(unsigned, f);
  const unsigned rn = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16, qnan = (u >> 16) | 0x40u;
  return (unsigned short)((u & 0x7FFFFFFFu) > 0x7F800000u ? qnan : rn);
}
// fp32 -> f16 bits, nearest even (v_cvt_f16_f32 under the default round mode). The empty asm keeps
// the caller's fp32 value an fp32 value: without it a preceding multiply may be folded into a
// v_fma_mix with a single rounding, which is not the reference's two-rounding arithmetic.
__device__ __forceinline__ unsigned short r4_f16_rn(float f) {
  asm("" : "+v"(f));
  return __builtin_bit_cast(unsigned short, (_Float16)f);
}
__device__ __forceinline__ float r4_f16_to_f32(unsigned short h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ float r4_bf16_to_f32(unsigned short h) {
  return __builtin_bit_cast(float, (unsigned)h << 16);
}

// ---- weight fake-quant (a measurement hook: the _wq entries) ------------------------------------------------
// Two decoded f16 weights of one column under its group scale s, the reference's rounding
// (third_party/libr4d/r4d_trellis_dq.h:438-470, src/model/fake_quant_w.h:103-118): rs = 1 / s (IEEE division),
// q = clamp(rint(w rs), -127, 127), the fp32 product q s, then one f16 rounding (the empty asm in r4_f16_rn keeps
// the product an fp32 value instead of a fused f16 conversion).
__device__ __forceinline__ unsigned r4_wq_round2(unsigned d, float rs, float s) {
  unsigned o = 0;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const float w = r4_f16_to_f32((unsigned short)(d >> (16 * hh)));
    float q = __builtin_rintf(w * rs);
    q = __builtin_fminf(__builtin_fmaxf(q, -127.0f), 127.0f);
    o |= (unsigned)r4_f16_rn(q * s) << (16 * hh);
  }
  return o;
}
// d[cs][h][j] of a decode lane (columns 8 cs + c of its tile) under the column scales s[cs]
__device__ __forceinline__ void r4_wq_apply(unsigned (&d)[2][2][4], const float (&s)[2]) {
#pragma unroll
  for (int cs = 0; cs < 2; ++cs) {
    const float rs = 1.0f / s[cs];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j) d[cs][h][j] = r4_wq_round2(d[cs][h][j], rs, s[cs]);
  }
}

// ---- the activation producers in front of a trellis linear's input transform ----------------------------
// sigmoid(x) = 1 / (1 + e^-x) in fp32: the device library's expf, a correctly rounded divide (the reference's
// element, src/kernels/src/r4dx_kernels.hip:38, src/kernels/src/trellis_transform.hip:106).
__device__ __forceinline__ float r4_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
// Where a transform reads its input x[row][k] (k inside the row):
//   R4_SRC_X    x itself (bf16 or f16 bits), rows ld apart;
//   R4_SRC_SILU bf16(g * sigmoid(g) * u) with g = p0[row ld + k], u = p0[row ld + off + k] (the MLP's
//               [gate | up] rows; the two products rounded to fp32 in that order, then to bf16 by RNE);
//   R4_SRC_GATE bf16(a * sigmoid(g)) with a = p0[row ld + k], g = p1[row ld + k] (attention's output gate).
// The producers' values are the bf16 numbers a separate producer kernel would have stored.
constexpr int R4_SRC_X = 0, R4_SRC_SILU = 1, R4_SRC_GATE = 2;
struct R4XSrc {
  const unsigned short* p0;
  const unsigned short* p1;
  long long ld, off;
};
// x[row][k] of a transform's input source (see R4XSrc), as fp32
template <int SRC, bool BF16>
__device__ __forceinline__ float r4_xsrc(const R4XSrc& s, long long row, long long k) {
  const long long i = row * s.ld + k;
  if constexpr (SRC == R4_SRC_X) {
    return BF16 ? r4_bf16_to_f32(s.p0[i]) : r4_f16_to_f32(s.p0[i]);
  } else if constexpr (SRC == R4_SRC_SILU) {
    const float g = r4_bf16_to_f32(s.p0[i]), u = r4_bf16_to_f32(s.p0[i + s.off]);
    return r4_bf16_to_f32(r4_bf16_rn(g * r4_sigmoid(g) * u));
  } else {
    const float a = r4_bf16_to_f32(s.p0[i]), g = r4_bf16_to_f32(s.p1[i]);
    return r4_bf16_to_f32(r4_bf16_rn(a * r4_sigmoid(g)));
  }
}

// ---- trellis value path -------------------------------------------------------------------------
#define R4_SAD_SEED 0x64006400u     // f16 1024.0 in both halves
#define R4_KINV2 0x1EEE1EEEu
#define R4_KBIAS2 0xC931C931u

// x = s * 0x83DCD12D mod 2^32 for the state in the HIGH half of w: a double-rate shift isolates
// the state and one full-rate v_mul_lo_u32 (not quarter rate on gfx950) forms the product.
__device__ __forceinline__ unsigned r4_hash_hi(unsigned w) { return (w >> 16) * 0x83DCD12Du; }
// ... for the state in the LOW half of w (a double-rate mask).
__device__ __forceinline__ unsigned r4_hash_lo(unsigned w) { return (w & 0xFFFFu) * 0x83DCD12Du; }
// Two hashes -> the packed f16 pair (x0's weight in the low half, x1's in the high half).
__device__ __forceinline__ unsigned r4_cb_pair(unsigned x0, unsigned x1) {
  const unsigned s0 = __builtin_amdgcn_sad_u8(x0, 0u, R4_SAD_SEED);
  const unsigned s1 = __builtin_amdgcn_sad_hi_u8(x1, 0u, s0);
  const r4h2 v = __builtin_elementwise_fma(__builtin_bit_cast(r4h2, s1), __builtin_bit_cast(r4h2, R4_KINV2),
                                           __builtin_bit_cast(r4h2, R4_KBIAS2));
  return __builtin_bit_cast(unsigned, v);
}

// The 32-bit stream window starting at bit b (relative to the first own word; -32 <= b, b a
// compile-time constant) of the lane's words W[0] = history, W[1..] = own words.
template <int B>
__device__ __forceinline__ unsigned r4_window(const unsigned* W) {
  constexpr int i = (B + 32) / 32 - 1 + 1;     // index into W (history at 0) of the word holding bit B
  constexpr int off = (B + 32) % 32;
  if constexpr (off == 0) return W[i];
  else return __builtin_amdgcn_alignbit(W[i], W[i + 1], 32 - off);
}

// The history word of a decode lane: the word before its own KB words in its tile's ring of 8 KB words
// (lane c of an 8-lane group owns words KB c .. KB c + KB - 1) is the last own word of lane c - 1 mod 8
// of the same group. Two DPP moves inside the 16-lane row (row_shr:1 gives lane i the value of lane
// i - 1, row_shl:7 that of lane i + 7) and a select for c = 0 replace a second load per step.
__device__ __forceinline__ unsigned r4_hist_word(unsigned last, int lane) {
  const unsigned from_prev = (unsigned)__builtin_amdgcn_mov_dpp((int)last, 0x111, 0xF, 0xF, true);
  const unsigned from_wrap = (unsigned)__builtin_amdgcn_mov_dpp((int)last, 0x107, 0xF, 0xF, true);
  return (lane & 7) == 0 ? from_wrap : from_prev;
}

// Fragment element of position (m, j) of column slot cs = j >> 2: half h = m >> 1,
// e = 4 ((j >> 1) & 1) + 2 (m & 1) + (j & 1)  (k = 2m + (j & 1) + 8 ((j >> 1) & 1)).
// The decode writes each fragment as 4 dwords d[cs][h][e >> 1] (two elements per dword).
//
// KB = 4: W[0] history, W[1..4] the lane's words 4c..4c+3. window(m, j), j < 4, starts at stream
// bit 32m + 4j - 12: its high half is the state of (m, j) [column c], its low half the state of
// (m, j + 4) [column c + 8]; j = 3 is a raw word.
template <int M>
__device__ __forceinline__ void r4_decode_k4_m(const unsigned* W, unsigned (&d)[2][2][4]) {
  constexpr int h = M >> 1, mo = M & 1;
  const unsigned w0 = r4_window<32 * M - 12>(W), w1 = r4_window<32 * M - 8>(W);
  const unsigned w2 = r4_window<32 * M - 4>(W), w3 = r4_window<32 * M>(W);
  d[0][h][0 + mo] = r4_cb_pair(r4_hash_hi(w0), r4_hash_hi(w1));
  d[0][h][2 + mo] = r4_cb_pair(r4_hash_hi(w2), r4_hash_hi(w3));
  d[1][h][0 + mo] = r4_cb_pair(r4_hash_lo(w0), r4_hash_lo(w1));
  d[1][h][2 + mo] = r4_cb_pair(r4_hash_lo(w2), r4_hash_lo(w3));
}
__device__ __forceinline__ void r4_decode_k4(const unsigned* W, unsigned (&d)[2][2][4]) {
  r4_decode_k4_m<0>(W, d);
  r4_decode_k4_m<1>(W, d);
  r4_decode_k4_m<2>(W, d);
  r4_decode_k4_m<3>(W, d);
}

// Generic KB (3 or 5): W[0] history, W[1..KB] the lane's words KB c .. KB c + KB - 1 (positions
// 32c..32c+31 occupy exactly those KB words). One window per state, its state in the low half:
// the window ending at the state's end bit.
template <int KB, int M, int J>
__device__ __forceinline__ unsigned r4_state_window(const unsigned* W) {
  constexpr int p = 8 * M + J;
  return r4_window<KB * (p + 1) - 32>(W);
}
template <int KB, int M, int J>
__device__ __forceinline__ unsigned r4_hash_mj(const unsigned* W) {
  return r4_hash_lo(r4_state_window<KB, M, J>(W));
}
template <int KB, int M>
__device__ __forceinline__ void r4_decode_gen_m(const unsigned* W, unsigned (&d)[2][2][4]) {
  constexpr int h = M >> 1, mo = M & 1;
  d[0][h][0 + mo] = r4_cb_pair(r4_hash_mj<KB, M, 0>(W), r4_hash_mj<KB, M, 1>(W));
  d[0][h][2 + mo] = r4_cb_pair(r4_hash_mj<KB, M, 2>(W), r4_hash_mj<KB, M, 3>(W));
  d[1][h][0 + mo] = r4_cb_pair(r4_hash_mj<KB, M, 4>(W), r4_hash_mj<KB, M, 5>(W));
  d[1][h][2 + mo] = r4_cb_pair(r4_hash_mj<KB, M, 6>(W), r4_hash_mj<KB, M, 7>(W));
}
template <int KB>
__device__ __forceinline__ void r4_decode_gen(const unsigned* W, unsigned (&d)[2][2][4]) {
  r4_decode_gen_m<KB, 0>(W, d);
  r4_decode_gen_m<KB, 1>(W, d);
  r4_decode_gen_m<KB, 2>(W, d);
  r4_decode_gen_m<KB, 3>(W, d);
}

template <int KB>
__device__ __forceinline__ void r4_decode(const unsigned* W, unsigned (&d)[2][2][4]) {
  if constexpr (KB == 4) r4_decode_k4(W, d);
  else r4_decode_gen<KB>(W, d);
}

__device__ __forceinline__ r4h8 r4_frag(const unsigned (&d)[4]) {
  const r4u4 u = {d[0], d[1], d[2], d[3]};
  return __builtin_bit_cast(r4h8, u);
}

// Word index (inside the lane's tile ring of 8 KB words) of W[i], i = 0 the history.
template <int KB>
__device__ __forceinline__ int r4_lane_word(int c, int i) {
  return (KB * c - 1 + i + 8 * KB) % (8 * KB);
}

// ---- wave64 FWHT-128 --------------------------------------------------------------------------
// Lane l holds v0 = element l and v1 = element l + 64 of one 128-block. Stages lg = 0..6 in order,
// each pair (i, i + 2^lg) -> (a + b, a - b) in fp32 (reference order: tests/kernels/trellis_ref.hpp:
// 120-131): for lg < 6 the partner is lane l ^ 2^lg and the lower index keeps a + b, the upper takes
// a - b (= partner - own); lg = 6 pairs the two registers.
// v of lane l ^ mask (mask a power of two below 64, a compile-time constant after unrolling). Masks 1-8 are
// DPP moves inside a row of 16 lanes (ALU latency; 4 and 8 as two mirrors: (l ^ 7) ^ 3 = l ^ 4, (l ^ 15) ^ 7
// = l ^ 8), 16 a ds_swizzle inside 32 lanes, 32 a ds_bpermute. Pure data movement: the values are unchanged.
__device__ __forceinline__ int r4_xor_lane_i(int v, int mask) {
  switch (mask) {
    case 1: return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);     // quad_perm [1, 0, 3, 2]
    case 2: return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);     // quad_perm [2, 3, 0, 1]
    case 4: return __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true), 0x1B, 0xF, 0xF, true);
    case 8: return __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, true), 0x141, 0xF, 0xF, true);
    case 16: return __builtin_amdgcn_ds_swizzle(v, (16 << 10) | 0x1F);  // bit mode, xor 16 inside 32 lanes
    default: return __shfl_xor(v, mask, R4_WAVE);
  }
}
__device__ __forceinline__ float r4_xor_lane(float v, int mask) {
  return __builtin_bit_cast(float, r4_xor_lane_i(__builtin_bit_cast(int, v), mask));
}
__device__ __forceinline__ void r4_fwht128_wave(float& v0, float& v1, int lane) {
#pragma unroll
  for (int lg = 0; lg < 6; ++lg) {
    const int hm = 1 << lg;
    const float p0 = r4_xor_lane(v0, hm), p1 = r4_xor_lane(v1, hm);
    const bool upper = (lane & hm) != 0;
    v0 = upper ? p0 - v0 : v0 + p0;
    v1 = upper ? p1 - v1 : v1 + p1;
  }
  const float a = v0, b = v1;
  v0 = a + b;
  v1 = a - b;
}
// The same transform with lane l holding elements 2 l (v0) and 2 l + 1 (v1): stage 0 pairs the two
// registers, stage lg >= 1 pairs lane l with lane l ^ 2^(lg - 1). Every element sees the same fp32
// operations in the same order as in r4_fwht128_wave.
__device__ __forceinline__ void r4_fwht128_wave_pairs(float& v0, float& v1, int lane) {
  {
    const float a = v0, b = v1;
    v0 = a + b;
    v1 = a - b;
  }
#pragma unroll
  for (int lg = 1; lg < 7; ++lg) {
    const int hm = 1 << (lg - 1);
    const float p0 = r4_xor_lane(v0, hm), p1 = r4_xor_lane(v1, hm);
    const bool upper = (lane & hm) != 0;
    v0 = upper ? p0 - v0 : v0 + p0;
    v1 = upper ? p1 - v1 : v1 + p1;
  }
}

// ---- misc ----------------------------------------------------------------------------------------
__device__ __forceinline__ r4f4 r4_mfma16(r4h8 a, r4h8 b, r4f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Grid-wide handoff of split partial sums. The partials are written with r4_store_coherent (agent-
// scope relaxed atomic stores: write-through past this XCD's L2) and read back with r4_load_coherent,
// so no agent-scope fence -- which on gfx950 writes back or invalidates the whole L2 of the XCD, a
// ~1 us serialisation per workgroup -- is needed: each thread waits for its own stores to be
// acknowledged (the workgroup-scope release), the block meets at a barrier, one thread takes a
// ticket; the block that completes the count finishes the group and resets the ticket to zero (the
// reference's self-resetting protocol, third_party/libr4d/r4d.h:365-371). Returns true in every
// thread of the last block.
__device__ __forceinline__ void r4_store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float r4_load_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Words per ticket: each 128-column group's counter owns a 128-byte line (the GEMV's ticket layout).
#define R4_TICKET_WORDS 32
__device__ __forceinline__ bool r4_ticket_last(unsigned* ticket, unsigned contributors, int* flag_lds) {
  // every coherent store of this thread acknowledged before the barrier (the workgroup-scope fence
  // alone emits no wait on gfx950)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old == contributors - 1;
    if (last) __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag_lds = last ? 1 : 0;
  }
  __syncthreads();
  return *flag_lds != 0;
}
