/* r4o.h -- CPU oracle for r4dx's quantized-weight matrix-product path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (r4dx_amd/, include/) may link, load or call
 * this code.  It is the checker the GPU kernels are compared against, restated in plain C from the
 * mathematics of the reference's CPU references (citations per function, paths relative to the
 * reference repository root).  Built by oracle/Makefile into oracle/_build/libr4o.so.
 *
 * Pinning (what holds each function to the reference, see tests/test_oracle.py):
 *   codebook / state / perm / pair grid .. known answers from tests/reference/test_trellis_quant.py
 *                                          (min, max, mean, std, distinct count, perm[0:8], [40:48]),
 *                                          and bit-equality with the reference's own trellis_ref.hpp
 *                                          compiled into oracle/_ref (when buildable).
 *   fwht128 ................................ H*H = 128 I, equality with a dense Sylvester matrix,
 *                                          and bit-equality with trellis_ref.hpp's FwhtLdsF32.
 *   transform / epilogue / linear ......... bit-equality with trellis_ref.hpp (oracle/_ref),
 *                                          fp64 closed forms (one-hot rows return rows of Q).
 *   int8 quantizers / reference GEMM ...... int8_gemm_proto_ref.h via oracle/_ref; exact integer
 *                                          brute force; single-nonzero-activation identities.
 *   w4a16 quantize + pack ................. byte-exact against tests/convert/fixtures/w4a16_*_g64.bin
 *                                          (committed copies in tests/golden/).
 *   argmax ................................. the order algebra of argmax_ref.hpp on NaN/-inf/ties.
 */
#ifndef R4O_H
#define R4O_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions (IEEE binary16 / bfloat16, round to nearest even) ---------------------- */
float    r4o_f16_to_f32(uint16_t h);
uint16_t r4o_f32_to_f16(float f);
uint16_t r4o_f64_to_f16(double x);
float    r4o_bf16_to_f32(uint16_t h);
uint16_t r4o_f32_to_bf16(float f);

/* ---- trellis format (tests/kernels/trellis_ref.hpp:40-115) ------------------------------------- */
void     r4o_codebook(uint16_t* out65536);                         /* trellis_ref.hpp:40-53  */
uint32_t r4o_trellis_state(const uint32_t* ring, int KB, int p);   /* trellis_ref.hpp:56-62  */
int      r4o_tc_perm(int p);                                       /* trellis_ref.hpp:65-70  */
size_t   r4o_pair_grid_index(int64_t K, int KB, int64_t tn, int64_t tk); /* :81-83           */
/* oracle layout [K/16][N/16][8KB] -> pair grid (trellis_ref.hpp:98-107) */
void     r4o_to_pair_grid(const uint32_t* words, int64_t K, int64_t N, int KB, uint32_t* grid);
/* pair grid -> Q[K][N] f16 bits (trellis_ref.hpp:109-115); nthreads <= 0: all cores */
void     r4o_decode_pair_grid(const uint32_t* grid, int64_t K, int64_t N, int KB, uint16_t* q,
                              int nthreads);

/* ---- FWHT-128 and the linear around the decode (trellis_ref.hpp:118-247) --------------------- */
void     r4o_fwht128_f32(float* v);                                /* trellis_ref.hpp:120-131 */
void     r4o_fwht128_f64(double* v);                               /* trellis_ref.hpp:134-143 */
float    r4o_transform_scale(int prescale_log2);                   /* trellis_ref.hpp:146-148 */
/* x: [M][K] bits, x_is_bf16 selects bf16 (the reference's r4dx_trellis_input_bf16) or f16 input;
 * suh fp32 [K]; a: f16 bits [M][K]  (trellis_ref.hpp:150-169, trellis_transform.hip:63-100) */
/* the activation producers (pinned: sigmoid's closed forms -- 0 -> 1/2, saturation at +-large -- and a float64
 * restatement within one bf16 ulp, tests/test_oracle.py) */
void     r4o_silu_mul_bf16(const uint16_t* gate_up, int64_t rows, int64_t intermediate, int64_t in_row_stride,
                           uint16_t* out);
void     r4o_attn_gate_mul_bf16(const uint16_t* attn_out, const uint16_t* gate, int64_t n, uint16_t* out);
void     r4o_transform_input(const uint16_t* x, int x_is_bf16, int64_t M, int64_t K,
                             const float* suh, int prescale_log2, uint16_t* a);
/* fp64 sums S[m][n] = sum_k A_p(n)[m][k] Q[k][n] (no output transform: the _raw entry's quantity) */
void     r4o_raw_sums_f64(const uint16_t* a0, const uint16_t* a1, int64_t n_split, int64_t M,
                          int64_t K, int64_t N, const uint16_t* q, double* s, int nthreads);
/* trellis_ref.hpp:173-196 LinearFromA: y fp64 [M][N] */
void     r4o_linear_from_a(const uint16_t* a0, const uint16_t* a1, int64_t n_split, int64_t M,
                           int64_t K, int64_t N, const uint16_t* q, const float* svh,
                           int prescale_log2, double* y, int nthreads);
/* trellis_ref.hpp:231-247 EpilogueFromRaw: fp32 sums -> bf16 bits */
void     r4o_epilogue_from_raw(const float* s, int64_t M, int64_t N, const float* svh,
                               float out_scale, uint16_t* c);

/* ---- int8 quantizers and reference (tests/kernels/int8_gemm_proto_ref.h) -------------------- */
uint16_t r4o_i8_rs_half(float s);                       /* int8_gemm_proto_ref.h:57-62 RsHalf  */
float    r4o_i8_seff(float s);                          /* :63 SEff                            */
int8_t   r4o_i8_quant_w(uint16_t wbits, uint16_t rsbits);  /* :74-77 QuantWTrick              */
int8_t   r4o_i8_quant_act(float x, float s);            /* :85-89 QuantAct                     */
/* per-(row,128) activation scales: X f16 bits [M][K] -> sa [K/128][M], ap [M][K] (:138-149) */
void     r4o_i8_quant_act_blk(const uint16_t* x, int M, int K, float* sa, int8_t* ap);
/* per-row activation scales (:178-189): sa [M], ap [M][K] */
void     r4o_i8_quant_act_row(const uint16_t* x, int M, int K, float* sa, int8_t* ap);
/* weight side from decoded Q [K][N]: per (col,128) table sw [K/128][N] (:124-137) or per column
 * sw [N] (:164-176), wp plain [N][K] */
void     r4o_i8_quant_w_blk(const uint16_t* q, int K, int N, float* sw, int8_t* wp);
void     r4o_i8_quant_w_col(const uint16_t* q, int K, int N, float* sw, int8_t* wp);
/* exact int32 sums acc[m][n] = sum_k A[m][k] W[n][k] (A [M][K], W [N][K]) */
void     r4o_i8_gemm_i32(const int8_t* a, const int8_t* w, int M, int N, int K, int32_t* acc,
                         int nthreads);
/* int8_gemm_proto_ref.h:95-110 RefGemmInt8 (fp64); mask bit0: sa per row, bit1: sw per column */
void     r4o_i8_gemm_ref(const int8_t* a, const float* sa, const int8_t* w, const float* sw,
                         int M, int N, int K, int mask, double* c, int nthreads);
/* A8 fragment layout of r4d_trellis_i8_layout.h:32-45 (plain [256][K] -> A8 bytes) */
size_t   r4o_a8_offset(int r, int k, int K);
void     r4o_pack_a8(const int8_t* ap, int K, int8_t* a8);
size_t   r4o_w8_offset(int n, int k, int K);
void     r4o_pack_w8(const int8_t* wp, int N, int K, int8_t* w8);

/* ---- w4a16 (src/convert/include/r4dx_convert/quant_int4.hpp) ---------------------------------- */
/* quant_int4.hpp:95-160 QuantizeInt4Asymmetric: w fp32 [N][K] -> q [N][K] 0..15, scale/zero
 * [N][K/group] */
void     r4o_w4_quantize(const float* w, int N, int K, int group, uint8_t* q, float* scale,
                         uint8_t* zero);
/* quant_int4.hpp:171-198 PackW4Nibbles: q -> wq u32 [N*K/8] */
void     r4o_w4_pack(const uint8_t* q, int N, int K, uint32_t* wq);
/* quant_int4.hpp:222-244 PackW4A16Scales: -> wsz u32 [N/16][K/group][16] */
void     r4o_w4_pack_scales(const float* scale, const uint8_t* zero, int N, int K, int group,
                            uint32_t* wsz);
/* dequant of the packed form: W[n][k] = f16(scale) * ((nibble ^ 8) - zero) as fp32 [N][K] */
void     r4o_w4_dequant(const uint32_t* wq, const uint32_t* wsz, int N, int K, int group,
                        float* w);
/* y[m][n] = sum_g scale * sum_{k in g} A[m][k] (q - zero), fp64; A f16 bits [M][K] */
void     r4o_w4_gemm_ref(const uint16_t* a, const uint32_t* wq, const uint32_t* wsz, int M, int N,
                         int K, int group, double* y, int nthreads);

/* ---- weight fake-quant (src/model/fake_quant_w.h:96-140; pinned: bit-equality with that header's
 * FakeQuantWTableRef / FakeQuantWApplyRef through oracle/_ref, all-zero groups -> 1, int8-grid fixed points,
 * ties to even, the s / 2 error bound, tests/test_oracle.py) ------------------------------------------ */
/* q f16 bits [K][N] -> t [K/group][N] */
void     r4o_wq_table(const uint16_t* q, int64_t K, int64_t N, int group, float* t);
/* q -> f16 bits of the rounded weight Q' [K][N] */
void     r4o_wq_apply(const uint16_t* q, int64_t K, int64_t N, int group, const float* t, uint16_t* out);

/* ---- argmax (src/kernels/include/r4dx/kernels/argmax_ref.hpp:22-41) ------------------------- */
int32_t  r4o_argmax_f32(const float* x, int64_t n, float* best_val);

/* ---- timing helper for the CPU baseline: decode + matmul of one trellis linear --------------- */
double   r4o_now_seconds(void);
int      r4o_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
