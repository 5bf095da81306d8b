/* r4d_mi355x.h -- the C ABI of libr4d_mi355x, the MI355X (gfx950) build of r4dx's quantized-weight
 * matrix-product path.  Every entry keeps the name, argument order and meaning of the reference
 * entry it replaces (cited per declaration, paths relative to the reference repository root), so the
 * engine's callers (src/model/linear.cpp ApplyLinear via src/core/include/r4dx/core/r4d.hpp) bind it
 * unchanged.  Device pointers and streams travel as int64_t, shapes as int.  Nothing on a launch
 * path allocates or synchronises.  An illegal shape throws std::runtime_error from the GEMM entries
 * (as the reference's do); every GEMM family also has a _check entry that returns NULL or a message
 * (valid until the calling thread's next check) without launching.
 *
 * Tuning knobs of the reference signatures (WV, MT, NP, U, NT, skw) are accepted and ignored:
 * this build plans its own geometry.  SKG (the grid K split) is honoured, because the caller sizes
 * ws by it.  SK of the M <= 64 GEMM chooses the summation order: SK = 1 or 2 runs one wave per tile
 * pair over the whole K slice (the order r4d_gemm_trellis_nt_m256 reproduces, so the engine's
 * PlanTrellisM256 -- which asks for a K-slice grouping skw <= SK, src/model/linear.cpp:705-722 -- can
 * plan an M = 64 row of SK 2); any other SK (0, 4, 8, 16), with ws and tickets given or SKG > 1, splits
 * each slice over 4 waves added in k order (an unsplit launch without ws always runs the one-wave form).
 * Results depend on (K, N, KB, SKG, that form) and never on M.  The MI355X tuning rows in the engine's
 * own formats are r4dx_amd/tables/ *.inc.
 */
#ifndef R4D_MI355X_H
#define R4D_MI355X_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- trellis GEMV / skinny GEMM, M = 1..64 ----------------------------------------------------- */
/* third_party/libr4d/r4d.h:372-375 r4d_gemm_trellis_nt_m64: C bf16 [M][N] =
 * bf16((FWHT128(A_p(n) @ Q) * svh) * out_scale); A f16 [M][K] (a1 = 0: a0), W the pair-grid words,
 * ws fp32 ws_bytes(M, N, SKG) (SKG M N 4 at most 2 GiB), tickets tickets_bytes(N) (one 128-byte line per
 * 128-column group) zeroed before first use (self-resetting). */
void r4d_gemm_trellis_nt_m64(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t svh, int64_t c,
                             int64_t ws, int64_t tickets, int M, int K, int N, int KB, int WV, int SK,
                             int MT, int NP, int SKG, int U, int NT, float out_scale, int64_t stream);
/* r4d.h:376-383 _raw: fp32 C [M][N] = A @ Q, no output transform; clk (0 = off): 4 uint64 that workgroup
   (0, 0)'s thread 0 fills with the shader clock and the 100 MHz wall clock at entry and at the end of its own
   work. */
void r4d_gemm_trellis_nt_m64_raw(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t c, int64_t ws,
                                 int64_t tickets, int M, int K, int N, int KB, int WV, int SK, int MT,
                                 int NP, int SKG, int U, int NT, int64_t clk, int64_t stream);
int    r4d_gemm_trellis_nt_m64_has_rate(int KB);                 /* r4d.h:384 */
int    r4d_gemm_trellis_nt_m64_max_m(void);                      /* r4d.h:385 */
size_t r4d_gemm_trellis_nt_m64_ws_bytes(int M, int N, int SKG);  /* r4d.h:386 */
size_t r4d_gemm_trellis_nt_m64_tickets_bytes(int N);             /* r4d.h:387: N/128 lines of 128 B */
/* r4d.h:389. Zeroes with a fill kernel on `stream` (no memset node: graph-capturable); tickets 4-byte aligned. */
void   r4d_gemm_trellis_nt_m64_zero_tickets(int64_t tickets, size_t bytes, int64_t stream);
/* r4d.h:390-393: the whole decoded Q[K][N] f16 bits, bit-exact against the format's decode. */
void   r4d_trellis_reconstruct_f16(int64_t w, int64_t q, int K, int N, int KB, int64_t stream);
/* No reference counterpart (the reference checks inside the throwing entry, r4d_gemm_trellis_nt_m64.hip:
 * 614-650): the legality rules of the two entries above without launching. */
const char* r4d_gemm_trellis_nt_m64_check(int M, int K, int N, int n_split, int KB, int SKG, int full,
                                          int have_svh, int have_ws);
/* No reference counterpart (the reference reads gemm_tuning_table_trellis.inc): this build's SKG for
 * a shape, the same for every M. */
int    r4d_mi355x_trellis_gemv_skg(int K, int N, int KB);
/* No reference counterpart (the engine runs r4dx_trellis_input_bf16 then r4d_gemm_trellis_nt_m64): the two
 * fused -- x f16 (x_is_bf16 = 0) or bf16 [M][K], suh0 (columns < n_split) / suh1 fp32 [K], prescale_log2 as the
 * transform's -- each workgroup transforms its own K slice into LDS. Bit-identical to the two-launch path.
 * Needs (K / 128) % SKG == 0 and the slice in LDS (r4dx_trellis_gemv_xf_check). */
void r4dx_trellis_gemv_xf(int64_t x, int x_is_bf16, int64_t suh0, int64_t suh1, int n_split, int prescale_log2,
                          int64_t w, int64_t svh, int64_t c, int64_t ws, int64_t tickets, int M, int K, int N, int KB,
                          int SKG, float out_scale, int64_t stream);
const char* r4dx_trellis_gemv_xf_check(int M, int K, int N, int n_split, int KB, int SKG, int have_ws);
/* No reference counterpart (the engine runs r4dx_trellis_input_bf16 with nout suh, then one GEMV per projection): the
 * input transform fused into r4dx_gemm_trellis_nt_m64_parts -- projections that read one input x (q | k | v, gdn
 * qkv | z), stored as one linear, as ONE launch; columns [n0[p], n0[p + 1]) use suh[p] (host arrays of `parts`, 1..4,
 * n0 as for _parts). Bit-identical to the transform followed by the parts launch at the same SKG. */
const char* r4dx_trellis_gemv_xf_parts_check(int parts, const int* n0, int M, int K, int N, int KB, int SKG,
                                             int have_ws);
void r4dx_trellis_gemv_xf_parts(int64_t x, int x_is_bf16, const int64_t* suh, const int* n0, int parts,
                                int prescale_log2, int64_t w, int64_t svh, int64_t c, int64_t ws, int64_t tickets,
                                int M, int K, int N, int KB, int SKG, float out_scale, int64_t stream);

/* No reference counterpart: for callers that cannot allocate or hold a workspace (code under HIP graph capture,
 * serving loops that forbid hipMalloc). r4d_gemm_trellis_nt_m64 (same C, A parts, SK and SKG meaning) with no ws or
 * tickets argument: the split partials and tickets live in a device array the library holds per GPU until the
 * process ends (16 MiB of partials -- SKG M N 4 bytes at most, r4dx_gemm_trellis_nt_m64_noalloc_max_ws_bytes() --
 * and tickets for N up to 262144). Nothing is allocated on any call. Every call on one GPU shares that GPU's array,
 * whatever its stream: calls that overlap on one GPU race, so callers on several streams of one GPU (an MTP head
 * beside the model) must order their calls (one stream, or events between them). The _check form returns NULL or the rule a launch breaks (sizes beyond the
 * array included); the entry throws on the same. */
void r4dx_gemm_trellis_nt_m64_noalloc(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t svh, int64_t c, int M,
                                      int K, int N, int KB, int SK, int SKG, float out_scale, int64_t stream);
const char* r4dx_gemm_trellis_nt_m64_noalloc_check(int M, int K, int N, int n_split, int KB, int SKG);
size_t r4dx_gemm_trellis_nt_m64_noalloc_max_ws_bytes(void);

/* ---- trellis prefill GEMM, M = 128 or 256 ------------------------------------------------------ */
/* r4d.h:416-419 r4d_gemm_trellis_nt_m256: the linear of r4d_gemm_trellis_nt_m64 for 128 or 256 rows
 * (two launches when SKG > 1: the slices, then their sum and the epilogue); ws fp32 ws_bytes(M, N,
 * SKG) required when SKG > 1 (the reference always requires it); tickets accepted and unused;
 * (K/16) must be divisible by 4 SKG. Every element equals, bit for bit, r4d_gemm_trellis_nt_m64's at
 * M = 64 with the same SK, SKG, ws and tickets (r4d.h:402-412): SK 0, 1 or 2 (0 means 1) the one-wave-per-pair
 * order; SK 4, 8 or 16 the 4-wave split order, which (like that kernel) it runs when SKG > 1 or ws and tickets are
 * given, else the one-wave order -- in two launches per 128-row half plus their finish passes, 1.4-1.8x the
 * one-wave form's time, data-parallel only. Any other SK is refused. NP, U, skw unused. */
void r4d_gemm_trellis_nt_m256(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t svh, int64_t c,
                              int64_t ws, int64_t tickets, int M, int K, int N, int KB, int SK, int NP,
                              int SKG, int U, float out_scale, int64_t stream, int skw);
/* r4d.h:420-421: NULL when the launch is legal, else the first rule it breaks. */
const char* r4d_gemm_trellis_nt_m256_check(int M, int K, int N, int n_split, int KB, int SK, int NP,
                                           int SKG, int U, int skw);
size_t r4d_gemm_trellis_nt_m256_ws_bytes(int M, int N, int SKG);   /* r4d.h:423 */
/* No reference counterpart (the m256 test entry of this build, like r4d_gemm_trellis_nt_m64_raw):
 * fp32 C = A @ Q with no output transform. */
void r4d_gemm_trellis_nt_m256_raw(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t c, int64_t ws,
                                  int64_t tickets, int M, int K, int N, int KB, int SKG, int64_t stream);
/* No reference counterpart (the reference plans with PlanTrellisM256, src/model/linear.cpp:680-724):
 * this build's SKG for a prefill shape. */
int r4d_mi355x_trellis_m256_skg(int K, int N, int KB);

/* ---- w4a16 group-quantized skinny GEMM (LM head, drafters) ------------------------------------- */
/* r4d.h:331-333: C bf16 [M][N] = A f16 [M][K] @ dequant(Wq, Wsz)^T at the build-default group 64; Wq in
 * the packed fragment order of quant_int4.hpp:171-198, Wsz (tile, group, row) dwords = f16 scale | f16
 * (-(1024 + zero)) << 16. WV, SK, MB, NPW, NT accepted and unused. M 1..64 at any K (A is staged in LDS in
 * K chunks), N % 16 == 0, K % 64 == 0. */
void r4d_gemm_w4a16_nt_m64(int64_t a, int64_t wq, int64_t wsz, int64_t c, int M, int K, int N, int WV, int SK,
                           int MB, int NPW, int NT, int64_t stream);
int  r4d_gemm_w4a16_nt_m64_max_m(void);            /* r4d.h:333 */
int  r4d_gemm_w4a16_nt_m64_group(void);            /* r4d.h:334 */
int  r4d_gemm_w4a16_nt_m64_has_group(int group);   /* r4d.h:340: 1 for 32 and 64 */
/* r4d.h:341-342: the same at a per-call group (32 or 64). */
void r4d_gemm_w4a16_nt_m64_g(int group, int64_t a, int64_t wq, int64_t wsz, int64_t c, int M, int K, int N, int WV,
                             int SK, int MB, int NPW, int NT, int64_t stream);
/* No reference counterpart: the legality rules of the two entries above without launching. */
const char* r4d_gemm_w4a16_nt_m64_check(int group, int M, int K, int N);
/* No reference counterpart (fp32 logits for the LM head's argmax; the reference C is bf16): the
 * same GEMM with fp32 C [M][N]. */
void r4d_gemm_w4a16_nt_m64_f32(int group, int64_t a, int64_t wq, int64_t wsz, int64_t c, int M, int K, int N,
                               int64_t stream);

/* ---- argmax (src/kernels/include/r4dx/kernels/kernels.h:297-330) -------------------------------- */
/* out_idx[0] = argmax over logits[0, vocab): larger value first, then lower index; a NaN never wins,
 * a row with nothing above -inf gives index 0 (argmax_ref.hpp:22-41). One launch; its partial keys and
 * tickets live in a scratch per (device, stream) that the library allocates at the stream's first argmax
 * (so that first call must not be under graph capture) and keeps, as the reference keeps its partials per
 * stream (r4dx_kernels.hip:1715-1734): calls on different streams never share it. */
void r4dx_argmax_f32(int64_t logits, int64_t out_idx, int64_t vocab, int64_t stream);          /* :308 */
void r4dx_argmax_val_f32(int64_t logits, int64_t out_idx, int64_t out_val, int64_t vocab,
                         int64_t stream);                                                       /* :316 */
void r4dx_argmax_bf16(int64_t logits, int64_t out_idx, int64_t vocab, int64_t stream);         /* :320 */
void r4dx_argmax_val_bf16(int64_t logits, int64_t out_idx, int64_t out_val, int64_t vocab,
                          int64_t stream);                                                      /* :321 */
/* kernels.h:328-329: rows (at most 64 here, 16 in the reference) of a [rows][row_stride] logits array;
 * row r's result at out_idx[r * out_stride] (and out_val[r * out_stride] when out_val != 0). */
void r4dx_argmax_rows_f32(int64_t logits, int64_t row_stride, int64_t out_idx, int64_t out_val,
                          int64_t out_stride, int64_t rows, int64_t vocab, int64_t stream);
/* No reference counterpart (the LM head's GEMM and argmax in one launch, for the decode step that
 * reads back only the token): r4d_gemm_w4a16_nt_m64_f32's logits c [M][N] plus r4dx_argmax_rows_f32's
 * result per row, out_idx[m] and out_val[m] (out_val may be 0), bit for bit the two calls' results.
 * Uses the same per-(device, stream) scratch as the argmax entries (first call not under capture). */
void r4d_gemm_w4a16_nt_m64_f32_argmax(int group, int64_t a, int64_t wq, int64_t wsz, int64_t c, int64_t out_idx,
                                      int64_t out_val, int M, int K, int N, int64_t stream);

/* ---- int8 x int8 prefill GEMM and its activation quantizers ------------------------------------ */
/* r4d.h:490-491 r4d_trellis_i8_quant_act: x f16 [256][K] (part p at x + p part_stride elements) -> the A8
 * fragment layout (r4d_trellis_i8_layout.h:32-45) at a8 + p 256 K bytes, SA [K/128][256] per part at
 * sa + p (K/128) 256 floats; s = amax / 127 per (row, 128 k) (1 for all zero), q = clamp(rint(x / s)). */
void r4d_trellis_i8_quant_act(int64_t x, int64_t a8, int64_t sa, int parts, int64_t part_stride, int K,
                              int64_t stream);
/* r4d.h:517-518 r4d_trellis_i8_quant_act_row: the same with one scale per row, SA [256] per part. */
void r4d_trellis_i8_quant_act_row(int64_t x, int64_t a8, int64_t sa, int parts, int64_t part_stride, int K,
                                  int64_t stream);
/* kernels.h:149-161 r4dx_trellis_input_i8: r4dx_trellis_input_bf16's arguments and arithmetic up to the f16 A, which
 * is not stored: each (row, 128-block) goes through r4d_trellis_i8_quant_act's quantizer into a8[o] (A8 layout)
 * and sa[o] ([K/128][256]) -- byte for byte the two-step result. M must be 256. */
void r4dx_trellis_input_i8(int64_t x, int64_t M, int64_t K, int nout, const int64_t* suh, const int64_t* a8,
                           const int64_t* sa, int prescale_log2, int64_t stream);
/* kernels.h:167-175 r4dx_trellis_input_i8r: the same with one scale per row (sa[o] [256]), as
 * r4d_trellis_i8_quant_act_row; the row's f16 values wait in LDS (nout K 2 bytes, at most 160 KiB). */
void r4dx_trellis_input_i8r(int64_t x, int64_t M, int64_t K, int nout, const int64_t* suh, const int64_t* a8,
                            const int64_t* sa, int prescale_log2, int64_t stream);
/* No reference counterpart: the same quantizers for any M into a plain row-major a8 [M][K] (for callers
 * that keep int8 activations row-major); blk != 0: sa [K/128][M], else sa [M]. */
void r4d_i8_quant_act_plain(int64_t x, int64_t a8, int64_t sa, int M, int K, int blk, int64_t stream);
/* No reference counterpart as an entry: the reference has the dense form only as its bench kernel
 * (i8g_kernel<TRELLIS = false>, r4d_trellis_i8.h:19-21), with the same operand layouts. C f16 [256][N].
 * a8: A8 layout (r4d_trellis_i8_quant_act / _row); w8: W8 block layout (r4d_trellis_i8_layout.h:24-27,
 * r4d_i8_pack_w). scale_mode 0: sa [256], sw [N] (one int32 sum per slice, scaled once); 1: sa [K/128][256],
 * sw [N]; 2: sa [K/128][256], sw [K/128][N] (per 128-k block: acc += float(int32) * scale). SKG > 1 splits K
 * over the grid: ws r4d_gemm_i8_dense_ws_bytes(M, N, SKG) and tickets u32 [N/128], zero before the first call
 * and self-resetting (the protocol of r4d.h:482-486). */
void r4d_gemm_i8_dense(int64_t a8, int64_t sa, int64_t w8, int64_t sw, int64_t c, int64_t ws, int64_t tickets, int M,
                       int K, int N, int SKG, int scale_mode, int64_t stream);
/* Test entry: the exact int32 sums [256][N] of the same kernel and split. */
void r4d_gemm_i8_dense_raw(int64_t a8, int64_t w8, int64_t c, int64_t ws, int64_t tickets, int M, int K, int N,
                           int SKG, int64_t stream);
/* Plain int8 [N][K] -> the W8 block layout (r4d_trellis_i8_layout.h:56-64 W8Offset); N % 32 == 0, K % 16 == 0. */
void r4d_i8_pack_w(int64_t wp, int64_t w8, int N, int K, int64_t stream);
const char* r4d_gemm_i8_dense_check(int M, int K, int N, int SKG);
size_t r4d_gemm_i8_dense_ws_bytes(int M, int N, int SKG);
int r4d_mi355x_i8_skg(int K, int N);
/* No reference counterpart: the dense GEMM's SKG by scale mode (0 = stream-K for the per-128 modes). */
int r4d_mi355x_i8_dense_skg(int K, int N, int scale_mode);

/* ---- int8 x int8 trellis prefill GEMM (r4d.h:456-521) ---------------------------------------- */
/* r4d.h:490-492: the weight scale table SW [K/128][N] fp32 (s_eff = 1 / rs, rs = f16(min(1 / s, 60000)),
 * s = max|w| / 127 per (column, 128 k), 1 for an all-zero group) from the pair-grid words, and the int8
 * weights the GEMM quantizes on the fly (w8: W8 block layout; wp, if not 0: plain [N][K]). */
size_t r4d_trellis_i8_wscale_count(int K, int N);
void   r4d_trellis_i8_wscale(int64_t w, int64_t sw, int K, int N, int KB, int64_t stream);
void   r4d_trellis_i8_dump_w(int64_t w, int64_t sw, int64_t w8, int64_t wp, int K, int N, int KB, int64_t stream);
/* r4d.h:495-499: C bf16 [256][N] = bf16((FWHT128(sum_kb float(int32(A8 . W8)) * (sa sw)) * svh) * out_scale);
 * columns >= n_split read a8_1 / sa_1 (a8_1 = 0: a8_0, then n_split = N); ws fp32 ws_bytes(M, N, skg) when
 * skg > 1 (then a second launch adds the slices); tickets accepted and unused; skw checked, not used.
 * SW must be a table of r4d_trellis_i8_wscale (each entry the correctly rounded fp32 1 / rs of an f16 rs): the
 * kernel recovers rs from it with the hardware reciprocal, which returns that rs exactly for such entries only (an
 * arbitrary fp32 scale can round to a different rs than the reference's divide). */
void r4d_gemm_trellis_nt_i8(int64_t a8_0, int64_t sa_0, int64_t a8_1, int64_t sa_1, int n_split, int64_t w,
                            int64_t sw, int64_t svh, int64_t c, int64_t ws, int64_t tickets, int M, int K, int N,
                            int KB, int skw, int skg, float out_scale, int64_t stream);
const char* r4d_gemm_trellis_nt_i8_check(int M, int K, int N, int n_split, int KB, int skw, int skg);
size_t r4d_gemm_trellis_nt_i8_ws_bytes(int M, int N, int SKG);
/* r4d.h:514-521: the coarse sibling: SWC [N] (one scale per column over K), SA [256] (per row, from
 * r4d_trellis_i8_quant_act_row), the int32 sum of the slice scaled once by sa[row] * swc[col]. */
size_t r4d_trellis_i8_wscale_col_count(int K, int N);
void   r4d_trellis_i8_wscale_col(int64_t w, int64_t swc, int K, int N, int KB, int64_t stream);
void   r4d_trellis_i8_dump_w_col(int64_t w, int64_t swc, int64_t w8, int64_t wp, int K, int N, int KB, int64_t stream);
void r4d_gemm_trellis_nt_i8c(int64_t a8_0, int64_t sa_0, int64_t a8_1, int64_t sa_1, int n_split, int64_t w,
                             int64_t swc, int64_t svh, int64_t c, int64_t ws, int64_t tickets, int M, int K, int N,
                             int KB, int skw, int skg, float out_scale, int64_t stream);

/* ---- input transform and FWHT (src/kernels/include/r4dx/kernels/kernels.h) --------------------- */
/* kernels.h:110-128 r4dx_trellis_input_bf16: out[o][m,k] = f16(FWHT128(fp32(x) * suh[o])[k] * scale),
 * scale = float(2^prescale_log2 / sqrt(128)); x bf16 [M][K]; suh / out: HOST arrays of nout device
 * pointers. */
void r4dx_trellis_input_bf16(int64_t x, int64_t M, int64_t K, int nout, const int64_t* suh,
                             const int64_t* out, int prescale_log2, int64_t stream);
/* The same for an f16 x (fp16 activations); no reference counterpart, same contract. */
void r4dx_trellis_input_f16(int64_t x, int64_t M, int64_t K, int nout, const int64_t* suh,
                            const int64_t* out, int prescale_log2, int64_t stream);
/* No reference counterpart: r4d_gemm_trellis_nt_m64 over up to four input parts. Projections that read one input
 * (q | k | v, gdn qkv | z) stored as one linear -- their pair grids, svh and outputs concatenated along N -- run as
 * one launch; columns [n0[p], n0[p + 1]) read a[p] (the transform of the input under that projection's suh). a and
 * n0 are host arrays of `parts` (1..4) entries, n0[0] = 0, rising in multiples of 128 below N. Every column equals
 * the one-part launch of its projection at the same SKG, bit for bit. The _check form returns nullptr or the rule. */
const char* r4dx_gemm_trellis_nt_m64_parts_check(int parts, const int* n0, int M, int K, int N, int KB, int SKG,
                                                 int have_ws);
void r4dx_gemm_trellis_nt_m64_parts(const int64_t* a, const int* n0, int parts, int64_t w, int64_t svh, int64_t c,
                                    int64_t ws, int64_t tickets, int M, int K, int N, int KB, int SKG,
                                    float out_scale, int64_t stream);
/* No reference counterpart: the prefill form of the above, r4d_gemm_trellis_nt_m256 (M = 128 or 256) over up to four
 * input parts with the same a / n0 rule; every column equals the one-part M = 256 launch of its range at the same
 * SKG. */
const char* r4dx_gemm_trellis_nt_m256_parts_check(int parts, const int* n0, int M, int K, int N, int KB, int SKG);
void r4dx_gemm_trellis_nt_m256_parts(const int64_t* a, const int* n0, int parts, int64_t w, int64_t svh, int64_t c,
                                     int64_t ws, int64_t tickets, int M, int K, int N, int KB, int SKG,
                                     float out_scale, int64_t stream);
/* r4d.h:425-454 weight fake-quant, a measurement hook: r4d_gemm_trellis_nt_m64 / _raw / r4d_gemm_trellis_nt_m256
 * with every decoded weight w rounded, right before the MFMA, to f16(clamp(rint(w (1 / s)), -127, 127) s) (all but
 * the last rounding in fp32) under its column's scale s of a group of 2^gsh k-tiles. The table [K / 16 >> gsh][N]
 * (r4d_trellis_wscale_count floats) holds s = max|Q| / 127 per (group, column), 1 for an all-zero group, built by
 * r4d_trellis_wscale_f32 from the pair-grid words with the GEMM's own decode (N a multiple of 32, KB 4 or 5).
 * The _wq entries take the plain entry's arguments and legality plus the table (null throws) and gsh (1, 2 or 3,
 * 16 << gsh dividing K); KB 4 or 5. The M = 256 form equals the M = 64 form at SK = 1 and the same SKG, bit for bit. */
size_t r4d_trellis_wscale_count(int K, int N, int gsh);
void r4d_trellis_wscale_f32(int64_t w, int64_t scale, int K, int N, int KB, int gsh, int64_t stream);
void r4d_gemm_trellis_nt_m64_wq(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t svh, int64_t c, int64_t ws,
                                int64_t tickets, int M, int K, int N, int KB, int WV, int SK, int MT, int NP, int SKG,
                                int U, int NT, float out_scale, int64_t wscale, int gsh, int64_t stream);
void r4d_gemm_trellis_nt_m64_raw_wq(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t c, int64_t ws,
                                    int64_t tickets, int M, int K, int N, int KB, int WV, int SK, int MT, int NP,
                                    int SKG, int U, int NT, int64_t wscale, int gsh, int64_t stream);
void r4d_gemm_trellis_nt_m256_wq(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t svh, int64_t c,
                                 int64_t ws, int64_t tickets, int M, int K, int N, int KB, int SK, int NP,
                                 int SKG, int U, float out_scale, int64_t stream, int skw, int64_t wscale,
                                 int gsh);
/* kernels.h:130-147 the fused producers: r4dx_trellis_input_bf16 (nout = 1) over the bf16 value a producer kernel
 * would have stored -- r4dx_silu_mul_trellis_bf16: bf16(g * sigmoid(g) * u) over gate_up rows [gate | up] of row
 * stride in_row_stride (>= 2 intermediate), out f16 [rows][intermediate]; r4dx_attn_gate_mul_trellis_bf16:
 * bf16(attn_out * sigmoid(gate)) over [rows][K]. Byte-identical to the producer followed by the transform.
 * Throws unless K (intermediate) is a positive multiple of 128, rows is 0..65535 (0: nothing), |prescale_log2|
 * <= 24 and the pointers are non-null. sigmoid(x) = 1 / (1 + expf(-x)) in fp32 (the device library's expf). */
void r4dx_silu_mul_trellis_bf16(int64_t gate_up, int64_t rows, int64_t intermediate, int64_t in_row_stride,
                                int64_t suh, int64_t out, int prescale_log2, int64_t stream);
void r4dx_attn_gate_mul_trellis_bf16(int64_t attn_out, int64_t gate, int64_t rows, int64_t K, int64_t suh,
                                     int64_t out, int prescale_log2, int64_t stream);
/* kernels.h:149-165, 167-179: the two producers quantized like r4dx_trellis_input_i8 (per (row, 128) scales, sa
 * [K/128][256]) and _i8r (one scale per row, sa [256]): a8 in the A8 layout; rows must be 256. */
void r4dx_silu_mul_trellis_i8(int64_t gate_up, int64_t rows, int64_t intermediate, int64_t in_row_stride, int64_t suh,
                              int64_t a8, int64_t sa, int prescale_log2, int64_t stream);
void r4dx_attn_gate_mul_trellis_i8(int64_t attn_out, int64_t gate, int64_t rows, int64_t K, int64_t suh, int64_t a8,
                                   int64_t sa, int prescale_log2, int64_t stream);
void r4dx_silu_mul_trellis_i8r(int64_t gate_up, int64_t rows, int64_t intermediate, int64_t in_row_stride,
                               int64_t suh, int64_t a8, int64_t sa, int prescale_log2, int64_t stream);
void r4dx_attn_gate_mul_trellis_i8r(int64_t attn_out, int64_t gate, int64_t rows, int64_t K, int64_t suh, int64_t a8,
                                    int64_t sa, int prescale_log2, int64_t stream);
/* kernels.h:90-91 r4dx_silu_mul_wide_bf16: out bf16 [rows][intermediate] = bf16(g * sigmoid(g) * u) over gate_up
 * rows of stride in_row_stride (rows or intermediate <= 0: nothing) -- the MLP producer alone. */
void r4dx_silu_mul_wide_bf16(int64_t gate_up, int64_t out, int64_t rows, int64_t intermediate, int64_t in_row_stride,
                             int64_t stream);
/* src/model/attention/include/r4dx/model/attention/attn_kernels.h:26-31 r4dx_model_attn_gate_mul_bf16:
 * out[i] = bf16(attn_out[i] * sigmoid(gate[i])) over n elements (n <= 0: nothing) -- the attention producer. */
void r4dx_model_attn_gate_mul_bf16(int64_t attn_out, int64_t gate, int64_t out, int64_t n, int64_t stream);
/* kernels.h:192-197 r4dx_fwht128_f32: in-place unnormalised FWHT of each 128-float block (use_lds
 * accepted: both butterflies are the same fp32 operations in the same order). */
void r4dx_fwht128_f32(int64_t x, int64_t blocks, int use_lds, int64_t stream);

#ifdef __cplusplus
}
#endif
#endif
