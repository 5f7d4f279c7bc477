/*
 * ratchet_hip.h — C ABI of libratchet_hip.so, the gfx950 (MI355X) kernels of the
 * ratchet-linear hot path.
 *
 * Conventions shared by every entry point:
 *   - Plain pointers to device memory, element strides (not bytes), int64 sizes.
 *   - `stream` is a hipStream_t passed as void* (NULL = the legacy default stream).
 *     Work is enqueued on that stream; nothing synchronizes with the host.
 *   - The library never allocates and never frees: the caller owns every buffer (the one
 *     exception is the file-scope scratch array of rk_grad_weight_bf16_noalloc).
 *   - Return value: RK_OK (0) or an RK_ERR_* code; the message of the last failure
 *     on the calling thread is available from rk_last_error(). Nothing throws
 *     across the ABI.
 *   - dtype codes: RK_F32 = float32, RK_BF16 = bfloat16 (raw uint16 bits).
 *
 * Reference interfaces are cited as file:line in LoomNode/local-ai-training,
 * src/local_ai_training/.
 */
#ifndef RATCHET_HIP_H
#define RATCHET_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  RK_OK = 0,
  RK_ERR_ARG = 1,         /* invalid shape, stride, dtype, null pointer, alignment  */
  RK_ERR_LAUNCH = 2,      /* the HIP runtime reported an error at launch           */
  RK_ERR_UNSUPPORTED = 3  /* a valid request the library does not implement         */
};

enum {
  RK_F32 = 0,
  RK_BF16 = 1,
  RK_I8 = 2,          /* int8 activations with a per-row scale                          */
  RK_F32_AS_BF16 = 3  /* float32 storage whose values are taken as bfloat16(x) (round to
                         nearest even, as x.to(torch.bfloat16)): rk_quantize_rows[_devseed] */
};

/* Library version (major*10000 + minor*100 + patch). */
int rk_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* rk_last_error(void);

/*
 * Per-token absmax int8 quantization of a 2-D tensor, optionally pre-scaled per
 * column and optionally stochastically rounded.
 *   x        [M, K] of dtype x_dtype, element strides (sxm, sxk)
 *   col_scale[K] float32 or NULL
 *   q        [M, K] int8, row stride ldq (unit column stride)
 *   scale    [M]    float32
 *   x_dtype  RK_F32, RK_BF16, or RK_F32_AS_BF16 (float32 x quantized as bf16(x): the
 *            gradient a bf16 output receives from a float32 residual stream, without a
 *            separate cast)
 *   x_bf16   NULL, or [M, K] bf16 (row stride ld_xb) receiving bf16(x) (unscaled):
 *            the cast that the BF16 grad_weight GEMM consumes, produced in the
 *            same pass.
 *   stochastic = 0: q = clamp(rint(x'/s), ±127); = 1: q = clamp(floor(x'/s + u), ±127)
 *            with u = Philox4x32-10(counter = (uint32)(m*K + k), key = seed) mapped
 *            to [0, 1); m counts rows from row_offset.
 * Replaces: quantize_rows            int8_matmul.py:251-259
 *           quantize_rows_colscaled  int8_matmul.py:262-277
 *           _quantize_rows_fused / _quantize_rows_kernel  int8_matmul.py:106-150, 181-207
 */
int rk_quantize_rows(const void* x, int x_dtype, int64_t M, int64_t K, int64_t sxm,
                     int64_t sxk, const float* col_scale, int stochastic, uint64_t seed,
                     int64_t row_offset, int8_t* q, int64_t ldq, float* scale,
                     uint16_t* x_bf16, int64_t ld_xb, void* stream);

/*
 * rk_quantize_rows with stochastic = 1 and the seed read from device memory when the
 * kernel runs: seed points to one int64 on the device (the same value rk_quantize_rows
 * would take as `seed`). A HIP graph that captures this call draws whatever seed the
 * caller stored there before each replay, so replays of a captured training step take
 * fresh random bits while the host still draws one seed per call.
 * Replaces: quantize_rows_colscaled(..., stochastic=True)  int8_matmul.py:262-277 with its
 *           per-call seed draw int8_matmul.py:200.
 */
int rk_quantize_rows_devseed(const void* x, int x_dtype, int64_t M, int64_t K, int64_t sxm,
                             int64_t sxk, const float* col_scale, const int64_t* seed,
                             int64_t row_offset, int8_t* q, int64_t ldq, float* scale,
                             uint16_t* x_bf16, int64_t ld_xb, void* stream);

/*
 * rk_quantize_rows (unit column stride) over a row split by columns across nparts (1..3)
 * separate tensors: row m is x0[m, :] | x1[m, :] | x2[m, :], each [M, part_cols] with row
 * stride ldx, so K = nparts * part_cols (part_cols % 8 == 0). seed_dev, when not NULL, is
 * read at kernel time as in rk_quantize_rows_devseed (stochastic only). Same results as
 * concatenating the parts first.
 * Replaces: the gradient concatenation autograd performs for the attention's q, k, v chunks
 *           (model.py:106-110, qkv.chunk(3)) ahead of quantize_rows_colscaled
 *           (ratchet.py:130-132).
 */
int rk_quantize_rows_parts(const void* x0, const void* x1, const void* x2, int nparts,
                           int64_t part_cols, int x_dtype, int64_t M, int64_t ldx,
                           const float* col_scale, int stochastic, uint64_t seed,
                           const int64_t* seed_dev, int64_t row_offset, int8_t* q, int64_t ldq,
                           float* scale, void* stream);

/*
 * Random words of the stochastic rounding: out[i] = first output word of
 * Philox4x32-10 for counter ((counter0 + i) mod 2^32, 0, 0, 0) and key
 * (seed & 0xffffffff, seed >> 32), exactly the words rk_quantize_rows(stochastic=1)
 * draws for counters m*K + k.
 * Replaces: tl.randint(seed, offsets) behind tl.rand, int8_matmul.py:143-144.
 */
int rk_philox_word0(uint64_t seed, uint32_t counter0, int64_t n, uint32_t* out, void* stream);

/*
 * Scaled int8 GEMM, "NT" form: C[m, n] = out( (float(sum_k A[m,k] * B[n,k]) * ls[m]) * rs[n] )
 * with int32 accumulation. A int8 [M, K] (row stride lda, unit k stride); B int8
 * [N, K] (row stride ldb, unit k stride). rs may be NULL (= ones). The product is
 * rounded to bf16 (round-to-nearest-even); c_dtype RK_BF16 stores it as bf16,
 * RK_F32 stores the same bf16 value widened to float32 (the reference's
 * `.to(inputs.dtype)` cast, fused).
 * Replaces: scaled_int8_mm  int8_matmul.py:289-343 (kernel 26-79) for a B operand
 *           presented as the transposed view of an [N, K] matrix.
 */
int rk_int8_gemm_nt(const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb,
                    const float* ls, const float* rs, void* C, int c_dtype, int64_t ldc,
                    int64_t M, int64_t N, int64_t K, void* stream);

/*
 * Same GEMM with B taken from the packed ratchet state: packed [N, K] uint8
 * (row stride ldp), code = (byte & 15) - max_code decoded while staging tiles.
 * Replaces: _RatchetMatmul.forward int8 branches  ratchet.py:46-53, 63-65, which
 *           call scaled_int8_mm(q, code.t().contiguous(), s_x, scale) after
 *           unpacking (ratchet.py:443-445, 195-199).
 */
int rk_int8_gemm_packed(const int8_t* A, int64_t lda, const uint8_t* packed, int64_t ldp,
                        int max_code, const float* ls, const float* rs, void* C,
                        int c_dtype, int64_t ldc, int64_t M, int64_t N, int64_t K,
                        void* stream);

/*
 * rk_int8_gemm_packed with a float32 output and a residual added in the epilogue:
 * C[m, n] = R[m, n] + float(bf16_RNE((acc * ls[m]) * rs[n])), the same float32 add as
 * adding R to rk_int8_gemm_packed's float32 output afterwards. R (row stride ldr) may be
 * C itself (R == C and ldr == ldc); any other overlap of R and C is rejected with
 * RK_ERR_ARG. 32x32x32-kernel shapes only (M > 16, K % 64 == 0, N % 8 == 0, 16-byte aligned
 * rows); RK_ERR_UNSUPPORTED otherwise.
 * Replaces: the residual adds around the attention projection and the feed-forward
 *           contraction, model.py:181-195 (inputs = inputs + self.attention(...),
 *           inputs = inputs + self.feed_forward(...)), whose last linears run through
 *           _RatchetMatmul (ratchet.py:22-67).
 */
int rk_int8_gemm_packed_residual(const int8_t* A, int64_t lda, const uint8_t* packed,
                                 int64_t ldp, int max_code, const float* ls, const float* rs,
                                 const float* R, int64_t ldr, float* C, int64_t ldc, int64_t M,
                                 int64_t N, int64_t K, void* stream);

/*
 * The same GEMM with the packed state as the K x N operand, read in place:
 *   C[m, n] = bf16( (float(sum_k A[m,k] * code[k, n]) * ls[m]) * rs[n] ),
 *   code[k, n] = (packed[k, n] & 15) - max_code, packed [K, N] uint8 (row stride ldp).
 * The int8 grad_input GEMM (grad_int8 [M, N_out] @ code [N_out, K_in]) contracts over the
 * packed rows; this form stages packed tiles as they lie and transposes them in LDS, so
 * no decoded/transposed copy of the codes is made.
 * Replaces: scaled_int8_mm(grad_int8, code, ...)  ratchet.py:133-134 (with the unpack of
 *           ratchet.py:195-199 and the transposed copy rk_unpack_transpose would make).
 * Requires K % 64 == 0, N % 8 == 0, 16-byte aligned rows (RK_ERR_UNSUPPORTED otherwise).
 */
int rk_int8_gemm_packed_t(const int8_t* A, int64_t lda, const uint8_t* packed, int64_t ldp,
                          int max_code, const float* ls, const float* rs, void* C,
                          int c_dtype, int64_t ldc, int64_t M, int64_t N, int64_t K,
                          void* stream);

/*
 * Decode + transpose the packed state: codeT[k, n] = (packed[n, k] & 15) - max_code.
 *   packed [N, K] (row stride ldp) -> codeT int8 [K, N] (row stride ldt).
 * Feeds the int8 grad_input GEMM (contraction over the output features), replacing
 * the `code` operand of scaled_int8_mm(grad_int8, code, ...)  ratchet.py:133-134.
 */
int rk_unpack_transpose(const uint8_t* packed, int64_t ldp, int max_code, int8_t* codeT,
                        int64_t ldt, int64_t N, int64_t K, void* stream);

/*
 * Unpack the packed state into code / pressure int8 tensors (either may be NULL).
 * Replaces: unpack_code_pressure  ratchet.py:195-199 (the .code / .pressure properties
 * 443-449).
 */
int rk_unpack(const uint8_t* packed, int64_t n, int max_code, int8_t* code,
              int8_t* pressure, void* stream);

/*
 * BF16 grad_input against the packed state:
 *   out[m, k] = bf16( sum_n G[m, n] * E[n, k] ),  E[n, k] = bf16( bf16(code[n, k]) * bf16(scale[n]) )
 *   G bf16 [M, N] (row stride ldg), packed [N, K] uint8 (row stride ldp), scale [N] fp32,
 *   out [M, K] (row stride ldo) bf16, or fp32 holding the bf16 value (out_dtype RK_F32).
 * float32 accumulation. E is decoded once into `work` (rk_grad_input_bf16_workspace(N, K)
 * bytes, 16-byte aligned, contents overwritten) in MFMA operand order, then read by the
 * GEMM. Requires N a positive multiple of 8, K % 8 == 0 and 16-byte aligned rows
 * (RK_ERR_UNSUPPORTED otherwise).
 * Replaces: effective = code.to(bf16) * scale.to(bf16)[:, None]; grad_input =
 *           gradient_bf16 @ effective  ratchet.py:136-141 (the lm_head's backward, and every
 *           layer's with int8_backward off).
 */
int64_t rk_grad_input_bf16_workspace(int64_t N, int64_t K);
int rk_grad_input_bf16(const uint16_t* g, int64_t ldg, const uint8_t* packed, int64_t ldp,
                       int max_code, const float* scale, void* out, int out_dtype, int64_t ldo,
                       int64_t M, int64_t N, int64_t K, void* work, int64_t work_bytes,
                       void* stream);

/*
 * Effective BF16 weight: W[n, k] = bf16(code[n,k]) * bf16(scale[n]) rounded to bf16.
 * Replaces: effective = code.to(bf16) * scale.to(bf16)[:, None]  ratchet.py:140, 61.
 */
int rk_effective_bf16(const uint8_t* packed, int64_t ldp, int max_code, const float* scale,
                      uint16_t* W, int64_t ldw, int64_t N, int64_t K, void* stream);

/*
 * Dequantized BF16 activations: Xh[m, k] = bf16(q[m,k]) * bf16(s[m]) rounded to bf16.
 * Replaces: quantized_inputs.to(bf16) * input_scale[:, None].to(bf16)  ratchet.py:73-75.
 */
int rk_dequant_bf16(const int8_t* q, int64_t ldq, const float* s, uint16_t* Xh, int64_t ldx,
                    int64_t M, int64_t K, void* stream);

/*
 * Transposed bf16 copy: T[n, m] = bf16_RNE(X[m, n]); X [M, N] of dtype x_dtype (row
 * stride ldx), T [N, M] bf16 (row stride ldt). Lays the upstream gradient out as the
 * K-contiguous operand of the BF16 grad_weight GEMM (grad_out_tile.to(bf16) in
 * ratchet.py:162, transposed so the GEMM runs in its fast NT form).
 */
int rk_transpose_bf16(const void* x, int x_dtype, int64_t ldx, uint16_t* t, int64_t ldt,
                      int64_t M, int64_t N, void* stream);

/*
 * Dequantize + transpose: T[k, m] = bf16(q[m,k]) * bf16(scale[m]) rounded to bf16.
 * The dequantized activations of ratchet.py:73-75, laid out [K, M] for the NT
 * grad_weight GEMM.
 */
int rk_dequant_transpose_bf16(const int8_t* q, int64_t ldq, const float* scale, uint16_t* t,
                              int64_t ldt, int64_t M, int64_t K, void* stream);

/*
 * BF16 weight gradient from the saved int8 activations, without transposed copies:
 *   Gw[n, k] = bf16( sum_m bf16(g[m, n]) * bf16(bf16(q[m, k]) * bf16(s[m])) )
 *   g  [M, N] float32 or bfloat16 (row stride ldg), q [M, K] int8 (row stride ldq),
 *   s  [M] float32, out [N, K] bf16 (row stride ldo).
 * The token axis is split into nsplit ranges (rk_grad_weight_splits gives the default);
 * workspace is float32 [nsplit, N, K] (caller-allocated, fully overwritten). Partial
 * sums are added in split order, so the result is reproducible. With nsplit == 1 and out
 * given, the GEMM writes the bf16 gradient itself (the same values) and workspace may be
 * NULL (it is not touched). Requires N % 8 == 0,
 * K % 16 == 0 and 16-byte aligned rows (RK_ERR_UNSUPPORTED otherwise).
 * Replaces: grad_weight_tile = grad_out_tile.to(bf16) @ inputs_bf16 over the 256-row
 *           tiles of ratchet.py:148-163, with inputs_bf16 from ratchet.py:71-76.
 */
int rk_grad_weight_bf16(const void* g, int g_dtype, int64_t ldg, const int8_t* q, int64_t ldq,
                        const float* s, int64_t M, int64_t N, int64_t K, float* workspace,
                        int nsplit, uint16_t* out, int64_t ldo, void* stream);

/*
 * rk_grad_weight_bf16 / rk_grad_weight_bf16_x with the gradient's columns split across
 * nparts (1..3) separate tensors g0 | g1 | g2, each [M, part_cols] with row stride ldg
 * (N = nparts * part_cols; part_cols a multiple of the output tile: 128, or 256 where the
 * large tiles apply; RK_ERR_UNSUPPORTED otherwise). The activations x: x_dtype RK_I8 (int8
 * with the per-row scale s) or RK_BF16 / RK_F32 (s unused). Same results as concatenating
 * the parts first.
 * Replaces: the qkv gradient concatenation (model.py:106-110) ahead of the BF16 grad_weight
 *           GEMM (ratchet.py:148-163).
 */
int rk_grad_weight_bf16_parts(const void* g0, const void* g1, const void* g2, int nparts,
                              int64_t part_cols, int g_dtype, int64_t ldg, const void* x,
                              int x_dtype, int64_t ldx, const float* s, int64_t M, int64_t N,
                              int64_t K, float* workspace, int nsplit, uint16_t* out,
                              int64_t ldo, void* stream);

/*
 * The same BF16 weight gradient with the activation operand given directly:
 *   Gw[n, k] = bf16( sum_m bf16(g[m, n]) * bf16(x[m, k]) )
 *   x  [M, K] float32 or bfloat16 (x_dtype, row stride ldx); other arguments and
 *   requirements as rk_grad_weight_bf16.
 * Replaces: grad_out_tile.to(bf16) @ flat_inputs.to(bf16)  ratchet.py:159-163 (and the
 *           non-fused bf16 grad_weight, ratchet.py:95-106), with x the dequantized
 *           activations (rk_dequant_bf16) or the layer inputs.
 */
int rk_grad_weight_bf16_x(const void* g, int g_dtype, int64_t ldg, const void* x, int x_dtype,
                          int64_t ldx, int64_t M, int64_t N, int64_t K, float* workspace,
                          int nsplit, uint16_t* out, int64_t ldo, void* stream);

/*
 * rk_grad_weight_bf16 without a workspace (no counterpart in the reference): for callers
 * that cannot allocate (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc). The nsplit float32 split partials live in a file-scope device array of
 * 16 Mi floats (64 MB) per GPU, held until the process ends; nsplit * N * K beyond that
 * returns RK_ERR_ARG. out is required. Same kernels and split order as rk_grad_weight_bf16,
 * so the same nsplit gives the same bits. Calls that overlap on one GPU share the array
 * and race. Allocates nothing (no hipMalloc / hipFree, no allocating library call).
 */
int rk_grad_weight_bf16_noalloc(const void* g, int g_dtype, int64_t ldg, const int8_t* q,
                                int64_t ldq, const float* s, int64_t M, int64_t N, int64_t K,
                                int nsplit, uint16_t* out, int64_t ldo, void* stream);

/*
 * grad_weight with the fused update in its last blocks: the partial sums of
 * rk_grad_weight_bf16 (x_dtype RK_I8: int8 x with per-row scale s, as rk_grad_weight_bf16;
 * RK_F32 / RK_BF16: as rk_grad_weight_bf16_x) go to workspace [nsplit, N, K]; each block
 * then counts its arrival for its row block, and the block that completes a row block runs
 * the update of rk_ratchet_update_partials on those rows (same arithmetic, same results:
 * packed, counts, row_rms, rms_ema, nonfinite, grad_out), so no separate update launch
 * follows. counters: int32 [rk_grad_weight_update_counters(N, K)], zero before the first
 * call; every call leaves them zero again (a call that fails part-way does not: zero them
 * before the next). rms_mean (needs row_rms) is written by the block that completes the
 * layer. Requires K % 8 == 0 plus rk_grad_weight_bf16's conditions. No trainable-scale
 * gradient (use rk_grad_weight_bf16 + rk_ratchet_update_partials for that).
 * Replaces: the grad_weight tile loop and its gradient_sink ratchet.py:148-169, with
 *           _capture_weight_gradient 487-537 run on each finished row block.
 */
int rk_grad_weight_update(const void* g, int g_dtype, int64_t ldg, const void* x, int x_dtype,
                          int64_t ldx, const float* s, int64_t M, int64_t N, int64_t K,
                          float* workspace, int nsplit, int32_t* counters, uint8_t* packed,
                          int64_t ldp, int max_code, int threshold, float low, float high,
                          float eps, float* rms_ema, float beta1, float beta2, int64_t* counts,
                          float* row_rms, int32_t* nonfinite, float* rms_mean,
                          uint16_t* grad_out, int64_t ld_grad_out, void* stream);

/* Length of the counters array rk_grad_weight_update needs for an [N, K] gradient. */
int64_t rk_grad_weight_update_counters(int64_t N, int64_t K);

/* Default token-range split count of rk_grad_weight_bf16 for an [M] x [N, K] problem. */
int rk_grad_weight_splits(int64_t M, int64_t N, int64_t K);

/*
 * Fused integer ratchet update on a normalized gradient z (float32 [rows, K], row
 * stride ldz). packed [rows, K] (row stride ldp) is updated in place. counts[4]
 * (int64) are INCREMENTED by (positive moves, negative moves, blocked positive,
 * blocked negative); the caller zeroes them when it wants fresh sums.
 * Replaces: _ratchet_update_core  ratchet.py:265-301 (+ bucket_pressure 248-262,
 *           pack/unpack 185-199), as driven by apply_normalized_gradient 582-611.
 */
int rk_ratchet_update(uint8_t* packed, int64_t ldp, const float* z, int64_t ldz,
                      int64_t rows, int64_t K, int max_code, int threshold, float low,
                      float high, int64_t* counts, void* stream);

/*
 * Fused normalize + update from a raw weight gradient g ([rows, K], dtype g_dtype,
 * row stride ldg), one wavefront per row:
 *   ms = sum_k g^2 / K (fixed lane order), rms = sqrt(ms) or sqrt(EMA),
 *   z = g / (rms + eps), then the integer update above.
 * Optional outputs (NULL to skip):
 *   rms_ema  [rows] float32, read and written (per-row EMA of ms; beta1 = beta,
 *            beta2 = 1 - beta as float32; rows with ms == 0 keep their value)
 *   row_rms  [rows] float32 <- sqrt(ms) (the instantaneous rms the stats sum)
 *   grad_scale [rows] float32 <- sum_k g * code (pre-update code; trainable scale)
 *   nonfinite int32 flag, set to 1 when a row holds a NaN/Inf; such rows are left
 *            unchanged and do not contribute to counts.
 *   rms_mean float32 <- mean of row_rms over the rows (the stats' gradient_rms_mean),
 *            summed in a fixed order by a one-block kernel after the update; needs
 *            row_rms.
 * Replaces: _capture_weight_gradient  ratchet.py:487-537 (isfinite guard 501, stats
 *           525-537), _normalize 539-556, apply_weight_gradient 558-580, and the
 *           trainable-scale reduction ratchet.py:143-147, 167-169.
 */
int rk_ratchet_update_grad(uint8_t* packed, int64_t ldp, const void* g, int g_dtype,
                           int64_t ldg, int64_t rows, int64_t K, int max_code, int threshold,
                           float low, float high, float eps, float* rms_ema, float beta1,
                           float beta2, int64_t* counts, float* row_rms, float* grad_scale,
                           int32_t* nonfinite, float* rms_mean, void* stream);

/*
 * The same fused normalize + update, fed by the grad_weight GEMM's split partials instead
 * of a materialized gradient: partials float32 [nsplit, rows, K] (as left in the
 * workspace by rk_grad_weight_bf16 / rk_grad_weight_bf16_x called with out = NULL) are
 * added in split order and rounded to bf16 exactly as those entry points' reduction does,
 * and the resulting rows go through rk_ratchet_update_grad's arithmetic with a bf16
 * gradient. State, counts, row_rms, grad_scale, nonfinite and rms_mean are therefore
 * bit-identical to reducing first and updating after, while the bf16 gradient never
 * reaches memory (unless grad_out, bf16 [rows, K] with row stride ld_grad_out, asks
 * for a copy). K % 8 == 0 and 16-byte aligned partials (RK_ERR_UNSUPPORTED otherwise).
 * Replaces: the hand-off of each grad_weight tile (ratchet.py:162-165, gradient_sink) to
 *           the fused update of _capture_weight_gradient (ratchet.py:487-537).
 */
int rk_ratchet_update_partials(uint8_t* packed, int64_t ldp, const float* partials,
                               int nsplit, int64_t rows, int64_t K, int max_code,
                               int threshold, float low, float high, float eps,
                               float* rms_ema, float beta1, float beta2, int64_t* counts,
                               float* row_rms, float* grad_scale, int32_t* nonfinite,
                               float* rms_mean, uint16_t* grad_out, int64_t ld_grad_out,
                               void* stream);

/*
 * One layer of rk_ratchet_update_multi. Device addresses are 64-bit integers (0 = absent
 * for the optional outputs rms_ema, counts, row_rms, grad_scale, nonfinite). g is the
 * layer's gradient [rows, K] (row stride ldg, dtype given by the call's src) or, for
 * src == RK_UPDATE_SRC_SPLITS, its float32 split partials [nsplit, rows, K] (split stride
 * rows * K). row_begin is the layer's first row in the call's concatenated row space:
 * layer i starts where layer i - 1 ends (row_begin[0] == 0). 160 bytes, 8-byte aligned.
 */
typedef struct rk_update_layer {
  uint64_t packed, g, counts, row_rms, rms_ema, grad_scale, nonfinite, reserved0;
  int64_t ldp, ldg, rows, K, row_begin, reserved1;
  int32_t max_code, threshold, nsplit, reserved2;
  float low, high, eps, beta1, beta2, reserved3[3];
} rk_update_layer;

enum { RK_UPDATE_SRC_SPLITS = 2 };

/*
 * The fused normalize + update of rk_ratchet_update_grad (src RK_F32 / RK_BF16) or
 * rk_ratchet_update_partials (src RK_UPDATE_SRC_SPLITS) for several layers in one launch:
 * every layer's state, counts, row_rms, rms_ema, grad_scale and nonfinite are bit-identical
 * to what that layer's own call gives (the same row code; counts add into the layer's
 * counts). table_host and table_dev hold the same nlayers entries, in host and device
 * memory: the host copy is validated and sizes the launch, the kernel reads the device
 * copy (which must stay unchanged until the launch has run; under graph capture, for as
 * long as the graph is replayed). Layers must not share packed state or outputs. The
 * rms means are not written (rk_row_rms_means takes them from row_rms).
 * Replaces: the per-layer fused update of the backward pass, _capture_weight_gradient
 *           ratchet.py:487-537 called from the tile loop 148-169, run for every layer of the
 *           model (model.py:252-273 collects its statistics) in one pass over their state.
 */
int rk_ratchet_update_multi(const rk_update_layer* table_host, const rk_update_layer* table_dev,
                            int nlayers, int src, void* stream);

/*
 * Means of segments of a row-rms buffer: means[s] = mean of row_rms[offsets[s] ..
 * offsets[s + 1]) for s < nseg (offsets: nseg + 1 device int64, non-decreasing; an empty
 * segment gives NaN), each summed in the order the update entry points use for their
 * rms_mean, so a layer's mean here equals the one its update launch would have written.
 * One launch for every layer of a model whose updates wrote their row rms into one buffer
 * with rms_mean = NULL.
 * Replaces: the per-layer mean of the row rms, ratchet.py:570 / 637 (gradient_rms_mean),
 *           averaged over layers in model.py:265-267.
 */
int rk_row_rms_means(const float* row_rms, int64_t n, const int64_t* offsets, int64_t nseg,
                     float* means, void* stream);

/*
 * Row normalization alone: z = g / (rms + eps) with rms = sqrt(sum_k g^2 / K) in the
 * same fixed order as rk_ratchet_update_grad (or sqrt of the per-row EMA, which is
 * updated in place when rms_ema is non-NULL). z float32 [rows, K] (row stride ldz);
 * row_rms (may be NULL) receives the instantaneous rms.
 * Replaces: DiscreteRatchetLinear._normalize  ratchet.py:539-556.
 */
int rk_normalize_rows(const void* g, int g_dtype, int64_t ldg, int64_t rows, int64_t K,
                      float eps, float* rms_ema, float beta1, float beta2, float* z,
                      int64_t ldz, float* row_rms, void* stream);

/*
 * Pressure leak: every nonzero pressure moves one unit toward zero.
 * Replaces: _maybe_leak_pressure  ratchet.py:613-625 (the firing cadence stays in
 * the host).
 */
int rk_pressure_leak(uint8_t* packed, int64_t n, int max_code, void* stream);

/*
 * State validation: flags[0] |= 1 if a code escapes [-max_code, max_code],
 * flags[1] |= 1 if a pressure escapes [-7, 7], flags[2] |= 1 if a scale is not
 * finite or <= 0 (scale may be NULL). flags is int32[3], caller-zeroed.
 * Replaces: _validate_state  ratchet.py:672-679 (three host reductions).
 */
int rk_validate_state(const uint8_t* packed, int64_t n, int max_code, const float* scale,
                      int64_t n_rows, int32_t* flags, void* stream);

/*
 * Fused RMSNorm + per-token absmax quantization:
 *   y = x * rsqrt(mean_k x^2 + eps) * w;  (q, s) = quantize_rows(y).
 * x [M, K] (dtype x_dtype, row stride ldx, unit k stride), w [K] float32.
 * Replaces: fused_rmsnorm_quantize  int8_fused.py:14-56.
 */
int rk_rmsnorm_quantize(const void* x, int x_dtype, int64_t ldx, const float* w, float eps,
                        int8_t* q, int64_t ldq, float* scale, int64_t M, int64_t K,
                        void* stream);

/*
 * Fused tanh-GELU + per-token absmax quantization:
 *   y = 0.5 x (1 + tanh(0.7978845608 (x + 0.044715 x^3)));  (q, s) = quantize_rows(y).
 * Replaces: fused_gelu_quantize  int8_fused.py:58-101.
 */
int rk_gelu_quantize(const void* x, int x_dtype, int64_t ldx, int8_t* q, int64_t ldq,
                     float* scale, int64_t M, int64_t K, void* stream);

/*
 * Fused head-merge transpose + quantization: x [B, H, S, D] (element strides
 * sb, sh, ss, sd) is read as rows [B*S, H*D] (row = b*S + s, col = h*D + d) and
 * row-quantized.
 * Replaces: fused_transpose_quantize  int8_fused.py:103-151.
 */
int rk_transpose_quantize(const void* x, int x_dtype, int64_t B, int64_t H, int64_t S,
                          int64_t D, int64_t sb, int64_t sh, int64_t ss, int64_t sd,
                          int8_t* q, int64_t ldq, float* scale, void* stream);

/*
 * Backward of the RMSNorm prologue, per row of x [M, K] and grad_y [M, K]:
 *   rsqrt = 1 / sqrt(sum(x^2) / K + eps);  dvar = sum(grad_y * w * x) * -0.5 * rsqrt^3
 *   grad_x = bf16(grad_y * w * rsqrt + dvar * 2 * x / K)   (stored in x_dtype)
 *   grad_w[k] = sum over rows of grad_y * x * rsqrt         (float32)
 * grad_w is summed in a fixed order (per-block partials in `workspace`, then a
 * reduction in block order), so it is identical run to run. `workspace` holds at
 * least rk_rmsnorm_backward_parts(M) * K floats. K <= 4096 (RK_ERR_UNSUPPORTED
 * otherwise); grad_x has row stride ldgx and the dtype of x.
 * Replaces: rmsnorm_backward  int8_backward.py:7-51.
 */
int rk_rmsnorm_backward(const void* grad_y, int gy_dtype, int64_t ldg, const void* x,
                        int x_dtype, int64_t ldx, const float* w, float eps, int64_t M,
                        int64_t K, void* grad_x, int64_t ldgx, float* grad_w, float* workspace,
                        int64_t workspace_floats, void* stream);

/*
 * rk_rmsnorm_backward for a float32 x whose rows also feed the residual stream:
 *   grad_x = float32(bf16(dx)) + residual_grad
 * (one float32 add per element, the add autograd performs where x has both uses), with
 * residual_grad [M, K] float32, row stride ldr. residual_grad may be grad_x itself (same
 * row stride); any other overlap is rejected. grad_w as rk_rmsnorm_backward.
 * Replaces: rmsnorm_backward  int8_backward.py:7-51 plus the residual add of the block,
 *           model.py:181-195 (inputs = inputs + self.attention(self.attention_norm(inputs))).
 */
int rk_rmsnorm_backward_residual(const void* grad_y, int gy_dtype, int64_t ldg, const float* x,
                                 int64_t ldx, const float* w, float eps, int64_t M, int64_t K,
                                 const float* residual_grad, int64_t ldr, float* grad_x,
                                 int64_t ldgx, float* grad_w, float* workspace,
                                 int64_t workspace_floats, void* stream);

/* Number of grad_w partial rows rk_rmsnorm_backward uses for M rows (0 for M <= 0, at most 1024). */
int rk_rmsnorm_backward_parts(int64_t M);

/*
 * Backward of the tanh-GELU prologue, elementwise over x [M, K]:
 *   t = tanh(0.7978845608 (x + 0.044715 x^3))
 *   grad_x = bf16(grad_y * (0.5 (1 + t) + 0.5 x (1 - t^2) 0.7978845608 (1 + 0.134145 x^2)))
 * stored in x_dtype with row stride ldgx.
 * Replaces: gelu_backward  int8_backward.py:53-89.
 */
int rk_gelu_backward(const void* grad_y, int gy_dtype, int64_t ldg, const void* x, int x_dtype,
                     int64_t ldx, int64_t M, int64_t K, void* grad_x, int64_t ldgx,
                     void* stream);

/* Token-embedding weight gradient: out[v, :] = sum of grad[t, :] over the T tokens with
 * ids[t] == v (float32 [V, D], every row written; ids outside [0, V) contribute nothing).
 * grad [T, D] float32 / bfloat16 with row stride ldg; ids int64 (ids_int64 = 1) or int32.
 * The sum order is fixed: tokens in chunks of 64 positions, token order within a chunk,
 * chunk order across chunks; no memset, no device-wide sort (legal under HIP-graph
 * capture). work holds rk_embedding_backward_workspace(T, V, D) bytes, 16-byte aligned
 * (per-chunk partial rows and a V x chunks byte table the call clears itself); nothing
 * needs clearing between calls.
 * D % 4 != 0 or D > 4096: RK_ERR_UNSUPPORTED.
 * Replaces: the backward of the model's token lookup, model.py:237 (an nn.Embedding,
 *           model.py:219, whose torch backward sorts the ids on the device).
 */
int64_t rk_embedding_backward_workspace(int64_t T, int64_t V, int64_t D);
int rk_embedding_backward(const void* grad, int grad_dtype, int64_t ldg, const void* ids,
                          int ids_int64, int64_t T, int64_t V, int64_t D, float* out,
                          int64_t ldo, void* work, int64_t work_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * KV-cached decode (one token per sequence, M <= 16 rows). The reference has no
 * incremental path: generate.py:183-201 runs the whole window through the model for
 * every token and reads the last position. These entry points compute that last
 * position's step against a key/value cache instead; a transformer layer is six
 * launches (qkv GEMV, attention partial + combine, proj / expand / contract GEMVs).
 * ------------------------------------------------------------------------- */
enum { RK_DEC_PRO_INT8 = 0, RK_DEC_PRO_PLAIN = 1, RK_DEC_PRO_RMSNORM = 2 };
enum { RK_DEC_EPI_STORE = 0, RK_DEC_EPI_GELU = 1, RK_DEC_EPI_ADD = 2 };

/* y = epilogue(bf16((q @ code^T) * s[m] * row_scale[n])) for M <= 16 token rows,
 * code = (packed & 15) - max_code, packed [N, K] (ldp).
 * Prologue, giving the int8 rows q and their scales s:
 *   RK_DEC_PRO_INT8     q = xq [M, K] (ldxq), s = xs [M] as given;
 *   RK_DEC_PRO_PLAIN    per-token absmax quantization of the float32 rows x [M, K]
 *                       (ldx): the arithmetic of rk_quantize_rows (round to nearest);
 *   RK_DEC_PRO_RMSNORM  x * rsqrt(mean(x^2) + eps) * norm_w, then quantized: the
 *                       arithmetic of rk_rmsnorm_quantize (same summation order).
 * Epilogue: RK_DEC_EPI_STORE writes the bf16 value (y_dtype RK_BF16) or it widened
 * (RK_F32); RK_DEC_EPI_GELU writes tanh-GELU of the widened value (float32, the input
 * of rk_gelu_quantize in int8_fused.py:58-84); RK_DEC_EPI_ADD adds it to the float32
 * rows y in place (the residual `hidden + out`). With the same q and s the int32 sums
 * and outputs equal rk_int8_gemm_packed's. Requires N % 16 == 0, K % 64 == 0,
 * K <= 6144, 16-byte aligned rows (RK_ERR_UNSUPPORTED otherwise). */
int rk_decode_gemv(const float* x, int64_t ldx, const int8_t* xq, int64_t ldxq,
                   const float* xs, int prologue, const float* norm_w, float eps,
                   const uint8_t* packed, int64_t ldp, int max_code, const float* row_scale,
                   void* y, int y_dtype, int64_t ldy, int epilogue, int64_t M, int64_t N,
                   int64_t K, void* stream);

/* Number of position splits rk_decode_attention uses for B sequences of H heads with
 * a cache of max_len positions (its workspace holds B * H * splits * (D + 4) floats). */
int64_t rk_decode_attention_splits(int64_t B, int64_t H, int64_t max_len);

/* One decode step of causal attention at position p = *pos (a device int64, so the
 * step can be captured once and replayed). qkv [B, 3*H*D] (ld_qkv; q | k | v, head h at
 * h*D) holds the step's projections; k_cache / v_cache are [B, H, max_len, D] with
 * element strides sb, sh, sl (d contiguous). The step's k and v are written to
 * position p, then softmax(q . k_j * scale) over j = 0..p weights v_j (float32
 * arithmetic, positions split across workgroups and merged with the log-sum-exp
 * rule). out [B, H*D] (ldo) receives the float32 rows, heads concatenated as the
 * reference's transpose + view (model.py:128-130). Head size 64, 128 or 256. A
 * position outside [0, max_len) writes nothing to the cache and NaN rows. */
int rk_decode_attention(const void* qkv, int qkv_dtype, int64_t ld_qkv, void* k_cache,
                        void* v_cache, int cache_dtype, int64_t sb, int64_t sh, int64_t sl,
                        const int64_t* pos, int64_t B, int64_t H, int64_t D, int64_t max_len,
                        float scale, float* work, int64_t work_floats, float* out,
                        int64_t ldo, void* stream);

/* hidden[b] = table[tokens[b]] + pos_table[*pos] (float32; model.py:237 at one
 * position). An id outside [0, vocab) or a position outside [0, n_pos) gives a NaN row. */
int rk_decode_embed(const int64_t* tokens, int64_t B, const float* table, int64_t vocab,
                    int64_t C, const float* pos_table, int64_t n_pos, const int64_t* pos,
                    float* hidden, int64_t ldh, void* stream);

/* Greedy pick and cache advance of one decode step, in one launch: tokens[b * ld_tokens]
 * (int64) = the argmax of logits row b (float32 [B, V], row stride ldl): the first index
 * of the largest value, a NaN ranking above every number, as torch.argmax; then, when pos
 * is not null, *pos += 1. Replaces: torch.argmax(next_logits, dim=-1) at temperature 0
 * (generate.py:188-189) and the window's growth by the picked token (generate.py:200). */
int rk_decode_greedy(const float* logits, int64_t ldl, int64_t B, int64_t V, int64_t* tokens,
                     int64_t ld_tokens, int64_t* pos, void* stream);

/*
 * Token cross-entropy, mean over the rows whose target is not ignore_index: per row of
 * logits [M, V] (float32 / bfloat16, row stride ldl, 16-byte aligned rows, V a multiple of
 * 4 / 8), m = max x, logsum = log(sum exp(x - m)), loss_row = -((x_t - m) - logsum);
 * *loss = (sum of loss_row in a fixed order) / count, *count = the number of rows counted
 * (float; 0 gives NaN). A target outside [0, V) other than ignore_index gives a NaN loss.
 * stats [3, M] float32 receives (m, logsum, loss_row) for rk_cross_entropy_backward.
 * targets int64 [M]. Shapes outside the aligned form: RK_ERR_UNSUPPORTED.
 * Replaces: F.cross_entropy(logits.flatten(0, 1), targets.flatten()), model.py:249
 *           (log_softmax + nll_loss forward).
 */
int rk_cross_entropy_forward(const void* logits, int dtype, int64_t ldl, const int64_t* targets,
                             int64_t M, int64_t V, int64_t ignore_index, float* stats,
                             float* loss, float* count, void* stream);

/*
 * Its backward: with g_t = -(*grad_loss / *count) for a counted row (0 for an ignored one),
 * grad[j] = [j == t] g_t - exp((x_j - m) - logsum) * g_t, stored as grad_dtype (float32 or
 * bfloat16, 16-byte aligned rows: ldg a multiple of 16 bytes); grad_loss and count are
 * device scalars (count from the forward). Nothing else is written.
 * Replaces: the backward of model.py:249 (nll_loss and log_softmax backward).
 */
int rk_cross_entropy_backward(const void* logits, int dtype, int64_t ldl, const int64_t* targets,
                              int64_t M, int64_t V, int64_t ignore_index, const float* stats,
                              const float* count, const float* grad_loss, void* grad,
                              int grad_dtype, int64_t ldg, void* stream);

/*
 * Causal self-attention forward (flash form): for bf16 q, k, v [B, H, S, D] with element
 * strides (batch, head, position; the feature stride is 1), D = 64 or 128,
 *   o[b, h, i, :] = sum_{j <= i} softmax_j(s_ij) v[b, h, j, :],  s_ij = (q_i . k_j) * scale,
 *   lse[b, h, i] = log(sum_{j <= i} exp(s_ij))  (float32 [B, H, S], contiguous),
 * o bf16 with its own strides (8-byte aligned rows). The scores and the softmax run in float32;
 * the probabilities enter the value product rounded to bf16. q, k, v 16-byte aligned, strides
 * multiples of 8 elements, one head's positions under 2^30 bytes; otherwise
 * RK_ERR_UNSUPPORTED. (o, lse) is the pair torch's memory-efficient attention backward takes.
 * Replaces: the forward of F.scaled_dot_product_attention(q, k, v, is_causal=True),
 *           model.py:117-123.
 */
int rk_attention_forward(const uint16_t* q, int64_t sqb, int64_t sqh, int64_t sqs,
                         const uint16_t* k, int64_t skb, int64_t skh, int64_t sks,
                         const uint16_t* v, int64_t svb, int64_t svh, int64_t svs, int64_t B,
                         int64_t H, int64_t S, int64_t D, float scale, uint16_t* o, int64_t sob,
                         int64_t soh, int64_t sos, float* lse, void* stream);

/* HBM streaming probe (measurement only; no counterpart in the reference): reads `bytes`
 * (a multiple of 16) from src in 16-byte vectors, `unroll` (1, 2, 4, 8) loads in flight
 * per thread, `blocks` blocks of 256 threads in a grid-stride loop; copy != 0 writes them
 * to dst, else nothing is written (dst must still hold blocks * 1 KB). The achieved rate is
 * the device's practical read / copy bandwidth for the bandwidth-bound kernels. */
int rk_hbm_stream(const void* src, void* dst, int64_t bytes, int copy, int unroll, int blocks,
                  void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RATCHET_HIP_H */
