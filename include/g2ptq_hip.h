/*
 * g2ptq_hip.h — C ABI of libg2ptq_hip.so, the MI355X (gfx950) implementation of
 * the GPTQ / GPTAQ / G2PTQ per-layer quantization path.
 *
 * Conventions
 *   - Every pointer argument is a device pointer owned by the caller unless the
 *     comment says "host".  `stream` is a hipStream_t passed as void*.
 *   - Calls are asynchronous on `stream` and allocate nothing; scratch memory
 *     comes in through `ws` / `ws_bytes` (size it with the *_workspace query).
 *   - Return value: 0 on success, < 0 on an argument / runtime error (see
 *     g2ptq_status_string and g2ptq_last_error), never an exception.
 *   - Numeric failures are reported through device-side `info` / `flags`
 *     integers that the caller reads at its own synchronisation point.
 *   - Matrices are row-major; "ld" is the leading dimension in elements.
 *     bf16 data is passed as uint16_t bit patterns.
 *
 * Paths in comments are relative to the reference repository (G2PTQ/G2PTQ).
 */
#ifndef G2PTQ_HIP_H
#define G2PTQ_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define G2PTQ_OK 0
#define G2PTQ_ERR_ARG (-1)
#define G2PTQ_ERR_HIP (-2)
#define G2PTQ_ERR_WORKSPACE (-3)
#define G2PTQ_ERR_UNSUPPORTED (-4)

/* Device-side flag bits (OR-ed into an int32 the caller owns). */
#define G2PTQ_FLAG_BAD_SCALE 1   /* a scale was <= 0 or NaN (quant_utils.py:432 assert) */
#define G2PTQ_FLAG_NAN_OUTPUT 2  /* NaN in quantized weights (gptq_utils.py:346-350) */
#define G2PTQ_FLAG_GROUP_SCALE 4 /* scales differ within a group (compressed_tensors_utils.py:35 assert) */

/* Compensation variants. */
#define G2PTQ_VARIANT_GPTQ 0
#define G2PTQ_VARIANT_GPTAQ 1
#define G2PTQ_VARIANT_G2PTQ 2

int g2ptq_abi_version(void);
const char* g2ptq_status_string(int status);
/* Detail message of the last failing call on the calling host thread. */
const char* g2ptq_last_error(void);

/* ------------------------------------------------------------------------
 * Quantizer grid — utils/quant_utils.py
 * ---------------------------------------------------------------------- */

/* Per-row min/max → (scale, zero) of one quantization group per row.
 * Replaces WeightQuantizer.find_params (utils/quant_utils.py:377-433, with
 * _minmax/_params_from_range_* :47-68) for mse=False, hclip=False.
 * x: rows × cols, ld ldx.  Writes scale[r*ldp], zero[r*ldp]. */
int g2ptq_find_params(void* stream, const float* x, int64_t rows, int64_t cols, int64_t ldx,
                      int bits, int sym, float* scale, float* zero, int64_t ldp, int* flags);

/* MSE clip search of WeightQuantizer.find_params with mse=True
 * (utils/quant_utils.py:406-425): grid × maxshrink² candidate ranges per row,
 * error sum(|fq − x|^norm), first strict improvement wins.
 * hclip (quant_utils.py:393-397, _quant_err :84-105): hdiag (nullable) is the
 * H_diag the reference reshapes to (hblocks, groups_per_row, cols), pitch ldh:
 * the rows split into hblocks equal consecutive shares, share b's error being
 * sum((fq − x)² · hdiag[b, k·cols + c]) for column group k = r % groups_per_row
 * (groups_per_row > 1 when weight_groupsize split each original row).  When
 * every hdiag entry is equal the plain search runs, as in the reference. */
int g2ptq_find_params_mse(void* stream, const float* x, int64_t rows, int64_t cols, int64_t ldx,
                          int bits, int sym, float norm, int grid, float maxshrink,
                          const float* hdiag, int64_t ldh, int64_t hblocks,
                          int64_t groups_per_row, float* scale, float* zero, int64_t ldp,
                          int* flags);

/* Round-to-nearest fake quantization with per-row, per-group parameters.
 * Replaces WeightQuantizer.fake_quantize (utils/quant_utils.py:435-459) and
 * fake_quantize_grouped (gptq_utils/common_utils.py:33-44).
 * Column c of row r uses scale[r*ldp + c/groupsize] (groupsize <= 0: column 0).
 * q_out: dequantized values; int_out (nullable): integer codes as float. */
int g2ptq_fake_quantize(void* stream, const float* x, int64_t rows, int64_t cols, int64_t ldx,
                        int64_t groupsize, const float* scale, const float* zero, int64_t ldp,
                        int bits, float* q_out, int64_t ldq, float* int_out, int64_t ldi,
                        int* flags);

/* ------------------------------------------------------------------------
 * Hessian accumulation
 * ---------------------------------------------------------------------- */

/* Bytes of workspace needed by the *_update calls below for T tokens of C
 * features (kind: 0 Hessian, 1 GPTAQ, 2 saliency-weighted with G groups;
 * G is ignored for kinds 0 and 1). */
int g2ptq_hessian_workspace(int64_t T, int64_t C, int kind, int64_t G, size_t* bytes);

/* H = beta·H + alpha·XᵀX (H symmetric C×C fp32, both triangles written).
 * X: T × C bf16 (ld ldx).  Replaces GPTQ.add_batch's update
 * (gptq_utils/gptq_utils.py:123-126; alpha = 2/n_new, beta = n_old/n_new). */
int g2ptq_hessian_update(void* stream, const uint16_t* X, int64_t T, int64_t C, int64_t ldx,
                         float alpha, float beta, float* H, int64_t ldh, void* ws, size_t ws_bytes);

/* Staged accumulation: the two halves of g2ptq_hessian_update, so a caller
 * can gather several calibration batches (add_batch payloads) into one Gram
 * launch.  g2ptq_hessian_stage writes Xᵀ of a T × C batch into XT (rows =
 * g2ptq_hessian_stage_rows(C) ≥ C, zero padded; ld ldt) at token column
 * t_off (a multiple of 64), zero padding the batch to a multiple of 64
 * tokens.  XT must be 16-byte aligned and ldt a multiple of 8.
 * g2ptq_hessian_gram then applies H = beta·H + alpha·XTᵀ·XT over the first K
 * staged columns; it may zero-pad columns up to K rounded up to a multiple of
 * 2048, so ldt must leave that room.  Together they replace the per-batch
 * update of GPTQ.add_batch (gptq_utils/gptq_utils.py:123-126). */
int g2ptq_hessian_stage_rows(int64_t C, int64_t* rows);
int g2ptq_hessian_stage(void* stream, const uint16_t* X, int64_t T, int64_t C, int64_t ldx,
                        uint16_t* XT, int64_t ldt, int64_t t_off);
int g2ptq_hessian_gram_workspace(int64_t K, int64_t C, size_t* bytes);
int g2ptq_hessian_gram(void* stream, uint16_t* XT, int64_t ldt, int64_t K, int64_t C, float alpha,
                       float beta, float* H, int64_t ldh, void* ws, size_t ws_bytes);
/* Sets *equal = 0 where the first `cols` columns of `rows` rows of two staged
 * buffers (pitches lda, ldb) differ; the caller sets *equal = 1 before.  No
 * counterpart in the reference: the reference accumulates every linear's
 * Hessian separately, and the Python layer uses this check before giving a
 * linear the Gram another linear computed from tokens staged from the same
 * input addresses (q/k/v, gate/up hooks), so the copy is taken only when the
 * staged operands are bit-identical.  cols, lda and ldb multiples of 8. */
int g2ptq_staged_equal(void* stream, const uint16_t* A, int64_t lda, const uint16_t* B,
                       int64_t ldb, int64_t rows, int64_t cols, int* equal);

/* GPTAQ: H = beta·H + alpha·XᵀX and Dx = beta·Dx + alpha·(X_fp − X)ᵀX, with
 * Dx[i][j] = Σ_t (x_fp − x)[t,i]·x[t,j].  Replaces GPTAQ.add_batch
 * (gptq_utils/gptaq_utils.py:130-148). */
int g2ptq_gptaq_update(void* stream, const uint16_t* X, const uint16_t* Xfp, int64_t T, int64_t C,
                       int64_t ldx, int64_t ldxf, float alpha, float beta, float* H, float* Dx,
                       int64_t ld, void* ws, size_t ws_bytes);

/* Staged GPTAQ accumulation (the two halves of g2ptq_gptaq_update, as for
 * g2ptq_hessian_stage / _gram).  XT holds three contiguous planes of
 * rows × ldt bf16 (rows = g2ptq_hessian_stage_rows(C)): Xᵀ and the bf16 high
 * and low parts of (X_fp − X)ᵀ.  Same alignment and padding rules as
 * g2ptq_hessian_stage / _gram.  Replaces the per-batch update of
 * GPTAQ.add_batch (gptq_utils/gptaq_utils.py:130-148). */
int g2ptq_gptaq_stage(void* stream, const uint16_t* X, const uint16_t* Xfp, int64_t T, int64_t C,
                      int64_t ldx, int64_t ldxf, uint16_t* XT, int64_t ldt, int64_t t_off);
int g2ptq_gptaq_gram_workspace(int64_t K, int64_t C, size_t* bytes);
int g2ptq_gptaq_gram(void* stream, uint16_t* XT, int64_t ldt, int64_t K, int64_t C, float alpha,
                     float beta, float* H, float* Dx, int64_t ld, void* ws, size_t ws_bytes);

/* Saliency-weighted Hessians for G groups:
 *   H[g] = beta·H[g] + alpha·Σ_t S[t,g]·x_t x_tᵀ   (H: G × C × C, stride sH)
 *   act  = act_beta·act + act_alpha·Σ_t x_t²       (act: C, nullable)
 * Replaces G2PTQ.add_batch (gptq_utils/g2ptq_utils.py:182-201) and
 * GPTQGuided.add_batch (gptq_utils/gptq_guided_utils.py:59-81).
 * S: T × G fp32 (ld lds). */
int g2ptq_weighted_hessian_update(void* stream, const uint16_t* X, int64_t T, int64_t C,
                                  int64_t ldx, const float* S, int64_t G, int64_t lds,
                                  float alpha, float beta, float* H, int64_t ldh, int64_t sH,
                                  float* act, float act_alpha, float act_beta,
                                  void* ws, size_t ws_bytes);

/* Staged weighted accumulation.  XT holds Xᵀ (rows × ldt bf16, rows =
 * g2ptq_hessian_stage_rows(C)) followed by G rows of ldt fp32 token weights
 * w[g][t] = S[t,g]·s_scale (the memory of 2G more bf16 rows:
 * g2ptq_hessian_stage_height(2, 0, C, G, ·) rows of ldt bf16 in all); s_scale
 * folds a per-batch factor (G2PTQ's 1/T_b) into the staged tokens.
 * g2ptq_weighted_stage also applies the act update of
 * g2ptq_weighted_hessian_update for the batch.  g2ptq_weighted_gram applies
 * H[g] = beta·H[g] + alpha·Σ_t x_t·(x_t·w[g][t])ᵀ over the first K staged
 * columns, all G groups in one launch, and its workspace depends on G.  Same
 * alignment and padding rules as g2ptq_hessian_stage / _gram.  Replace the
 * per-batch updates of G2PTQ.add_batch (gptq_utils/g2ptq_utils.py:182-201)
 * and GPTQGuided.add_batch (gptq_utils/gptq_guided_utils.py:59-81). */
int g2ptq_weighted_stage(void* stream, const uint16_t* X, int64_t T, int64_t C, int64_t ldx,
                         const float* S, int64_t G, int64_t lds, float s_scale, uint16_t* XT,
                         int64_t ldt, int64_t t_off, float* act, float act_alpha, float act_beta);
int g2ptq_weighted_gram_workspace(int64_t K, int64_t C, int64_t G, size_t* bytes);
int g2ptq_weighted_gram(void* stream, uint16_t* XT, int64_t ldt, int64_t K, int64_t C, int64_t G,
                        float alpha, float beta, float* H, int64_t ldh, int64_t sH, void* ws,
                        size_t ws_bytes);

/* Staged accumulation of any of the three kinds (kind 0 Hessian, 1 GPTAQ,
 * 2 weighted) for activations of dtype code 0 (bf16), 1 (fp16) or 2 (fp32):
 * the reference takes any float input and accumulates in fp32
 * (inp.float(), gptq_utils/gptq_utils.py:125, gptaq_utils.py:139-146,
 * g2ptq_utils.py:193-201).  X (and Xfp) are T × C of that dtype.  Xᵀ is
 * staged as P bf16 planes that sum to it exactly (P = 1, 2, 3), followed by
 * the kind's planes as above (GPTAQ: hi, lo of X_fp − X; weighted with
 * P > 1: hi, lo of x·S[t,g]·s_scale per group; weighted bf16: the weight
 * rows of g2ptq_weighted_stage); g2ptq_hessian_stage_planes gives the count
 * of feature planes (rows × ldt each) and g2ptq_hessian_stage_height the
 * buffer's height in rows of ldt bf16 (planes × rows, plus the bf16
 * weighted kind's 2G).  g2ptq_hessian_gram_ex runs each product once per plane of Xᵀ as
 * its column operand (the plain Hessian's row operand is all P planes),
 * accumulating: the same H / Dx / H[g] updates as g2ptq_hessian_gram,
 * g2ptq_gptaq_gram and g2ptq_weighted_gram (whose bf16 paths these equal
 * bit for bit), at P times their work for GPTAQ's cross term and the
 * weighted kind and P² times for the plain Hessian.  Same alignment and
 * padding rules as g2ptq_hessian_stage / _gram; act (kind 2) as in
 * g2ptq_weighted_stage. */
int g2ptq_hessian_stage_planes(int kind, int dtype, int64_t G, int64_t* planes);
int g2ptq_hessian_stage_height(int kind, int dtype, int64_t C, int64_t G, int64_t* rows);
int g2ptq_hessian_stage_ex(void* stream, int kind, int dtype, const void* X, const void* Xfp,
                           int64_t T, int64_t C, int64_t ldx, int64_t ldxf, const float* S,
                           int64_t G, int64_t lds, float s_scale, uint16_t* XT, int64_t ldt,
                           int64_t t_off, float* act, float act_alpha, float act_beta);
int g2ptq_hessian_gram_ex_workspace(int kind, int dtype, int64_t K, int64_t C, int64_t G,
                                    size_t* bytes);
int g2ptq_hessian_gram_ex(void* stream, int kind, int dtype, uint16_t* XT, int64_t ldt, int64_t K,
                          int64_t C, int64_t G, float alpha, float beta, float* H, int64_t ldh,
                          int64_t sH, float* Dx, int64_t ldd, void* ws, size_t ws_bytes);

/* ------------------------------------------------------------------------
 * Hessian preparation and factor
 * ---------------------------------------------------------------------- */

/* In place on H (B × C × C) and W (B × R × C): an all-zero H[b] becomes the
 * identity, a zero diagonal entry d becomes 1 and column d of W[b] (and of
 * Dx[b], nullable) is zeroed; where H[b] was all zero, Grad[b] (B × Rg × C,
 * nullable) is zeroed.  Replaces gptq_utils/gptq_utils.py:272-277,
 * gptaq_utils.py:302-308, g2ptq_utils.py:394-401.  ws: at least
 * 256·⌈8B/256⌉ + 256·⌈4BC/256⌉ bytes. */
int g2ptq_prepare_hessian(void* stream, float* H, int64_t B, int64_t C, float* W, int64_t R,
                          float* Dx, float* Grad, int64_t Rg, void* ws, size_t ws_bytes);

int g2ptq_factor_workspace(int64_t B, int64_t C, size_t* bytes);

/* U[b] = upper Cholesky factor of (H[b] + p·mean(diag H[b])·I)⁻¹, i.e. the
 * factor the reference computes as
 *   chol(cholesky_inverse(chol(H + damp·I)), upper=True)
 * (gptq_utils/gptq_utils.py:295-302), computed here as J·chol(J·A·J)⁻¹·J.
 * Entries with skip[b] != 0 (nullable, device) are left untouched.
 * info[b] (device): 0 ok, k > 0 leading minor k not positive definite,
 * -1 NaN in the factor (the reference's retry triggers). */
int g2ptq_inv_chol_upper(void* stream, const float* H, int64_t B, int64_t C, float percdamp,
                         const int* skip, float* U, int* info, void* ws, size_t ws_bytes);

/* ------------------------------------------------------------------------
 * Compensation
 * ---------------------------------------------------------------------- */

/* One compensation block on the reference's transposed block layout
 * (B, bs, R): the run_eager operators of gptq_utils/gptq_utils.py:67-90
 * (variant 0), gptaq_utils.py:74-100 (variant 1, needs p and column_weight)
 * and g2ptq_utils.py:97-126 (variant 2, needs z and ghinv; ghinv updated in
 * place).  weight is overwritten by the dequantized block; int_weight and
 * error receive codes and scaled errors; scale/zero are per element. */
int g2ptq_block_sweep(void* stream, int variant, int64_t B, int64_t bs, int64_t R, int maxq,
                      float* weight, const float* hinv, const float* p, const float* scale,
                      const float* zero, const float* z, float* ghinv, float* column_weight,
                      float* int_weight, float* error, int* flags);

int g2ptq_compensate_workspace(int variant, int64_t B, int64_t R, int64_t C, int64_t blocksize,
                               size_t* bytes);

/* The lazy-batch loop of _run_compensation for one layer batch:
 * gptq_utils/gptq_utils.py:165-232 (variant 0), gptaq_utils.py:193-261
 * (variant 1), g2ptq_utils.py:252-347 (variant 2).
 *   W   (B,R,C) fp32 in/out (block tails are applied in place, like the reference)
 *   U   (B,C,C) upper factor;  P (B,C,C) GPTAQ only;  Z, GH (B,R,C) G2PTQ only (GH in/out)
 *   Quantizer groups: groupsize g (-1: one group).  dynamic (static_groups == 0 and
 *   g > 0): params of the group starting at column i are fitted on W[:, :, i:i+g]
 *   when the loop reaches i (gptq_utils.py:194-205).  Otherwise scale_tab/zero_tab
 *   must already hold every group's params and colgroup (C ints, nullable) maps
 *   column → group (static groups with act-order: perm[c] // g).  mse_grid > 0 fits
 *   dynamic groups with the MSE clip search (g2ptq_find_params_mse semantics);
 *   hdiag (hblocks × C, nullable) are its hclip weights, the diagonal of the
 *   undamped Hessians in the loop's column order (gptq_utils.py:253-257,
 *   314-315); the B·R rows split into hblocks equal shares (one per layer).
 *   scale_tab/zero_tab: ngroups × (B·R) fp32, group-major (row b·R + r of group g
 *   at g·B·R + b·R + r), ngroups = 1 if g == -1 else ceil(C / g).
 *   Q, Wint, Scale: (B,R,C) outputs (Wint and Scale nullable). */
int g2ptq_compensate(void* stream, int variant, int64_t B, int64_t R, int64_t C,
                     int64_t blocksize, float* W, const float* U, const float* P, const float* Z,
                     float* GH, int bits, int sym, int64_t groupsize, int static_groups,
                     int mse_grid, float mse_norm, float mse_maxshrink, const float* hdiag,
                     int64_t hblocks, const int* colgroup, float* scale_tab, float* zero_tab, float* Q,
                     float* Wint, float* Scale, int* flags, void* ws, size_t ws_bytes);

/* g2ptq_compensate without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference: it exists only for
 * those callers.  The loop's error columns live in a file-scope device array
 * of 32 MiB (33554432 bytes), one per device, held until the process ends;
 * B·R·blocksize·4 must not exceed it (at blocksize 128, B·R ≤ 65536 rows),
 * else the call fails with G2PTQ_ERR_ARG before touching the device.  With
 * B·R·512·4 within it (B·R ≤ 16384; G2PTQ also keeps one block's near-tail
 * operand, B·R·640·4 in all, so B·R ≤ 13107 there) the loop runs as
 * g2ptq_compensate does with a one-buffer workspace; beyond that it applies
 * every 128-column block's tail separately.  It never overlaps tails on a side stream.  All calls on one
 * device share the array: calls that overlap in time on one device (two
 * streams or two host threads) race on it.  Everything else is as for
 * g2ptq_compensate; nothing is allocated. */
int g2ptq_compensate_noalloc(void* stream, int variant, int64_t B, int64_t R, int64_t C,
                             int64_t blocksize, float* W, const float* U, const float* P,
                             const float* Z, float* GH, int bits, int sym, int64_t groupsize,
                             int static_groups, int mse_grid, float mse_norm,
                             float mse_maxshrink, const float* hdiag, int64_t hblocks,
                             const int* colgroup, float* scale_tab, float* zero_tab, float* Q,
                             float* Wint, float* Scale, int* flags);

/* GPTAQ P = alpha·triu(Dx·Uᵀ, 1)·U for B layers (gptq_utils/gptaq_utils.py:349-352). */
int g2ptq_gptaq_p(void* stream, const float* Dx, const float* U, int64_t B, int64_t C, float alpha,
                  float* P, void* ws, size_t ws_bytes);

/* G2PTQ trust region (gptq_utils/g2ptq_utils.py:459-476) for BG row groups of
 * Rg rows: with A⁻¹ = UᵀU, GA = Grad·A⁻¹, E0 = Q0 − W0,
 *   loss = |(E0⊙GA + E0²/2) / diag(A⁻¹)|,
 *   c    = max(rowsum(Grad⊙GA) − GA²/diag(A⁻¹), 2α·loss, tiny),
 *   beta = mean_j(1 − sqrt(max(1 − 2α·loss/c, 0)))  per row,
 *   Z = beta·(Grad·Uᵀ),  GH = Z·U = beta·GA.
 * enabled == 0 gives beta = 0 and Z = GH = 0.  beta: BG·Rg floats. */
int g2ptq_trust_region(void* stream, const float* Grad, const float* U, const float* Q0,
                       const float* W0, int64_t BG, int64_t Rg, int64_t C, float alpha,
                       int enabled, float* beta, float* Z, float* GH, void* ws, size_t ws_bytes);

int g2ptq_trust_region_workspace(int64_t BG, int64_t Rg, int64_t C, size_t* bytes);

/* ------------------------------------------------------------------------
 * Small device helpers used by the host classes
 * ---------------------------------------------------------------------- */

/* act-order permutation: perm = argsort(mean_b diag(H[b]) or key, descending,
 * ties by index) (gptq_utils/gptq_utils.py:279-282, g2ptq_utils.py:417-419).
 * key_mode 0: key[c] = mean_b H[b][c][c] (H: B × C × C);  key_mode 1: key[c] =
 * mean_b A[b][c] (A: B × C, e.g. act_square).  perm, invperm: C int32 (device). */
int g2ptq_act_order(void* stream, const float* src, int64_t B, int64_t C, int key_mode, int* perm,
                    int* invperm, void* ws, size_t ws_bytes);

/* out[b][r][c] = in[b][r][cols[c]] for a (B·R) × C matrix (column gather). */
int g2ptq_permute_cols(void* stream, const float* in, float* out, int64_t rows, int64_t C,
                       const int* cols);

/* out[b][i][j] = in[b][perm[i]][perm[j]] (symmetric permutation, B × C × C). */
int g2ptq_permute_sym(void* stream, const float* in, float* out, int64_t B, int64_t C,
                      const int* perm);

/* Cast fp32 → bf16/fp16 (dtype 0 bf16, 1 fp16, 2 fp32 copy) with a NaN check
 * (sets G2PTQ_FLAG_NAN_OUTPUT), the write-back of gptq_utils.py:346-353. */
int g2ptq_cast_check(void* stream, const float* in, void* out, int64_t n, int dtype, int* flags);

/* out fp32 = in (bf16/fp16/fp32 by dtype code as above), n elements. */
int g2ptq_to_f32(void* stream, const void* in, float* out, int64_t n, int dtype);

/* ------------------------------------------------------------------------
 * compressed-tensors export
 * ---------------------------------------------------------------------- */

/* One layer's pack-quantized checkpoint tensors, the work of
 * utils/compressed_tensors_utils.py:22-45 (compress) with compressed-tensors
 * 0.18.0's pack_to_int32:
 *   packed[r][w] = OR_{i < 32/bits} ((int8(codes[r][w·(32/bits) + i]) + 2^(bits−1))
 *                  mod 2^bits) << (bits·i), columns past cols contributing 0;
 *   scale_out[r][k] = scale[r][k·groupsize] cast to dtype (0 bf16, 1 fp16, 2 fp32),
 *   and G2PTQ_FLAG_GROUP_SCALE in flags if any scale of a group differs from
 *   the group's first (the reference asserts).
 * codes, scale: rows × cols fp32 (ld ldc, lds); packed: rows × ceil(cols·bits/32)
 * int32 (ld ldp); scale_out (nullable: pack only): rows × cols/groupsize (ld ldo). */
int g2ptq_pack_quantized(void* stream, const float* codes, int64_t ldc, const float* scale,
                         int64_t lds, int64_t rows, int64_t cols, int bits, int64_t groupsize,
                         int32_t* packed, int64_t ldp, void* scale_out, int dtype, int64_t ldo,
                         int* flags);

/* ------------------------------------------------------------------------
 * Calibration statistics — gptq_utils/g2ptq_utils.py (SaliencyCache, GradientCache)
 * ---------------------------------------------------------------------- */

/* SaliencyCache.grad_hook (g2ptq_utils.py:604-618): out[t][g] = mean over the
 * g-th of `groups` equal column groups of x[t][·]², x rows × cols (ld ldx,
 * dtype 0 bf16, 1 fp16, 2 fp32), out rows × groups fp32.  The mean is the
 * fp32 sum times fp32(1/group size). */
int g2ptq_group_mean_square(void* stream, const void* x, int dtype, int64_t rows, int64_t cols,
                            int64_t ldx, int64_t groups, float* out);

/* GradientCache.cache_gradient (g2ptq_utils.py:704-714), elementwise over n:
 * cache = cache·keep + grad·inv_count in fp32 (keep = fp32(k/(k+1)),
 * inv_count = fp32(1/fp32(n_tokens·(k+1))), torch's division by a Python
 * number on the GPU); first != 0: cache = 0 + grad·inv_count (no read). */
int g2ptq_running_mean_update(void* stream, float* cache, const void* grad, int dtype, int64_t n,
                              float keep, float inv_count, int first);

/* Concatenation of n device buffers into dst: bytes [off[b], off[b+1]) of dst
 * receive the first off[b+1] − off[b] bytes of src[b].  src (n device
 * addresses) and off (n + 1 byte offsets, off[0] = 0, non-decreasing) are
 * themselves in device memory; max_bytes is at least the largest block.
 * One launch for the torch.stack(torch.cat(...)) expert stacking of
 * utils/models/mixins.py:93-144 (MoEMixin.stack_experts). */
int g2ptq_concat(void* stream, const uint64_t* src, const int64_t* off, int64_t n,
                 int64_t max_bytes, void* dst);

/* Generic batched fp32 GEMM (MFMA): D = alpha·A·op(B) + beta·C for `batch`
 * matrices; A row-major M×K, B row-major K×N (b_trans = 0) or N×K
 * (b_trans = 1).  Exported for the host classes' small products. */
int g2ptq_gemm_f32(void* stream, int64_t M, int64_t N, int64_t K, int64_t batch, const float* A,
                   int64_t lda, int64_t sA, const float* B, int64_t ldb, int64_t sB, int b_trans,
                   const float* C, int64_t ldc, int64_t sC, float* D, int64_t ldd, int64_t sD,
                   float alpha, float beta);

#ifdef __cplusplus
}
#endif

#endif /* G2PTQ_HIP_H */
