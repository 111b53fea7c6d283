/*
 * C ABI of the MI355X (gfx950) GPTQ+ per-linear quantization hot path.
 *
 * Every entry point takes device pointers allocated by the caller (no entry point allocates
 * device memory), a hipStream_t passed as `void*`, launches asynchronously on that stream and
 * returns an int status:  0 = ok, <0 = argument / HIP error (RQ_E*).  The one static device
 * allocation is the scratch array of rq_hessian_accum_noalloc: RQ_NOALLOC_SCRATCH_BYTES
 * (128 MiB) of `__device__` memory that the loader places on every GPU the library's code
 * object is loaded on, held until the process ends, whether or not that entry point is
 * called.  Shapes are
 * validated on the host before any launch.  Matrices are row-major with explicit leading
 * dimensions (in elements).  The reference implementation is Python; the citations name
 * the reference code each call replaces (file:line in Mrluxianseng/gptq_plus_mp_quant).
 */
#ifndef GPTQPLUS_HIP_H
#define GPTQPLUS_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RQ_OK 0
#define RQ_EINVAL (-1)
#define RQ_EHIP (-2)
#define RQ_ENOTSUP (-3)

/* element types of caller tensors */
#define RQ_F16 0
#define RQ_BF16 1
#define RQ_F32 2

/* g_update modes of rq_quant_block / rq_trailing_update (gptq_plus_utils.py:580-584) */
#define RQ_GMODE_FROZEN 0           /* gh_eff = GH                                          */
#define RQ_GMODE_SURROGATE_BLOCK 1  /* gh_eff = GH + beta_r (W_block_start - anchor)          */
#define RQ_GMODE_SURROGATE_ONLINE 2 /* gh_eff = GH + beta_r (W_live - anchor), per column      */
#define RQ_GMODE_BLOCK_GD 3         /* gh_eff = GH, W updates scaled by second_order_scale      */

/* quantizer modes of rq_quant_block / rq_writeback */
#define RQ_QMODE_CHANNEL 0 /* one scale per row            (gptq_plus_utils.py:1008-1020) */
#define RQ_QMODE_STATIC 1  /* per column-group, act_order  (gptq_plus_utils.py:994-1002)  */
#define RQ_QMODE_DYNAMIC 2 /* per block, from block start  (gptq_plus_utils.py:1202-1209) */

/* Library version (major*10000 + minor*100 + patch). */
int rq_version(void);

/* GPTQPlus.add_batch -- gptq_utils/gptq_plus_utils.py:798-857.
 * H[g] (C x C, fp32, g < G) += X^T diag(sal[:, g]) X over `ntok` tokens, upper-triangle
 * 128x128 tiles only (the lower triangle is filled by rq_hessian_finalize);
 * act_sq[c] += sum_t x[t,c]^2 (act_sq may be NULL), summed in the order of torch's CPU
 * `(x.float() ** 2).sum(0)` (:856), so the result is the reference's bit for bit.
 * X is [ntok, C] (row stride ldx) of type x_dtype,
 * sal is [ntok, G] fp32 (row stride ld_sal).  fp32 products accumulated in fp32
 * (rq_hessian_math), deterministic (bitwise reproducible).  workspace (optional, device, 256-byte aligned, zero-filled when first
 * allocated; the library leaves it reusable): with at least rq_hessian_workspace_bytes
 * bytes the items of a partly filled last round are split along the tokens so the launch
 * ends with full rounds; NULL runs whole items only.  Calls that overlap in time on one
 * device need separate workspaces.  The size depends on x_dtype (fp32 X needs its 16-bit row
 * pieces and fp32 column copy). */
int64_t rq_hessian_workspace_bytes(int64_t ntok, int C, int ntargets, int x_dtype);

/* Kernel choice (process-wide).  The split kernels form each fp32 product x * fl32(x * s) on
 * the 16-bit MFMA pipe from the weighted operand cut into 16-bit pieces (after an exact
 * power-of-two column scaling), and accumulate in fp32; they need the workspace (with less
 * than rq_hessian_workspace_bytes the fp32 kernel runs instead).
 * RQ_HMATH_SPLIT16X3 (default): the reference's fp32 products exactly.  fp16 and bf16 X with
 *   the weighted operand in three pieces (11 + 11 + 2 or 8 + 8 + 8 bits; for fp16, every
 *   operand within 2^15 of its column's largest, below that within 2^-40 of the largest);
 *   fp32 X on the fp32 MFMA kernel.
 * RQ_HMATH_SPLIT16 (opt-in, faster, narrower products): fp16 X in two pieces (22 of the
 *   operand's 24 bits: each product within 2^-23 relative of the reference's, 2/3 of the MFMA
 *   work), bf16 X in three; fp32 X with x itself in two fp16 pieces, three MFMAs per product
 *   (hi w0, hi w1, lo w0: each product within ~2^-20.5 relative; k_hessian_split32, about 3x
 *   the fp32 MFMA kernel's speed).
 * RQ_HMATH_FP32: fp32 MFMA on converted operands for every input type (exact fp32 products).
 * mode < 0 queries.  Returns the previous mode, or RQ_EINVAL.  No counterpart in the
 * reference (its bmm runs in fp32, gptq_plus_utils.py:845-847). */
#define RQ_HMATH_SPLIT16 0
#define RQ_HMATH_FP32 1
#define RQ_HMATH_SPLIT16X3 2
int rq_hessian_math(int mode);
/* Measurement hook, no counterpart in the reference: the next Hessian product-kernel launch
 * (k_hessian_split or k_hessian_accum, whichever runs; k_hessian_split issues one call's
 * items as one dispatch per round of whole items, and the pair brackets all of them) records
 * start_event before it and stop_event after it on its stream, so a caller can time that
 * kernel alone (hipEvent_t handles created with timing enabled; both NULL clears).
 * Process-wide, one call per pair. */
int rq_hessian_timing_events(void* start_event, void* stop_event);
int rq_hessian_accum(const void* x, int x_dtype, int64_t ntok, int64_t ldx, int C,
                     const float* sal, int64_t ld_sal, int G, float* H, float* act_sq,
                     void* workspace, int64_t workspace_bytes, void* stream);

/* rq_hessian_accum for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  Same arguments, kernels and results as rq_hessian_accum minus the workspace: a
 * scratch array of the library (RQ_NOALLOC_SCRATCH_BYTES on every GPU the library runs on,
 * held until the process ends) serves as the workspace, so the call allocates nothing.
 * Returns RQ_EINVAL when the call needs more scratch than that (the split kernel needs about
 * 2 * ntok * C bytes for its copy of the chunk: pass fewer tokens per call).  Every call on a
 * GPU shares that GPU's array, which keeps the last call's contents: calls that overlap in time
 * on one GPU race. */
#define RQ_NOALLOC_SCRATCH_BYTES (128u << 20)
int rq_hessian_accum_noalloc(const void* x, int x_dtype, int64_t ntok, int64_t ldx, int C,
                             const float* sal, int64_t ld_sal, int G, float* H, float* act_sq,
                             void* stream);

/* Cross-module fused accumulation: the add_batch of several GPTQPlus objects whose modules read
 * the same input (q/k/v, gate/up; their forward hooks receive the same tensor,
 * gptq_plus_utils.py:6991-7003) in one launch, so X is streamed once for all of them.
 * Target t (< 32) accumulates H[t] (C x C) += X^T diag(s_t) X with s_t = sal[t][i * ld_sal[t]],
 * and act_sq[t] (when act_sq and act_sq[t] are non-NULL) += sum_t x^2.  sal, ld_sal, H and
 * act_sq are HOST arrays of device pointers / strides. */
int rq_hessian_accum_multi(const void* x, int x_dtype, int64_t ntok, int64_t ldx, int C,
                           int ntargets, const float* const* sal, const int64_t* ld_sal,
                           float* const* H, float* const* act_sq, void* workspace, int64_t workspace_bytes,
                           void* stream);

/* GPTQPlus.finalize_hessian -- gptq_plus_utils.py:859-908 (world size 1).
 * H = sym(upper(H)) / h_div [/ sal_scale if != 1]; non-finite entries are counted into
 * *nonfinite (device int, accumulated; may be NULL) and, with sanitize != 0 (GPTQPlus,
 * :895-906), set to 0; sanitize = 0 keeps them (classic GPTQ, gptq_utils.py:63-106, whose
 * Cholesky retries then fail and raise).  act_sq /= seq_len. */
int rq_hessian_finalize(float* H, float* act_sq, int G, int C, double h_div, double sal_scale,
                        double seq_len, int sanitize, int* nonfinite, void* stream);

/* WeightQuantizer.find_params, per-channel min/max -- utils/quant_utils.py:390-421
 * (static column groups: gptq_plus_utils.py:994-1002).  For each group k of `group_size`
 * columns (group_size <= 0: one group of all C columns) and row r:
 * scale[k*R + r], zero[k*R + r].  clip_zero != 0: the range is widened to include 0
 * (find_params); clip_zero = 0: the group's own min / max (find_params_weight_groupwise,
 * :333-352). */
int rq_find_params(const void* w, int w_dtype, int R, int C, int64_t ldw, int group_size,
                   int maxq, int sym, int clip_zero, float* scale, float* zero, void* stream);

/* WeightQuantizer.find_params with mse=True (the --w_clip grid search) -- utils/quant_utils.py:
 * 408-448 (groupwise: :354-386): per (row, group) min/max start, then int(maxshrink*grid)^2
 * shrunken (xmin, xmax) candidates scored by sum |q - x|^norm; the first strict minimum is
 * kept.  Same layouts and clip_zero as rq_find_params. */
int rq_find_params_mse(const void* w, int w_dtype, int R, int C, int64_t ldw, int group_size,
                       int maxq, int sym, int clip_zero, double norm, int grid, double maxshrink,
                       float* scale, float* zero, void* stream);

/* act_order permutation -- gptq_plus_utils.py:1046, 1050 (classic GPTQ: argsort of diag(H)):
 * perm = torch.argsort(act_sq, descending=True) exactly as torch returns it on the CPU, ties
 * included (the order libstdc++'s introsort leaves equal keys in; NaN first), and
 * invperm = argsort(perm).  int64 outputs.  C <= RQ_ACT_ORDER_MAXC (the widest linear of
 * today's models has 53248 input columns), else RQ_EINVAL. */
#define RQ_ACT_ORDER_MAXC 65536
int rq_act_order_perm(const float* act_sq, int C, int64_t* perm, int64_t* invperm, void* stream);

/* Per-subgroup slicing, dead columns and act_order gather -- gptq_plus_utils.py:1033-1050.
 * dead[c] = (H_g[c,c] == 0).  W_sub[r,j] = dead[p_j] ? 0 : w[r, p_j] (fp32),
 * G_sub[r,j] = grad[r, p_j] (skipped when grad == NULL), H_sub[i,j] = H_g[p_i, p_j] with
 * H_sub[i,i] = 1 where dead[p_i]; p = perm (identity when perm == NULL).  w/grad point at the
 * subgroup's first row.  H_sub must not overlap H_g, w, grad, W_sub or G_sub: its first 2*C
 * words carry the gathers' column indices on the stream before the H gather writes it. */
int rq_prepare_subgroup(const void* w, int w_dtype, int64_t ldw, const float* grad, int64_t ldg,
                        const float* H_g, int R_s, int C, const int64_t* perm, float* W_sub,
                        int64_t ld_wsub, float* G_sub, int64_t ld_gsub, float* H_sub, void* stream);

/* Most matrices one rq_chol_hinv_attempt call factorises (nb). */
#define RQ_CHOL_MAXBATCH 64

/* Bytes of device workspace rq_chol_hinv_attempt needs per C x C matrix. */
int64_t rq_chol_workspace_bytes(int C);

/* One attempt of GPTQPlus._compute_hessian_inverse_with_fallback -- gptq_plus_utils.py:519-533,
 * for a batch of nb <= RQ_CHOL_MAXBATCH subgroup matrices H_work[b] = H_work + b*C*C (one per row group):
 * H_work[b][i,i] += fl32(damp_percent[b]) * mean(diag(H_work[b]))  (in place: retries
 * accumulate, as in the reference), then Hinv[b] = upper Cholesky factor of H_work[b]^-1
 * (Hinv^T Hinv = H_work^-1), when Hinv_init != NULL, Hinv_init[b] = H_work[b]^-1, and when
 * Hinv_diag != NULL, Hinv_diag[b] (C floats at b*C) = diag(H_work[b]^-1), the reference's
 * torch.diagonal(hinv_init) (:184), without forming the matrix.  damp_percent is a HOST array; entries <= 0 are skipped (left untouched).  Factorisation in
 * fp64 (blocked, MFMA).  info (device int[nb]) is written per entry: 0 = done, > 0 = not
 * positive definite or non-finite result (caller raises the damping and retries that entry),
 * -1 = skipped.  workspace holds nb * rq_chol_workspace_bytes(C) bytes. */
int rq_chol_hinv_attempt(float* H_work, int C, int nb, const double* damp_percent, void* workspace,
                         float* Hinv, float* Hinv_init, float* Hinv_diag, int* info, void* stream);

/* GPTQPlus._compute_gradient_terms -- gptq_plus_utils.py:563-578 with
 * compute_safe_beta_from_reference_loss -- :174-194, for nsub subgroups at once: subgroup b
 * owns rows [b*R_s, (b+1)*R_s) of G (row stride ldg), Z and GHinv (row stride ldz), beta
 * (beta_mode 1) and GH0, the upper factor Hinv + b*C*C (Hinv^T Hinv = Hinv_init), hinv_diag +
 * b*C = diag(Hinv_init) (from rq_chol_hinv_attempt) and z_nonzero[b].
 * beta_mode 0: beta = 0 (alpha <= 0 or gradient update off; beta has 1 element);
 * beta_mode 1: beta[r] from G, hinv_diag and the reference's G Hinv_init (:180), formed as
 * (G Hinv^T) Hinv in the GH0 workspace [nsub*R_s, C] (two triangular products, no H^-1).
 * Z = (G Hinv^T) * beta, GHinv = Z Hinv.  HinvT (optional workspace, nsub*C*C floats, used by
 * beta_mode 1): with it, and C a multiple of 16, the products run as batched 128-tile NT GEMMs.
 * z_nonzero[b] (device ints) is set to 1 when any Z element of subgroup b is non-zero or NaN;
 * 0 lets later kernels skip provably-zero first-order work. */
int rq_gptqplus_terms(const float* G, int64_t ldg, const float* hinv_diag, const float* Hinv,
                      float* HinvT, int R_s, int nsub, int C, double alpha_eff, double reference_loss,
                      int beta_mode, float* beta, float* Z, float* GHinv, int64_t ldz, float* GH0,
                      int* z_nonzero, void* stream);

/* One block of the fasterquant loop for ALL subgroups -- gptq_plus_utils.py:1169-1372:
 * columns [i1, i1+count) of the permuted working weight Wp [R, C] (row stride ldw),
 * subgroup s = rows [s*R_s, (s+1)*R_s) with upper Hinv_all + s*C*C.
 * Non-atomic: the column-serial quantize / error / rank-1 update (:1296-1367) incl. the
 * GPTQ+ GHinv terms.  atomic != 0: quantize the block start at once and solve
 * Err * Hinv1 = W - Q - GHinv1 (:1238-1288; the caller passes atomic = 0 for the last block).
 * Writes int16 codes [R, C] (permuted order) and err [R, count] for rq_trailing_update.
 * qmode: RQ_QMODE_CHANNEL scale[r]; RQ_QMODE_STATIC scale[col_group[i1+i]*R + r];
 * RQ_QMODE_DYNAMIC computes scale from the block start into dyn_scale[r] (caller offsets it
 * per block).  count <= 128.
 * gmode (RQ_GMODE_*): in the surrogate modes the GHinv term is refreshed before every
 * column (:1190-1199, :1360-1367) from anchor (the permuted weight before the first block,
 * [R, C] row stride ld_anchor) and beta[r] (fp32, one per row of all subgroups); both may be
 * NULL for RQ_GMODE_FROZEN / RQ_GMODE_BLOCK_GD.  RQ_GMODE_BLOCK_GD scales every in-block
 * weight update by second_order_scale (:1344-1349; ignored by the other modes).
 * block_backward's inner loop is RQ_GMODE_SURROGATE_ONLINE (:1190). */
int rq_quant_block(float* Wp, int64_t ldw, const float* Hinv_all, int C, const float* GH,
                   const float* Z, int64_t ldgh, int R, int R_s, int i1, int count, int qmode,
                   const float* scale, const int32_t* col_group, float* dyn_scale, int maxq,
                   int sym, int atomic, const int* z_nonzero, int16_t* codes, float* err,
                   int gmode, const float* anchor, int64_t ld_anchor, const float* beta,
                   double second_order_scale, void* stream);

/* Outer (trailing) update after a block -- gptq_plus_utils.py:1500-1570:
 * Wp[:, i2:] -= err Hinv[i1:i2, i2:] + (count GH[:, i2:] - (Z[:, i1:i2] D) Hinv[i1:i2, i2:]),
 * GH[:, i2:] -= Z[:, i1:i2] Hinv[i1:i2, i2:], D = [count-1, ..., 0], per subgroup; the Z
 * terms are skipped when *z_nonzero == 0.  fp32 MFMA.  For the surrogate gmodes the GH of
 * the first term is GH + beta[r] (Wp - anchor) (outer refresh "surrogate_block",
 * :1500-1511); the GH update is unchanged.  RQ_GMODE_BLOCK_GD scales the whole W update by
 * second_order_scale (:1546-1549); block_backward's outer update is RQ_GMODE_FROZEN.
 * z_zero != 0 is the caller's statement that Z (hence GH) is identically zero, i.e. that
 * *z_nonzero == 0 (read back once after rq_gptqplus_terms): the frozen / block_gd modes then
 * run a W-only kernel with 128x128 tiles.  Pass 0 when unknown; *z_nonzero then decides. */
int rq_trailing_update(float* Wp, int64_t ldw, float* GH, const float* Z, int64_t ldgh,
                       const float* Hinv_all, int C, int R, int R_s, int i1, int count,
                       const float* err, const int* z_nonzero, int z_zero, int gmode, const float* anchor,
                       int64_t ld_anchor, const float* beta, double second_order_scale,
                       void* stream);

/* The frozen-mode column loop's per-block pair -- rq_trailing_update for block k
 * (gptq_plus_utils.py:1512-1519) and rq_quant_block for block k+1 (:1296-1367) -- in one
 * launch, for Z (hence GH) identically zero; equal to the two calls bit for bit.  Block k =
 * columns [i1, i1+count) with its err [R, count]; block k+1 = [i1+count, i1+count+count_next).
 * The workgroups that quantise block k+1 first apply block k's update to their own rows of
 * its columns (the CPU matmul's order, written back to Wp); the rest apply block k's update to
 * the columns past block k+1 meanwhile.  Writes block k+1's codes and its err to err_next
 * ([R, count_next], a different buffer from err); dyn_scale is block k+1's, atomic applies
 * to block k+1.  Needs count % 8 == 0, C % 4 == 0, (i1 + count + count_next) % 4 == 0 and
 * Hinv_all, err 16-byte aligned (else RQ_EINVAL: use the two calls).  No single counterpart in
 * the reference: it fuses two of its steps for the look-ahead over blocks. */
int rq_quant_block_lookahead(float* Wp, int64_t ldw, const float* Hinv_all, int C, int R, int R_s,
                             int i1, int count, const float* err, int count_next, int qmode,
                             const float* scale, const int32_t* col_group, float* dyn_scale,
                             int maxq, int sym, int atomic, int16_t* codes, float* err_next,
                             void* stream);

/* Un-permute and write back -- gptq_plus_utils.py:1850-1875:
 * natural column c of row r takes permuted column j = invperm[c] (identity if NULL):
 * Q = scale(r, j) * code[r, j]; q_out (layer dtype q_dtype, [R, C] row stride ldq) = Q;
 * optional fp32 W_int / Scale (export_to_et, :1866-1871) when the pointers are non-NULL.
 * *nan_flag (device int) is set to 1 if any written weight is NaN (:1882-1896).
 * dynamic mode: dyn_scale[(j / blocksize) * R + r]. */
int rq_writeback(const int16_t* codes, int R, int C, const int64_t* invperm, int qmode,
                 const float* scale, const int32_t* col_group, const float* dyn_scale,
                 int blocksize, void* q_out, int q_dtype, int64_t ldq, float* w_int_out,
                 float* scale_out, int* nan_flag, void* stream);

/* Packed export.  The reference's export_to_et keeps codes and scales as two fp32 [R, C]
 * tensors (gptq_plus_utils.py:1866-1871) and saves the `quantizers` dict next to the
 * fake-quantized state_dict (gptq_utils/main.py:68-71); this is the compact form of the
 * same information.  Row r of `out` is a little-endian bitstream of C fields of nbits bits:
 * field c = code[r, invperm ? invperm[c] : c] + 2^(nbits-1), at bits [c*nbits, (c+1)*nbits),
 * bit b in bit (b & 31) of 32-bit word (b >> 5); trailing bits are zero.
 * nbits = bits for sym, bits + 1 for asym (codes lie in [-(maxq+1), maxq],
 * quant_utils.py:477).  Returns the words per row (ceil(C*nbits/32)), or RQ_EINVAL. */
int64_t rq_packed_words_per_row(int C, int nbits);

/* Pack int16 codes [R, C] (row stride ldc; permuted order when invperm != NULL) into
 * out [R, ldo] uint32.  A code outside [-2^(nbits-1), 2^(nbits-1)) (incl. the NaN marker)
 * sets *range_flag (device int, optional) and is stored masked.  2 <= nbits <= 16. */
int rq_pack_codes(const int16_t* codes, int R, int C, int64_t ldc, const int64_t* invperm,
                  int nbits, uint32_t* out, int64_t ldo, int* range_flag, void* stream);

/* Inverse of rq_pack_codes, optionally dequantizing: codes_out[r, c] (int16 [R, C], optional)
 * and q_out[r, c] = scales[g_idx[c] * lds + r] * code (fp32 product, then cast to q_dtype,
 * [R, C] row stride ldq), g_idx NULL = one group.  Equal, bit for bit, to the weight
 * fasterquant wrote (rq_writeback) when scales / g_idx describe its scale table. */
int rq_unpack_dequant(const uint32_t* packed, int R, int C, int64_t ldp, int nbits,
                      const float* scales, int64_t lds, const int32_t* g_idx, void* q_out,
                      int q_dtype, int64_t ldq, int16_t* codes_out, void* stream);

/* The refresh g_update modes (block_gd, block_backward): the caller's layer backward runs
 * between blocks on the current weight; these entry points prepare its input and apply its
 * output.
 *
 * Current effective weight -- gptq_plus_utils.py:1389-1396, 1412-1420, 1578-1588, 1690-1692:
 * value(r, j) = j < i_q ? fl32(scale(r, j) * code[r, j]) : Wp[r, j] (permuted column j, scale
 * by qmode as in rq_writeback); out[r, c] = value(r, invperm ? invperm[c] : c)
 * - (sub_ref ? sub_ref[r, c] : 0).  invperm un-permutes (the snapshot handed to the caller);
 * without it the output stays in the permuted order (block_backward's new anchor, or with
 * sub_ref = W_fp the hessian regularizer's difference, :766). */
int rq_current_weight(const float* Wp, int64_t ldw, const int16_t* codes, int R, int C, int i_q,
                      int qmode, const float* scale, const int32_t* col_group,
                      const float* dyn_scale, int blocksize, const int64_t* invperm,
                      const float* sub_ref, int64_t ld_ref, float* out, int64_t ldo, void* stream);

/* dst[r, j] = src[r, perm[j]] (perm NULL = copy): the refreshed gradient in act_order's
 * column order (:1430-1432, 1688-1690). */
int rq_gather_cols(const float* src, int64_t lds, const int64_t* perm, int R, int C, float* dst,
                   int64_t ldd, void* stream);

/* H-Adam curvature -- build_kfac_curvature_diag :4601-4640 as called at :1144-1151: for each
 * of nsub matrices H_work[s] (dead-fixed, permuted, undamped), curv[s][j] =
 * max(d_j, 0) / max(mean(max(d, 0)), 1e-12) + damping (damping added only when > 0). */
int rq_kfac_curvature(const float* H_work, int C, int nsub, double damping, float* curv,
                      void* stream);

/* Hessian regularizer product -- :765-768: out[s] = diff[s] (R_s x C, row stride ldd) times
 * H_reg[s][:, i2:] (H_reg [G, C, C]), out [R, C - i2] row stride ldo.  fp32 MFMA. */
int rq_hessian_reg_gemm(const float* diff, int64_t ldd, const float* H_reg, int C, int R, int R_s,
                        int i2, float* out, int64_t ldo, void* stream);

/* One block_gd optimizer step on the trailing permuted columns [i2, C) of all rows --
 * _compute_grad_optimizer_update :616-655 + _apply_first_order_regularizer :730-796 +
 * W_sub[:, i2:] -= update :1828-1834.  grad: natural order [R, C] (row stride ldg), read
 * through perm.  optimizer 0 sgd, 1 adam (exp_avg, exp_avg_sq [R, C]), 2 h_adam (exp_avg,
 * curvature [G, C]); step = the optimizer's step count after its increment; betas 0.9 /
 * 0.999, eps 1e-8.  reg_strategy 0 none, 1 l2 (w_fp [R, C]), 2 hessian (hreg from
 * rq_hessian_reg_gemm), 3 quant_error_gate, 4 quant_error_gate_optimized (gate maps:
 * gate_qmode RQ_QMODE_CHANNEL -> gate_scale[r] / gate_zero[r], RQ_QMODE_STATIC ->
 * [col_group[j] * R + r]).  stats_parts (optional, 4 * R * (C - i2) floats, the
 * refresh_full_metrics statistics' inputs :1688-1770): planes [4][R][C - i2] of the
 * optimizer step (optimizer_update_raw), the applied update (optimizer_update), the
 * regularizer part (gate_regularizer_update: the l2 / hessian term, or gated - step) and the
 * sine part (sine_regularizer_update). */
int rq_block_gd_step(float* Wp, int64_t ldw, int R, int R_s, int C, int i2, const float* grad,
                     int64_t ldg, const int64_t* perm, int optimizer, int step, double lr,
                     double grad_clip, float* exp_avg, float* exp_avg_sq, const float* curvature,
                     int reg_strategy, double reg_lambda, const float* w_fp, int64_t ld_fp,
                     const float* hreg, int64_t ld_hreg, int gate_qmode, const float* gate_scale,
                     const float* gate_zero, const int32_t* col_group, int maxq, int sym,
                     double gate_floor, double gate_sharpness, double sine_amp, float* stats_parts,
                     void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GPTQPLUS_HIP_H */
