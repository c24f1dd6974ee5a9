/* sdcguard_hip.h -- C ABI of libsdcguard_hip.so, the MI355X (gfx950) verification hot path of sdcguard.
 *
 * Plain pointers (device memory), element strides, sizes and a hipStream_t; no torch types.  Every entry
 * point queues work on `stream` and returns at once (no host synchronisation), returning 0 on success or a
 * negative status:
 *   -1 SDC_EINVAL       an argument is out of range (shape, stride, null pointer)
 *   -2 SDC_EUNSUPPORTED a case this library does not implement; the caller must not treat it as checked
 *   -3 SDC_EWORKSPACE   the workspace is smaller than the matching *_workspace() call asked for
 *   -4 SDC_ELAUNCH      a HIP launch error
 * dtype: 0 = bf16, 1 = fp16.  Integer results wrap modulo 2^64 like the reference's int64 arithmetic.
 */
#ifndef SDCGUARD_HIP_H
#define SDCGUARD_HIP_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- serving check of one linear layer --------------------------------------------------------------------
 * Replaces the custom op sdcguard::check_static (serve.py:465-489) and what it runs: _serve_fast.check
 * (_serve_fast.py:632) = check_v1/check_v3 (:265-313, :539-587), i.e. E = x @ parts then the block sums of y and
 * the scoring of _check/_judge/_report (:102-262, :334-452); same arithmetic as serve._check_static_impl
 * (serve.py:301-396).
 *   x (m x k), y (m x n): element strides (sxm, sxk), (sym, syn); both of `dtype`.
 *   parts: the three low-precision parts of the layer's block sums B2 / scale (k x 6nb, LayerChecksums.parts,
 *     serve.py:186), element (kk, c) at parts[kk * spk + c * spc]; spk must be 1 (k-contiguous columns).
 *     nparts must be 3.
 *   sign_table: 128 x 128 fp32, row w-1 = the epoch-0 +-1 pattern of width w (_group.py:262-291).
 *   scale, b2n, b2max, bsum: (nb, 2) fp32; bmax, bmax_bias: (nb,) fp32 (LayerChecksums.tensors()).
 *   state: the layer's row of the guard's state (int64): keys at [0], [1]; with counts != 0, checks executed
 *     at [2] and unjudged checksums at [3] (serve.py:55-65).  slot: the layer's slot (capture flag index).
 *   cap_meta / cap_data (may be NULL): the capture buffers of serve.py:67-88; cap_flags = CAP_FLAGS,
 *     cap_slots = CAPTURE_SLOTS, cap_stride = cap_data's row stride, cap_w = where x starts in a row.
 *   workspace: device memory of at least sdc_check_static_workspace(m, k, n, bs) bytes.
 *   scores_out (may be NULL): every checksum's score, (m, nb, 2) fp32, plain then signed (for tests).
 *   kernel: 0 or 1 = v1, the GEMM then one persistent pass over y that sums and scores every pair (fastest at
 *     every batch size measured on MI355X); 3 = v3, the block sums of y on a side stream concurrently with the
 *     GEMM, then a scoring pass (the reference's SDCGUARD_SERVE_KERNEL=v1|v3 switch); 4 = v3 on `stream` alone.
 *   block_consts (may be NULL): the same per-block constants packed as (nb, 12) fp32, 16-byte aligned, per block
 *     [scale0, scale1, bsum0, bsum1, b2n0, b2n1, b2max0, b2max1, bmax, bmax_bias, 0, 0]: three 16-byte loads
 *     per block instead of ten scattered ones; the separate arrays are still required.
 *   parts_frag (may be NULL; no counterpart in the reference): the parts in sdc_parts_fragments' order, 16-byte
 *     aligned, made once per layer: with them (k-contiguous 16-bit x, depth a multiple of 512) the expected side
 *     runs on the register-streamed tall-tile GEMM (two planes of E) instead of the staged one. */
int64_t sdc_check_static_workspace(int64_t m, int64_t k, int64_t n, int64_t bs);
int sdc_check_static(int dtype, const void* x, int64_t sxm, int64_t sxk, const void* y, int64_t sym, int64_t syn,
                     int64_t m, int64_t k, int64_t n, int64_t bs, const void* parts, int64_t spk, int64_t spc,
                     int nparts, const float* sign_table, const float* scale, const float* b2n,
                     const float* b2max, const float* bmax, const float* bmax_bias, const float* bsum,
                     int64_t* state, int counts, int64_t slot, float z, float abs_floor, int64_t* cap_meta,
                     float* cap_data, int64_t cap_stride, int64_t cap_w, int64_t cap_tag, int64_t cap_flags,
                     int64_t cap_slots, void* workspace, int64_t workspace_bytes, float* scores_out, int kernel,
                     const float* block_consts, const void* parts_frag, hipStream_t stream);

/* ---- check of one matmul (training / one-off) -------------------------------------------------------------
 * Replaces checksum.matmul_zscores (checksum.py:400-432, `_zscores` :435-530) and the Triton group it routes to
 * (_group.Group.add/launch/row, _group.py:749-902): the column-block check of C = beta * bias + alpha * (A @ B)
 * with B's block sums made on the device for this call, unjudged checksums scoring -1 (checksum.py:346-383).
 *   A (batch_a, m, k), B (batch_b, k, n), C (batch_c, m, n): element strides per dimension; batch_a / batch_b may
 *     be 1 (shared) or equal to batch_c (bmm); all of `dtype`.
 *   bias_kind 0: none; 1: a vector of n (stride sbias_n); 2: a matrix (strides sbias_b, sbias_m, sbias_n; sbias_b
 *     0 for a 2-D bias shared by the batches) -- addmm / baddbmm biases (checksum.py:471-479).
 *   sign_table: the 128 x 128 table of the epoch in use (epoch 0: as serving; a later epoch: _group._sign_table).
 *   result: int64[3], zeroed by the caller: the worst checksum's key (bits of z << 32 | flat index, flat =
 *     ((batch * m + row) * nb + block) * 2 + signed), the key with its noise, and the number of checksums that
 *     could not be judged.  Several checks may share no result row.
 *   workspace: at least sdc_matmul_check_workspace(batch_a, batch_b, m, k, n, bs) bytes.
 *   scores_out (may be NULL): every checksum's score, (batch_c, m, nb, 2) fp32 (tests). */
int64_t sdc_matmul_check_workspace(int64_t batch_a, int64_t batch_b, int64_t m, int64_t k, int64_t n, int64_t bs);
int sdc_matmul_check(int dtype, const void* A, int64_t sab, int64_t sam, int64_t sak, int64_t batch_a,
                     const void* B, int64_t sbb, int64_t sbk, int64_t sbn, int64_t batch_b, const void* C, int64_t scb,
                     int64_t scm, int64_t scn, int64_t batch_c, int64_t m, int64_t k, int64_t n, int64_t bs,
                     const void* bias, int bias_kind, int64_t sbias_b, int64_t sbias_m, int64_t sbias_n, float alpha,
                     float beta, float z, float abs_floor, const float* sign_table, int64_t* result, void* workspace,
                     int64_t workspace_bytes, float* scores_out, hipStream_t stream);

/* ---- precise check of one matmul with an fp32 output (the accumulator itself) ------------------------------
 * Replaces checksum.matmul_zscores_acc / _acc_zscores / check_matmul_acc (checksum.py:537-692): the column-block check
 * of C = beta * bias + alpha * (A @ B) for bf16/fp16 A and B (dtype) and an fp32 C that was not rounded to 16 bits.
 * Both sides of every checksum are float64 (block sums of B and of C, A @ B2); the noise is the fp32 accumulation's
 * rounding u (C1 sqrt(k) |alpha| |a_row|_2 |B_block|_F + (C2 sqrt(k) + C3 k / nfma + sqrt(width)) |C_block|_2),
 * u = 2^-24, C1 = 0.6, C2 = C3 = 1; Inf/NaN judged as checksum._judge_nonfinite with fp32 outputs.
 *   A, B, C, batches, strides, bs (<= 128), sign_table, result, scores_out: as sdc_matmul_check (C fp32; batch_a and
 *     batch_b are 1 or batch_c).  nfma: products per tensor-core truncation step (0: none).
 *   bias_kind: 0 none, 1 vector of n (stride sbias_n), 2 matrix (strides sbias_b, sbias_m, sbias_n); + 4 when the
 *     bias is fp32 (otherwise of dtype).  k >= 1 (a product with k = 0 is checked as one zero column).
 *   workspace: at least sdc_matmul_check_acc_workspace(batch_a, batch_b, batch_c, m, k, n, bs) bytes. */
int64_t sdc_matmul_check_acc_workspace(int64_t batch_a, int64_t batch_b, int64_t batch_c, int64_t m, int64_t k,
                                       int64_t n, int64_t bs);
int sdc_matmul_check_acc(int dtype, const void* A, int64_t sab, int64_t sam, int64_t sak, int64_t batch_a,
                         const void* B, int64_t sbb, int64_t sbk, int64_t sbn, int64_t batch_b, const float* C,
                         int64_t scb, int64_t scm, int64_t scn, int64_t batch_c, int64_t m, int64_t k, int64_t n,
                         int64_t bs, const void* bias, int bias_kind, int64_t sbias_b, int64_t sbias_m,
                         int64_t sbias_n, float alpha, float beta, float nfma, float z, float abs_floor,
                         const float* sign_table, int64_t* result, void* workspace, int64_t workspace_bytes,
                         float* scores_out, hipStream_t stream);

/* ---- the precise check scored from the fused GEMM's block statistics ----------------------------------------
 * Replaces fused.zscores_from_stats (fused.py:181-235): the check of sdc_matmul_check_acc for C = A @ B + bias (2-D,
 * alpha = beta = 1) with C's plain, signed, squared and absolute block sums read from stats ((m, nb, 4) float64,
 * strides sst_m, sst_b in doubles, as sdc_fused_mm writes them) instead of C.  bias: a vector of n (of dtype, or fp32
 * with bias_f32) or null.  Blocks of 128 columns (one of n when n < 128).  k >= 1.  workspace: at least
 * sdc_matmul_check_acc_workspace(1, 1, 1, m, k, n, 128) bytes. */
int sdc_matmul_check_acc_stats(int dtype, const void* A, int64_t sam, int64_t sak, const void* B, int64_t sbk,
                               int64_t sbn, const double* stats, int64_t sst_m, int64_t sst_b, int64_t m, int64_t k,
                               int64_t n, const void* bias, int bias_f32, float nfma, float z, float abs_floor,
                               const float* sign_table, int64_t* result, void* workspace, int64_t workspace_bytes,
                               float* scores_out, hipStream_t stream);

/* ---- a linear layer's matmul with its precise check fused in ------------------------------------------------
 * Replace fused.fused_mm (fused.py:116-170) and fused.fused_mm_checked (fused.py:462-546).  C = A @ B + bias, A (m, k)
 * and B (k, n) of dtype (bf16/fp16) with any strides (B is typically a weight's transpose), C (m, n) of dtype with
 * row stride scm and unit column stride, computed on MFMA with fp32 accumulation and rounded once (bias, a vector
 * of n of dtype or fp32 with bias_f32, added in fp32 first).  inject != 0 adds inj_v to the accumulator at
 * (inj_m, inj_n) before rounding (fault-injection experiments).  m, n >= 1, k >= 0 (k = 0: C is the bias).
 * Operands that are not depth-contiguous with 16-byte aligned rows, or whose k is not a multiple of 32, are copied
 * into the workspace first.  workspace: at least sdc_fused_mm_workspace(...) bytes (0 is possible for sdc_fused_mm).
 *   sdc_fused_mm: also stats ((m, ceil(n / 128), 4) float64, contiguous): per row and block of 128 columns the
 *     plain sum, signed sum (the block width's pattern from sign_table), sum of squares and sum of absolute values
 *     of the fp32 accumulator before rounding; sdc_matmul_check_acc_stats scores them.
 *   sdc_fused_mm_checked: the check scored in the kernel (no float64 on the expected side): A times three 16-bit
 *     parts of each block sum of B on MFMA, summed with compensation; precise mode's noise model plus the expected
 *     side's rounding (C1 sqrt(32) u |a_row| |block sums|_2 + 4 u |expected|); result, scores_out ((m, nb, 2) or
 *     null) as sdc_matmul_check; expected_out ((m, nb, 2) float64 or null) receives the expected sides. */
int64_t sdc_fused_mm_workspace(const void* A, int64_t sam, int64_t sak, const void* B, int64_t sbk, int64_t sbn,
                               int64_t m, int64_t k, int64_t n, int checked);
int sdc_fused_mm(int dtype, const void* A, int64_t sam, int64_t sak, const void* B, int64_t sbk, int64_t sbn,
                 int64_t m, int64_t k, int64_t n, const void* bias, int bias_f32, const float* sign_table, void* C,
                 int64_t scm, double* stats, int64_t inj_m, int64_t inj_n, float inj_v, int inject, void* workspace,
                 int64_t workspace_bytes, hipStream_t stream);
int sdc_fused_mm_checked(int dtype, const void* A, int64_t sam, int64_t sak, const void* B, int64_t sbk,
                         int64_t sbn, int64_t m, int64_t k, int64_t n, const void* bias, int bias_f32,
                         const float* sign_table, void* C, int64_t scm, float nfma, float z, float abs_floor,
                         int64_t* result, float* scores_out, double* expected_out, int64_t inj_m, int64_t inj_n,
                         float inj_v, int inject, void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* ---- the check of a serving layer's FP8 input quantization ---------------------------------------------------
 * Replaces serve_fp8.quant_check_torch (serve_fp8.py:79-178): did the FP8 codes xq the GEMM got, and their scale(s)
 * xs, come from this step's real rows of x by the layer's recipe (0 static: xs[0] against static_ref[0] when given;
 * 1 dynamic per tensor: max |x| over the real rows / 448 against xs[0], noting a scale equal to the maximum over
 * every row; 2 dynamic per token: each sampled row's max |x| / 448, capped by scale_ub[0] when given and at least
 * 1 / (448 * 512), against xs[row])?  Two rows sampled per call ((step * 7919 + j * 104729) % rows) are quantized
 * as the layer's kernels do (x / scale per token, x * (1 / scale) otherwise, clamped to +-448, E4M3 rounded to
 * nearest even) and compared with xq in code order: two or more steps apart is wrong, one step is counted.
 *   dtype: of x, 0 bf16, 1 fp16, 4 fp32; x (m, k) strides sxm, sxk; xq (mq >= m, k) uint8 codes, strides sqm, sqk;
 *   xs: xs_n fp32 scales, stride sxs (per token: indexed by row).  rows_buf[0] * mult (clamped to m): the step's
 *   real rows (0: nothing judged); stepbuf[0]: the step; mult: input rows per token.
 *   state_row: the layer's 8 int64 counters (calls, wrong scales, scales from outside rows, sampled rows with wrong
 *   values, values one step off, last finding (step & 0x7FFFFFFF) << 32 | kind << 24 | row, worst scale ratio bits,
 *   static scale changed), added to.  workspace: sdc_fp8_quant_check_workspace(m) bytes (used by recipe 1).  No
 *   host synchronisation, no memory set: the call can be captured in a graph. */
int64_t sdc_fp8_quant_check_workspace(int64_t m);
int sdc_fp8_quant_check(int dtype, const void* x, int64_t sxm, int64_t sxk, int64_t m, int64_t k, const uint8_t* xq,
                        int64_t sqm, int64_t sqk, int64_t mq, const float* xs, int64_t xs_n, int64_t sxs, int recipe,
                        const float* scale_ub, const float* static_ref, const int64_t* rows_buf,
                        const int64_t* stepbuf, int64_t mult, int64_t* state_row, void* workspace,
                        int64_t workspace_bytes, hipStream_t stream);

/* ---- the sampled recompute of a fused MoE layer ---------------------------------------------------------------
 * Replaces serve_moe.moe_check_torch / moe_check_triton (serve_moe.py:127-506): when the step in stepbuf[0] (low 32
 * bits; the step's real rows above them, 0 unknown) modulo nlayers is this layer's index, recompute SAMPLES = 2 rows
 * ((step / nlayers * 7919 + j * 104729) % rows) of y = sum_k g_k W2_e (act(W13_e[:I] x) * W13_e[I:] x) with the
 * fused kernel's roundings (dtype: 0 bf16, 1 fp16, of x, out and the weights) and score each output against
 * u |r| + 4u max_k |c_k| + u sqrt(sum_k g_k^2 sum_i (W2_ni h_i)^2) + max |g W2| s + spacing (u, spacing, fmax: the
 * dtype's unit roundoff, subnormal spacing and largest value); also count the known real rows whose expert ids are
 * all or partly -1.  Otherwise nothing is computed.
 *   x, out (m, H) row strides sx, so; gw (m, K) routing weights (gdtype 0 bf16, 1 fp16, 4 fp32); ids (m, K) int32;
 *   w13 (E, 2I, H) strides s13e, s13n; w2 (E, H, I) strides s2e, s2n; n_experts = E; expert_map (map_len entries,
 *   global -> local expert, -1 for another GPU's) or null.  An id that is neither -1 nor in [0, map_len) (no map:
 *   [0, E)), or a map entry outside [-1, E), is never read: its slot adds nothing to the recompute (whose output
 *   then disagrees) and a known real row holding one counts with the rows missing experts.  act 0 SiLU, 1 GELU; routed_first: the routing weight multiplies the first matmul's result.  H <= 8192.
 *   state_row: the layer's 11 int64 (worst keys z << 32 | row, column, output bits, recompute bits, step; active
 *   calls; rows checked; unjudged outputs; real rows unrouted, partly routed; (step << 32) | last such row + 1).
 *   cap_meta (claimed, row, step, z bits), cap_x, cap_y (H floats), cap_ids (K int64), cap_g (K floats): the first
 *   sampled row over `line`.  scores_out: (2, H) fp32 or null.  workspace: sdc_moe_check_workspace(H, I, K) bytes.
 *   No host synchronisation, no memory set. */
int64_t sdc_moe_check_workspace(int64_t H, int64_t I, int64_t K);
int sdc_moe_check(int dtype, const void* x, int64_t sx, const void* out, int64_t so, const void* gw, int gdtype,
                  const int32_t* ids, const void* w13, int64_t s13e, int64_t s13n, const void* w2, int64_t s2e,
                  int64_t s2n, const int32_t* expert_map, int64_t n_experts, int64_t map_len, int64_t m, int64_t H,
                  int64_t I, int64_t K, int act,
                  int routed_first, const int64_t* stepbuf, int64_t nlayers, int64_t index, float u, float spacing,
                  float fmax, float line, int64_t* state_row, int32_t* cap_meta, float* cap_x, float* cap_y,
                  int64_t* cap_ids, float* cap_g, float* scores_out, void* workspace, int64_t workspace_bytes,
                  hipStream_t stream);

/* ---- the MoE router check -------------------------------------------------------------------------------------
 * Replaces serve_route.route_check_torch / route_check_triton (serve_route.py:141-184, the Triton kernel
 * _route_kernel :216-353, its launcher :359-373): when the step in stepbuf[0] (low 32 bits) modulo nlayers is this
 * router's index and rows_buf[0] (the step's real rows, clamped to m) is positive, recompute the routing policy in
 * fp32 for SAMPLES = 2 rows ((step / nlayers * 7919 + j * 104729) % real rows) and judge the router's choice as
 * serve_route.judge does (:91-138): each chosen expert's choice score (softmax, or sigmoid, scores plus the
 * correction bias when there is one) at least the k-th best of the groups surely chosen less the tolerance
 * 1e-6 max(|v|, 1) + 4u |v|, and with groups (DeepSeek's grouped top-k; a group scores its two best choice scores
 * with a bias, its best without; groups within twice the tolerance of the cut may be in or out) also the k-th best of
 * its group and of the groups that may be chosen; the k ids distinct and in [0, E); the weights the chosen experts'
 * scores, renormalized over them when renormalize is set, times scale, to 2e-5 + (1e-4 + 6u) |weight|.  A row whose
 * ids are all -1 is padding and isn't judged.  Otherwise nothing is computed.
 *   logits (m, E) row stride sl, ldt 0 fp32 / 1 bf16 / 2 fp16; weights (m, K) row stride sw, wdt likewise; ids
 *   (m, K) row stride si, idt 0 int32 / 1 int64; bias (E) fp32 or null; groups 0 (plain top-k) or a divisor of E up
 *   to 64 with 0 < topk_group <= groups and topk_group * E / groups >= K; u: 0 for fp32 logits, half the epsilon of
 *   16-bit ones.  E <= 2048, K <= 32.
 *   state_row: the router's 6 int64 (calls judged; rows with a wrong expert set; rows with a wrong weight; the
 *   largest (step & 0x7FFFFFFF) << 32 | kind << 24 | row of a wrong row, kind 2 experts, 1 weights; the worst weight
 *   difference's float bits; rows judged), added to.  cap_meta (taken, row, step, kind, E, ldt), cap_lg (E floats),
 *   cap_ids (K int64), cap_w (K floats): the first wrong row while cap_meta[0] is 0.  No host synchronisation, no
 *   memory set: the call can be captured in a graph. */
int sdc_route_check(const void* logits, int64_t sl, int ldt, const void* weights, int64_t sw, int wdt,
                    const void* ids, int64_t si, int idt, const float* bias, int64_t m, int64_t E, int64_t K,
                    int scoring, int renormalize, int groups, int topk_group, float scale, float u,
                    const int64_t* rows_buf, const int64_t* stepbuf, int64_t nlayers, int64_t index,
                    int64_t* state_row, int64_t* cap_meta, float* cap_lg, int64_t* cap_ids, float* cap_w,
                    hipStream_t stream);

/* ---- both block checksums of one linear layer, one pass over y (no counterpart function in the reference) --------
 * y = x @ W^T (+ bias): the column-block check of sdc_check_static (the serving check, serve.py:301-396) and the
 * row-block check of sdc_matmul_check on the transposed views (W, x^T, y^T, bias[:, None]; checksum.py:435-530),
 * with the same scores, keys and counts, from one read of y.
 *   x (m x k) row stride sxm, W (n x k) row stride swn, y (m x n) row stride sym: bf16 (dtype 0; fp16 returns
 *     SDC_EUNSUPPORTED), k- / n-contiguous; x and y with 16-byte aligned rows and n a multiple of 8 (otherwise
 *     SDC_EUNSUPPORTED: the caller runs the two checks separately).  Blocks are 128 wide.
 *   bias (n) or NULL; parts / spc / block_consts / w_norms: the layer's constants from sdc_layer_constants
 *     (k-contiguous part columns spc elements apart, the (nb, 12) block table, W's row norms [2][n]);
 *     parts_frag: the same parts in fragment order (sdc_parts_fragments, made once per layer), or NULL (then, when
 *     k is a multiple of 256, each call makes them in the workspace); sign_table: the epoch-0 128 x 128 table.
 *   state: int64[4] of the column check (sdc_check_static's row, counts on); row_result: int64[3] of the row check
 *     (sdc_matmul_check's result row; flat index ((column * mb + row block) * 2 + signed), mb = ceil(m / 128)).
 *   workspace: sdc_linear_check_workspace(m, k, n) bytes.
 *   col_scores (m, nb, 2) / row_scores (n, mb, 2): every checksum's score, or NULL.  flags bit 0: run the column
 *     check's GEMM on a side stream, concurrently with the row check's x pass and GEMM. */
int64_t sdc_linear_check_workspace(int64_t m, int64_t k, int64_t n);
/* The layer's three part planes in the fragment order the register-streamed expected-side GEMM reads (no
 * counterpart in the reference; a layout of this library): for depth step s (16 deep), part p and 32-column
 * fragment f, 1024 contiguous bytes, lane l's 16 bytes = part p, column 32 f + l % 32, depths
 * 64 (s / 4) + 32 (l / 32) + 8 (s % 4) .. + 7.  parts as sdc_linear_check's (N = 2 nb columns of pitch spc), k a
 * multiple of 64; out: sdc_parts_fragments_bytes(N, k) bytes, 16-byte aligned. */
int64_t sdc_parts_fragments_bytes(int64_t N, int64_t k);
int sdc_parts_fragments(const void* parts, int64_t spc, int64_t N, int64_t k, void* out, hipStream_t stream);
/* The int8 check's two base-128 digit planes of the block sums (QuantChecksums.parts: [2][N][spc] int8,
 * k-contiguous per column) in the int8 fragment order of the tall-tile GEMM (8 bytes a lane: digit p, column 32 f +
 * l % 32, the same permuted depths as the 16-bit fragments), made once per layer and passed to sdc_quant_check as
 * parts_frag for kind 0.  No counterpart in the reference (its int8 check multiplies unsplit block sums).
 * k a multiple of 64; out: sdc_digit_fragments_bytes(N, k) bytes, 8-byte aligned. */
int64_t sdc_digit_fragments_bytes(int64_t N, int64_t k);
int sdc_digit_fragments(const void* parts, int64_t spc, int64_t N, int64_t k, void* out, hipStream_t stream);
int sdc_linear_check(int dtype, const void* x, int64_t sxm, const void* W, int64_t swn, const void* y, int64_t sym,
                     const void* bias, int64_t m, int64_t k, int64_t n, const void* parts, int64_t spc,
                     const void* parts_frag, const float* block_consts, const float* w_norms, const float* sign_table, int64_t* state,
                     int64_t* row_result, float z, float abs_floor, void* workspace, int64_t workspace_bytes,
                     float* col_scores, float* row_scores, int flags, hipStream_t stream);

/* ---- check of a MoE grouped GEMM ----------------------------------------------------------------------------
 * Replaces guard._grouped_checks (guard.py:102-143) + one checksum._zscores per group for torch._grouped_mm's
 * forward layout: out (rows x n) = A (rows x k, tokens sorted by expert) @ B[g] (k x n) for the rows of group g,
 * offs (groups, int64, on the device) the cumulative group ends.  No host synchronisation: the offsets are read on
 * the device (rows past offs[groups-1] belong to no group and are not checked; empty groups are skipped).
 *   B (groups, k, n): strides sbg, sbk, sbn; A strides (sam, sak); out strides (scm, scn), scn must be 1 or scm
 *   not 1.  bias (n values, stride sbias) shared by every group, or NULL.
 *   results: int64[groups][3], zeroed by the caller: per group the worst checksum's key (bits of z << 32 | flat,
 *   flat = (global row * nb + block) * 2 + signed), the key with its noise, the unjudged count (as
 *   sdc_matmul_check's result row).  workspace: sdc_grouped_check_workspace(groups, rows, k, n, bs) bytes;
 *   scores_out (rows, nb, 2) or NULL. */
int64_t sdc_grouped_check_workspace(int64_t groups, int64_t rows, int64_t k, int64_t n, int64_t bs);
int sdc_grouped_check(int dtype, const void* A, int64_t sam, int64_t sak, const void* B, int64_t sbg, int64_t sbk,
                      int64_t sbn, int64_t groups, const void* C, int64_t scm, int64_t scn, int64_t rows, int64_t k,
                      int64_t n, int64_t bs, const int64_t* offs, const void* bias, int64_t sbias, float z,
                      float abs_floor, const float* sign_table, int64_t* results, void* workspace,
                      int64_t workspace_bytes, float* scores_out, hipStream_t stream);

/* ---- the grouped check's serving form ------------------------------------------------------------------------
 * No counterpart in the reference (its grouped check, guard._grouped_checks, makes every expert's block sums in
 * every call): for served MoE layers, whose expert weights do not change between calls, the B-side constants are
 * made once per layer and each call runs only the expected-side GEMM and the pass over out.
 *   sdc_grouped_constants: from B (groups, k, n; strides sbg, sbk, sbn) and an optional shared bias (n values at
 *     stride sbias), into consts (sdc_grouped_constants_bytes bytes, 256-byte aligned): per expert its block sums'
 *     column norms, maxima and power-of-two scales, each block's largest |B|, the bias's block sums, the three
 *     16-bit parts of the scaled block sums and (depth a multiple of 512) the same parts in the register-streamed
 *     GEMM's fragment order, one set per expert.  workspace: sdc_grouped_constants_workspace bytes of scratch.
 *   sdc_grouped_check_consts: sdc_grouped_check against those constants (has_bias: whether they hold a bias);
 *     the same results and scores.  workspace: sdc_grouped_check_consts_workspace bytes. */
int64_t sdc_grouped_constants_bytes(int64_t groups, int64_t k, int64_t n, int64_t bs);
int64_t sdc_grouped_constants_workspace(int64_t groups, int64_t k, int64_t n, int64_t bs);
int sdc_grouped_constants(int dtype, const void* B, int64_t sbg, int64_t sbk, int64_t sbn, int64_t groups, int64_t k,
                          int64_t n, int64_t bs, const void* bias, int64_t sbias, const float* sign_table,
                          void* consts, int64_t consts_bytes, void* workspace, int64_t workspace_bytes,
                          hipStream_t stream);
int64_t sdc_grouped_check_consts_workspace(int64_t groups, int64_t rows, int64_t k, int64_t n, int64_t bs);
int sdc_grouped_check_consts(int dtype, const void* A, int64_t sam, int64_t sak, const void* consts, int64_t groups,
                             const void* C, int64_t scm, int64_t scn, int64_t rows, int64_t k, int64_t n, int64_t bs,
                             const int64_t* offs, int has_bias, float z, float abs_floor, const float* sign_table,
                             int64_t* results, void* workspace, int64_t workspace_bytes, float* scores_out,
                             hipStream_t stream);

/* ---- per-layer constants of the serving check -------------------------------------------------------------
 * Replaces LayerChecksums._initialize (serve.py:149-211): built on the device from W (n x k, row stride swn, rows
 * k-contiguous) and an optional bias (n values at stride sbias, NULL: none), blocks of bs <= 128 output rows.
 *   parts: the three 16-bit parts (hi, mid, lo) of B2 / scale, B2 = the plain and signed block sums of W's rows
 *     (k x 2nb fp32), as (3 x 2nb) columns of parts_pitch = k rounded up to 8 elements (zero padded), part p of
 *     column c at parts[(p * 2nb + c) * parts_pitch]: the layout sdc_check_static and sdc_linear_check read.
 *   consts_bias, consts_plain: fp32 [nb][12] per block (the scoring pass's table), with and without the bias:
 *     scale (plain, signed), bias block sums (2), |B2 column|_2 (2), max |B2| (2), max |W| of the block,
 *     max |bias| of the block, 0, 0.
 *   row_norms: fp32 [2][n], |w_j|_2^2 then |w_j|_1 of every row j of W (what sdc_linear_check's row-block check
 *     takes as w_norms), or NULL.
 *   sign_table: as sdc_check_static.  workspace: sdc_layer_constants_workspace(n, k, bs) bytes. */
int64_t sdc_layer_constants_workspace(int64_t n, int64_t k, int64_t bs);
int sdc_layer_constants(int dtype, const void* W, int64_t swn, int64_t n, int64_t k, int64_t bs, const void* bias,
                        int64_t sbias, const float* sign_table, void* parts, int64_t parts_pitch, float* consts_bias,
                        float* consts_plain, float* row_norms, void* workspace, int64_t workspace_bytes,
                        hipStream_t stream);

/* ---- check of one quantized GEMM ----------------------------------------------------------------------------
 * Replaces modes.judge (modes.py:231-291) for its int8 and fp8 branches, on the device, and extends the fp8 one to
 * per-row activation scales sa and per-column weight scales sb (C = sa_i sb_j sum_k Aq[i,k] Bq[k,j]).
 *   kind 0 = int8 W8A8: A (m x k) int8, C (m x n) int32 (c_dtype 2); parts = the block sums of B (plain, then
 *     signed, per block) as two base-128 int8 digits, hi then lo, (2 x 2nb) columns of k bytes at spc bytes apart
 *     (B2 = 128 hi + lo, |lo| <= 64).  The check is exact: every differing sum is a wrong block.  Any depth, stride
 *     and address: an odd k, odd sam / spc or odd addresses are copied into zero-padded workspace buffers first.
 *   kind 1 = fp8 e4m3: A (m x k) fp8 e4m3fn (k-contiguous rows, any row stride and alignment: rows that are not
 *     16-byte aligned or a depth that is not a multiple of 32 take bounds-checked loads), sa (m) fp32 or NULL (1),
 *     C fp32 (c_dtype 0) or
 *     bf16 (1); parts = the three bf16 parts of B2s = sum_j w_j sb_j Bq[:,j] per checksum column (3 x 2nb columns
 *     of k elements, spc apart); bfrob (nb) = |sb Bq|_F per block; bcol (n) = |sb_j Bq[:,j]|_2 per column;
 *     unit = the accumulation's rounding unit (2^-14 for an fp8 tensor-core accumulation of unknown precision,
 *     modes.acc_unit), nfma = products per accumulation step (16, modes.n_fma; 0: none).
 *   A row stride sam, C strides (scm, scn), in elements (any C layout: the row-block check passes C^T, strides
 *     (1, m)).  sign_table: as sdc_check_static (epoch 0).
 *   result: int64[4], zeroed by the caller: the worst block's key (bits of z << 32 | row * nb + block), the key with
 *     its noise, the number of wrong blocks (z > z; int8: any differing sum), blocks with a non-finite sum.
 *   parts_frag: the parts in the tall-tile GEMM's order -- fp8: sdc_parts_fragments', int8: sdc_digit_fragments'
 *     -- made once with the weight's constants, or NULL (the library makes them in the workspace when the GEMM
 *     takes them: depth a multiple of 1024).
 *   workspace: at least sdc_quant_check_workspace(kind, m, k, n, bs) bytes; scores_out: (m, nb) z or NULL. */
int64_t sdc_quant_check_workspace(int kind, int64_t m, int64_t k, int64_t n, int64_t bs);
int sdc_quant_check(int kind, const void* A, int64_t sam, const void* parts, int64_t spc,
                    const void* parts_frag, const float* sa,
                    const void* C, int64_t scm, int64_t scn, int c_dtype, int64_t m, int64_t k, int64_t n, int64_t bs,
                    const float* sign_table, const float* bfrob, const float* bcol, float unit, float nfma, float z,
                    int64_t* result, void* workspace, int64_t workspace_bytes, float* scores_out, hipStream_t stream);

/* Depth split the expected-side GEMM uses for an (m x k) @ (k x ncols) product (sizes the workspace). */
int64_t sdc_expected_splits(int64_t m, int64_t k, int64_t ncols);

/* ---- integer fingerprints --------------------------------------------------------------------------------
 * sdc_fingerprint3: out[0..2] += recompute.fingerprint's three sums (recompute.py:72-116; the Triton kernel
 *   _fingerprint.py:51-65 / fingerprint_bits :128-130) of n words of word_bytes (2: int16, 1: int8) bytes,
 *   word positions numbered from `start`.  out must be zeroed by the caller for a fresh fingerprint.
 * sdc_fingerprint2: out[0..1] += serve_weights.fingerprint's two sums (serve_weights.py:172-185; kernel
 *   :194-204) of n words; kind 0 = int16, 1 = int32, 2 = uint8 (serve_weights._int_view :151-161). */
int sdc_fingerprint3(const void* bits, int64_t n, int word_bytes, int64_t start, int64_t* out, hipStream_t stream);
int sdc_fingerprint2(const void* bits, int64_t n, int kind, int64_t* out, hipStream_t stream);

/* ---- paged-KV block fingerprints (no counterpart function in the reference; each block's value is
 * recompute.fingerprint of the block's bytes as a tensor of its own, recompute.py:72-116, words numbered from 0) --
 * out[i][0..2] (int64, zeroed by the caller) += the fingerprint of block ids[i] of a cache of nblocks blocks of
 * `words` words each, block b at cache + b * block_bytes; word_bytes 2: int16 words (16-bit and wider element
 * dtypes), 1: int8 words (1-byte element dtypes such as fp8 caches, recompute.py:86-87); ids == NULL: entry i is
 * block i (n = nblocks).  An entry whose id is negative or >= nblocks is left unchanged (a block-table walk passes
 * the table's rows).  Blocks of whole 128-byte chunks (words * word_bytes a multiple of 128, at most 65536; cache
 * and block_bytes 16-byte aligned) run on the int8 matrix cores against a 2 MB weight table per word size held in
 * static device memory: the first such call on a device builds it and waits for it (a call made while the stream
 * is captured, before that, takes the vector kernel instead, with the same result). */
int sdc_kv_fingerprint(const void* cache, int64_t nblocks, int64_t block_bytes, int64_t words, int word_bytes,
                       const int64_t* ids, int64_t n, int64_t* out, hipStream_t stream);

/* ---- sampled attention recompute from a paged KV cache, and the sampled tokens' KV-write check ------------
 * Replaces serve_attn.attn_check_triton (serve_attn.py:574-602) and its two kernels _attn_part / _attn_judge
 * (:335-571); the arithmetic of attn_check_torch (:165-280).  One launch, no host synchronisation.
 *   q, o (T, Hq, D): element strides (sqt, sqh), last dimension contiguous; dtype 0 = bf16, 1 = fp16 (the KV
 *     cache, key and val are of the same dtype).
 *   kv (NB, Hkv, N, 2D): K in [.., :D], V in [.., D:2D], element strides (skb, skh, skn, skd).
 *   key, val (T, Hkv, D): the keys and values the layer wrote this call, strides (skt, skh2), (svt, svh), last
 *     dimension contiguous; slots (SN,) int64: vLLM's slot_mapping.  Only read when has_write != 0.
 *   qsl (R + 1) int32 query_start_loc, seq_lens (R) int32, bt (R, W) int32 block table with row stride sbt.
 *   state: the layer's 18-column int64 row (serve_attn.py:87-89) at state + slot * 18; ctrl int64[2] =
 *     (step, active): the call checks only when active != 0 and step % nl == idx.
 *   capm (slots, 12) int32, capq / capo (slots, capw) fp32: the capture of the first sample over `line`; capkv
 *     (caprows, 2, capw) in the cache's dtype + capkvm int32[4]: the keys and values it attended (keep_kv), or NULL.
 *   samples: (token, head) pairs recomputed per call, 1..1024 (SAMPLES = 4 in the reference; more reuse its
 *     picking rule).
 *   workspace: sdc_attn_check_workspace(samples, W * N, D) bytes, ZEROED before its first use: its first 4 KiB
 *     hold per-sample counters at fixed places, which every call leaves at zero again, so one buffer serves calls
 *     of any sample count and context length; may be NULL when sdc_attn_splits(samples, W * N) == 1.  Calls that
 *     share a workspace must not overlap (one stream).
 *   scores_out (may be NULL): each judged sample's per-dimension scores, (samples, D) fp32 (tests). */
int64_t sdc_attn_splits(int64_t samples, int64_t max_keys);
int64_t sdc_attn_check_workspace(int64_t samples, int64_t max_keys, int64_t head_size);
int sdc_attn_check(int dtype, const void* q, int64_t sqt, int64_t sqh, const void* o, int64_t sot, int64_t soh,
                   int64_t T, int64_t Hq, int64_t D, const void* kv, int64_t skb, int64_t skh, int64_t skn,
                   int64_t skd, int64_t NB, int64_t Hkv, int64_t N, const void* key, int64_t skt, int64_t skh2,
                   const void* val, int64_t svt, int64_t svh, const int32_t* qsl, const int32_t* seq_lens, int64_t R,
                   const int32_t* bt, int64_t sbt, int64_t W, const int64_t* slots, int64_t SN, int64_t* state,
                   int64_t slot, const int64_t* ctrl, int64_t nl, int64_t idx, float scale, int64_t left, float line,
                   int32_t* capm, float* capq, float* capo, int64_t capw, void* capkv, int32_t* capkvm,
                   int64_t caprows, int samples, void* workspace, int64_t workspace_bytes, int has_write,
                   int keep_kv, float* scores_out, hipStream_t stream);

/* sdc_attn_check without a workspace argument: it allocates nothing.  No counterpart in the reference; it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments and results as sdc_attn_check minus workspace / workspace_bytes.  Its workspace
 * is a static device array of SDC_ATTN_SCRATCH_BYTES per GPU, held from the first call on that GPU (which must be
 * the current device) until the process ends; a call that would need more returns SDC_EWORKSPACE (none does within
 * the limits above: samples x splits <= 1024, head size <= 256).  All calls on one GPU share that array: calls
 * that overlap in time on one GPU (several streams or host threads) race and must not be made. */
#define SDC_ATTN_SCRATCH_BYTES 4456448
int sdc_attn_check_noalloc(int dtype, const void* q, int64_t sqt, int64_t sqh, const void* o, int64_t sot,
                           int64_t soh, int64_t T, int64_t Hq, int64_t D, const void* kv, int64_t skb, int64_t skh,
                           int64_t skn, int64_t skd, int64_t NB, int64_t Hkv, int64_t N, const void* key, int64_t skt,
                           int64_t skh2, const void* val, int64_t svt, int64_t svh, const int32_t* qsl,
                           const int32_t* seq_lens, int64_t R, const int32_t* bt, int64_t sbt, int64_t W,
                           const int64_t* slots, int64_t SN, int64_t* state, int64_t slot, const int64_t* ctrl,
                           int64_t nl, int64_t idx, float scale, int64_t left, float line, int32_t* capm,
                           float* capq, float* capo, int64_t capw, void* capkv, int32_t* capkvm, int64_t caprows,
                           int samples, int has_write, int keep_kv, float* scores_out, hipStream_t stream);

/* ---- per-kernel timing (no counterpart in the reference; for benchmarks) ------------------------------------
 * With profiling on, every kernel launch is bracketed by two HIP events on its stream; sdc_profile_read waits for
 * them and sums the durations of one kernel: "expected_gemm" (serving GEMM), "serve_fused", "serve_sums",
 * "serve_score", "b_stage", "b_finish", "split", "train_gemm", "train_score" (also the grouped check's),
 * "col_gemm", "xstage", "xfinish", "row_gemm", "ypass" (sdc_linear_check), "quant_gemm_i8", "quant_gemm_fp8",
 * "quant_score_i8", "quant_score_fp8", "fingerprint3", "fingerprint2", "kv_fingerprint", "attn_check", "acc_bsums",
 * "acc_finish", "acc_anorm", "acc_gemm", "acc_score" (sdc_matmul_check_acc, sdc_matmul_check_acc_stats),
 * "fused_pack", "fused_side", "fused_mm", "fused_mm_checked" (sdc_fused_mm, sdc_fused_mm_checked), "fp8q_amax",
 * "fp8q_judge" (sdc_fp8_quant_check), "moe_up", "moe_act", "moe_down", "moe_compare" (sdc_moe_check), "route_check" (sdc_route_check). */
int sdc_profile_enable(int on);
int sdc_profile_reset(void);
int sdc_profile_read(const char* name, double* total_ms, int64_t* launches);

/* Name of the HIP error behind the last SDC_ELAUNCH returned to the calling thread. */
const char* sdc_last_error(void);

/* ---- self-tests ---------------------------------------------------------------------------------------------
 * No counterpart in the reference: checks the MFMA operand layout the GEMM kernels assume.
 * C (32 x 32 fp32) = A (32 x 16 bf16, row-major) @ B (16 x 32 bf16, column-major), one wave. */
int sdc_mfma_layout_selftest(const void* A, const void* B, float* C, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* SDCGUARD_HIP_H */
