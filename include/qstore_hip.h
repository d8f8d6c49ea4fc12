/*
 * qstore_hip.h -- C ABI of the MI355X (gfx950) QStore quantized-weight hot path.
 *
 * Every entry point takes raw device pointers, element counts / leading dimensions
 * (in elements) and a hipStream_t (passed as void*), enqueues its kernels on that
 * stream and returns a qs_status.  Nothing here allocates device memory unless the
 * comment says so, nothing synchronises the stream, and no C++ exception crosses the
 * boundary.  On a non-zero return, qs_last_error() holds a message for the calling
 * thread.
 *
 * Numerical contracts follow the reference (JHollenb/mrun-pub); the file:line cited
 * on each declaration is the reference interface that entry point replaces.
 */
#ifndef QSTORE_HIP_H_
#define QSTORE_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status / dtype codes ------------------------------------------------------- */
enum qs_status {
  QS_OK = 0,
  QS_ERR_INVALID = -1,     /* bad shape / pointer / argument  -> ValueError     */
  QS_ERR_UNSUPPORTED = -2, /* well-formed but not implemented -> RuntimeError   */
  QS_ERR_HIP = -3,         /* HIP runtime error               -> RuntimeError   */
  QS_ERR_LIMIT = -4        /* exceeds a documented maximum    -> ValueError     */
};

enum qs_dtype { QS_F32 = 0, QS_BF16 = 1, QS_F16 = 2, QS_I32 = 3, QS_I64 = 4 };

/* Library version (major*10000 + minor*100 + patch). */
int qs_version(void);
/* Message of the last failed call on this thread ("" when none). */
const char* qs_last_error(void);

/* ---- int8 row-scaled ("qrow") linears --------------------------------------------
 * codes: int8 [N, K] row-major, scales: fp32 [N].  Dequantized weight
 * W[n,k] = float(codes[n,k]) * scales[n] (one IEEE fp32 multiply).               */

/* Replaces _dequant_qrow (src/mrun/engine/kernels/qstore.py:385-399) and the device
 * dequant of QStore.weight (qstore.py:1057, 1066-1071, 1076-1077):
 * out[n,k] = cast_out_dtype(float(codes[n,k]) * scales[n]), out_dtype F32/BF16/F16
 * (BF16/F16 by round-to-nearest-even of the fp32 product). ld_out in elements. */
int qs_qrow_dequant(const int8_t* codes, const float* scales, void* out, int out_dtype,
                    int64_t N, int64_t K, int64_t ld_out, void* stream);

/* Replaces the qrow branch of QStore.embed_rows (src/mrun/engine/kernels/qstore.py:1099-1128):
 * out[i, k] = float(codes[rows[i], k]) * scales[rows[i]] in fp32 for i < n_rows; rows int64
 * device indices in [0, N) (an index outside that range yields a zero row, never a read). */
int qs_qrow_dequant_rows(const int8_t* codes, const float* scales, int64_t N, int64_t K,
                         const int64_t* rows, int64_t n_rows, float* out, void* stream);

/* Replaces QStore.matmul (qstore.py:1082-1092), fused_qrow_matmul +
 * _qrow_w8a16_kernel (src/mrun/engine/kernels/dense_qstore_cuda.py:1105-1153, 467-512)
 * and dequantized_reference_matmul (dense_qstore_cuda.py:1003-1013):
 *   y[M,N] = x[M,K] @ W^T.
 *   x_dtype F32 : W in fp32, fp32 accumulate, y F32 (QStore fp32 compute contract).
 *   x_dtype BF16: W rounded to bf16 per element, fp32 accumulate, y BF16 (W8A16).
 *   x_dtype F16 : W rounded to fp16 per element, fp32 accumulate, y F16.
 * M <= 2 (decode) and fp32 use a VALU kernel, larger M an MFMA kernel; results agree
 * within the fp32-accumulation tolerance but are not bitwise batch invariant. */
int qs_qrow_matmul(const void* x, int x_dtype, int64_t ldx, const int8_t* codes,
                   const float* scales, void* y, int64_t ldy, int64_t M, int64_t N,
                   int64_t K, void* stream);

/* Replaces QStore.matmul_row_stable / _row_stable_loaded_matmul (qstore.py:49-76,
 * 1094-1097): same contract as qs_qrow_matmul, and every output row is reduced in one
 * fixed order whatever M is, so row b equals the M = 1 result for x[b] bit for bit. */
int qs_qrow_matmul_row_stable(const void* x, int x_dtype, int64_t ldx, const int8_t* codes,
                              const float* scales, void* y, int64_t ldy, int64_t M, int64_t N,
                              int64_t K, void* stream);

/* Several qrow linears sharing one activation x (e.g. q/k/v projections,
 * src/mrun/engine/kernels/paged_forward.py:481-490) in one launch; same contract as
 * qs_qrow_matmul for each linear i: y_i[M,N_i] = x @ W_i^T. n_linear <= 4. */
int qs_qrow_matmul_multi(const void* x, int x_dtype, int64_t ldx, int n_linear,
                         const int8_t* const* codes, const float* const* scales,
                         void* const* y, const int64_t* ldy, const int64_t* N, int64_t M,
                         int64_t K, void* stream);

/* Batched decode (M rows of bf16/f16 activations, 1 <= M <= 32), same contracts as
 * qs_qrow_matmul_multi (W8A16, y in the activation dtype) and qs_qrow_swiglu (x, y BF16),
 * for the reference's batched decode through fused_qrow_matmul / fused_qrow_swiglu
 * (dense_qstore_cuda.py:1105-1153, 1053-1102).  K % 128 == 0, K <= 16384, otherwise
 * QS_ERR_UNSUPPORTED; weight and activation rows 16-byte aligned; a K split (rows longer
 * than 2048) needs every N % 4 == 0.  The K order of every sum (waves per slice, slices)
 * is chosen from (N, K) only and the slices' fp32 partial sums are added in slice order,
 * so every row equals the same row computed alone (M = 1 through this entry point) bit
 * for bit.
 *   workspace: qs_qrow_batched_workspace_bytes(M, n_linear, N, K, swiglu) bytes, 16-byte
 *              aligned (0 when K is not split), contents clobbered; calls that run
 *              concurrently (other streams) need their own. */
size_t qs_qrow_batched_workspace_bytes(int64_t M, int n_linear, const int64_t* N, int64_t K,
                                       int swiglu);
int qs_qrow_matmul_batched(const void* x, int x_dtype, int64_t ldx, int n_linear,
                           const int8_t* const* codes, const float* const* scales,
                           void* const* y, const int64_t* ldy, const int64_t* N, int64_t M,
                           int64_t K, void* workspace, size_t workspace_bytes, void* stream);
int qs_qrow_swiglu_batched(const void* x, int64_t ldx, const int8_t* gate_codes,
                           const float* gate_scales, const int8_t* up_codes,
                           const float* up_scales, void* y, int64_t ldy, int64_t M, int64_t N,
                           int64_t K, void* workspace, size_t workspace_bytes, void* stream);

/* Replaces fused_qrow_swiglu + _qrow_w8a16_paired_swiglu_kernel
 * (dense_qstore_cuda.py:1053-1102, 515-575); reference contract
 * fused_qrow_swiglu_reference (dense_qstore_cuda.py:1037-1050):
 *   g = bf16(x @ Wg^T), u = bf16(x @ Wu^T) (W8A16 each),
 *   y = bf16( float(bf16(g * sigmoid(g))) * float(u) ).  x, y BF16. */
int qs_qrow_swiglu(const void* x, int64_t ldx, const int8_t* gate_codes,
                   const float* gate_scales, const int8_t* up_codes, const float* up_scales,
                   void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* stream);

/* Replaces fused_qrow_top2 / _qrow_w8a16_block_top2_kernel / _reduce_top2_blocks_kernel
 * (src/mrun/engine/kernels/dense_qstore_cuda.py:578-674, 1239-1317): the two best rows of
 * the first row_count rows of a head page for every activation row, with no logits in
 * memory.  Logits follow qs_qrow_matmul's weight contract (W8A16 for BF16/F16 x, fp32 for
 * F32 x) with fp32 sums.  out_indices[m][0..1] (int32) = start_row + row, out_values[m][0..1]
 * the logits: the first is the largest (lowest index on ties), the second the largest of
 * the other rows.  workspace: qs_qrow_top2_workspace_bytes(M, row_count) bytes of device
 * memory for the per-block candidates.  row_count >= 2. */
size_t qs_qrow_top2_workspace_bytes(int64_t M, int64_t row_count);
int qs_qrow_top2(const void* x, int x_dtype, int64_t ldx, const int8_t* codes, const float* scales,
                 int64_t M, int64_t row_count, int64_t K, int64_t start_row, void* workspace,
                 size_t workspace_bytes, int32_t* out_indices, float* out_values, void* stream);

/* No counterpart in the reference.  qs_qrow_top2 without the workspace argument, for
 * callers that cannot allocate device memory (code under HIP graph capture, tight decode
 * serving loops, harnesses that forbid hipMalloc).  Same contract and results as
 * qs_qrow_top2; the candidates live in a per-device scratch array of
 * QS_TOP2_SCRATCH_BYTES bytes held by the library until the process ends, so the call
 * allocates nothing.  Sizes whose qs_qrow_top2_workspace_bytes(M, row_count) exceeds
 * that array are rejected with QS_ERR_LIMIT (about 6 activation rows of a 151,936-row
 * head).  Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (two streams, two threads) race and must be serialised by the caller. */
#define QS_TOP2_SCRATCH_BYTES (4 << 20)
int qs_qrow_top2_noalloc(const void* x, int x_dtype, int64_t ldx, const int8_t* codes,
                         const float* scales, int64_t M, int64_t row_count, int64_t K,
                         int64_t start_row, int32_t* out_indices, float* out_values,
                         void* stream);

/* Replaces _rerank_qrow_candidates_fp32 (dense_qstore_cuda.py:1189-1236): candidates[m][c]
 * (int64 global rows, 1 <= C <= 16) scored as sum_k float(x[m][k]) * (float(code) * scale)
 * in fp32; out_indices[m] (int64) is the best candidate (lowest index on ties) and
 * out_values[m] its score.  A candidate outside [start_row, start_row + page_rows) scores
 * -inf. */
int qs_qrow_rerank_fp32(const void* x, int x_dtype, int64_t ldx, const int8_t* codes,
                        const float* scales, int64_t page_rows, int64_t K, int64_t start_row,
                        const int64_t* candidates, int C, int64_t M, int64_t* out_indices,
                        float* out_values, void* stream);

/* ---- W8A8 (int8 weights x per-token int8 activations) ------------------------------ */

/* Activation quantizer of w8a8_matmul (src/mrun/engine/kernels/w8a8.py:118-121):
 * per row m, v = x*keep (keep nullable, fp32 [K]); s[m] = max|v|/127 (0 -> 1);
 * q[m,k] = clamp(round_half_even(v/s[m]), -127, 127).  IEEE fp32 ops, bit-exact. */
int qs_act_quant_i8(const void* x, int x_dtype, int64_t ldx, const float* keep, int8_t* q,
                    float* scale, int64_t M, int64_t K, void* stream);

/* Outlier column selection of w8a8_matmul (w8a8.py:98-102): colmax[k] = max_m |x[m,k]|,
 * idx = the k largest (1 <= k <= 64, ties -> lower column), keep = 1 except 0 at idx.
 * colmax is caller-provided workspace of K floats and holds the column maxima on return. */
int qs_outlier_topk(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int k,
                    float* colmax, int64_t* idx, float* keep, void* stream);

/* Operands of the exact fp32 side path (w8a8.py:108-112): xp[m,p] = float(x[m, idx[p]]),
 * wp[n,p] = float(qw[n, idx[p]]) * sw[n]; 1 <= P <= 64. */
int qs_w8a8_side_gather(const void* x, int x_dtype, int64_t ldx, const int8_t* qw,
                        const float* sw, const int64_t* idx, int P, int64_t M, int64_t N,
                        int64_t K, float* xp, float* wp, void* stream);

/* The protect_k front end of w8a8_matmul (w8a8.py:92-121) in two launches: the column
 * maxima of x, then one kernel in which every workgroup selects the k outlier columns
 * exactly as qs_outlier_topk does, quantizes its rows as qs_act_quant_i8 does with those
 * columns' keep factor 0, and writes its share of the side operands exactly as
 * qs_w8a8_side_gather does.  Bit for bit the outputs of those three entry points.
 * 1 <= k <= 16, k <= K; K <= 8192 with K % 8 == 0 (f32: K <= 4096, K % 4 == 0); x rows
 * 16-byte aligned.  colmax_ws: ceil(M / 1024) * K floats of workspace, 16-byte aligned (keep too).  q [M, K] int8,
 * act_scale [M], xp [M, k], wp [N, k]; idx [k] and keep [K] are optional (null: not
 * written). */
int qs_w8a8_protect_quant(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int k,
                          const int8_t* qw, const float* sw, int64_t N, float* colmax_ws,
                          int8_t* q, float* act_scale, float* xp, float* wp, int64_t* idx,
                          float* keep, void* stream);

/* Replaces _int8_gemm / torch._int_mm (w8a8.py:33-64): acc[M,N] = qx[M,K] . qw[N,K]^T,
 * exact int32 accumulation (v_mfma_i32_32x32x32_i8). */
int qs_gemm_i8i8_i32(const int8_t* qx, const int8_t* qw, int32_t* acc, int64_t M, int64_t N,
                     int64_t K, void* stream);

/* GEMM + epilogue of w8a8_matmul (w8a8.py:123-125):
 * y[m,n] = side[m,n] + (float(acc[m,n]) * act_scale[m]) * w_scale[n], with
 * side[m,n] = sum_p side_x[m,p] * side_w[n,p] (P = 0: no side path, y is the bare
 * product bit for bit); y_dtype F32 or BF16 (RNE of the fp32 value). */
int qs_w8a8_gemm(const int8_t* qx, const float* act_scale, const int8_t* qw,
                 const float* w_scale, const float* side_x, const float* side_w, int P, void* y,
                 int y_dtype, int64_t M, int64_t N, int64_t K, void* stream);

/* ---- routed MoE ---------------------------------------------------------------------- */

/* Router of Qwen3MoeDecodeRuntime.forward (src/mrun/engine/qwen3_moe_cuda.py:3702-3707):
 * p = softmax(float(logits[t])), top-k (ties -> lower expert), optional renormalisation
 * by the kept sum, weights stored as F32 or BF16.  E <= 1024, k <= 16. */
int qs_moe_router(const void* logits, int logit_dtype, int64_t T, int E, int k, int norm_topk,
                  int64_t* top_idx, void* top_w, int w_dtype, void* stream);

/* Replaces grouped_route_tensors(_with_inverse) / _triton_route_{count,prefix,scatter}
 * (src/mrun/engine/olmoe_cuda.py:989-1135, 131-182): expert-major queue of the T*k
 * assignments in STABLE order (identical to the reference's CPU stable argsort):
 * token_ids[q] = a / k, coef[q] = float(top_w[a]), counts[e], starts[e] (exclusive
 * prefix), inverse[a] = q (nullable).  Expert ids must lie in [0, E); E <= 512.  An
 * assignment whose expert lies outside [0, E) is left out of the queue: it counts for no
 * expert, its inverse entry is -1, and the queue rows past sum(counts) hold token 0 with
 * coefficient 0, so no consumer reads an unwritten index. */
int qs_moe_route(const void* top_idx, int idx_dtype, const void* top_w, int w_dtype, int64_t T,
                 int k, int E, int64_t* token_ids, float* coef, int32_t* starts, int32_t* counts,
                 int64_t* inverse, void* stream);

/* qs_moe_route plus the W8A8 per-token quantization of the T source rows
 * (quantize_fp8_activation olmoe_cuda.py:1173-1176 with the int8 recipe of
 * w8a8.py:118-121, applied before the gather of FP8ExpertBackend.moe :1340-1345):
 * q[t] / scale[t] = the codes and scale of source row t, unpermuted, in the same launch as
 * the route when E * T * k <= 2^22 and the rows are 16-byte aligned with H % 8 == 0
 * (otherwise two launches).  A row's codes do not depend on its expert, so
 * qs_moe_grouped_gemm_i8_rows(q, scale, token_ids, ...) multiplies exactly the rows
 * qs_moe_gather_quant(source, token_ids) would produce. */
int qs_moe_route_quant(const void* top_idx, int idx_dtype, const void* top_w, int w_dtype, int64_t T,
                       int k, int E, int64_t* token_ids, float* coef, int32_t* starts, int32_t* counts,
                       int64_t* inverse, const void* source, int src_dtype, int64_t ld_src, int64_t H,
                       int8_t* q, float* scale, void* stream);

/* Replaces build_expert_queue / build_expert_queue_flat / build_expert_queue_device
 * (src/mrun/engine/kernels/expert_queue.py:242-470): compiles A router packets into
 * expert-major ranges in STABLE order (equal to the reference's CPU argsort(stable=True)).
 * Dense form (tokens = slots = nullptr, A = rows * top_k): packet a is route slot a % top_k of
 * row a / top_k.  Flat form: tokens[a], slots[a] given.  experts I32/I64 [A], weights
 * F32/BF16/F16 [A] (stored as fp32 coefficients), row_epochs / row_deadlines int64 [rows].
 * Outputs (queue order): token_ids, expert_ids, route_slots, coefficients, epochs and
 * deadlines (of the packet's row) [A]; starts / counts [E] as I32 or I64 (count_dtype).  A
 * packet whose expert lies outside [0, E) is left out (the host validates first where the
 * reference does); the rows it frees at the end hold token 0, expert -1, slot -1, epoch
 * INT64_MIN.  E <= 512. */
int qs_expert_queue_build(const void* experts, int expert_dtype, const int64_t* tokens,
                          const int64_t* slots, const void* weights, int weight_dtype,
                          const int64_t* row_epochs, const int64_t* row_deadlines, int64_t A,
                          int top_k, int64_t rows, int E, int64_t* token_ids, int64_t* expert_ids,
                          int64_t* route_slots, float* coefficients, int64_t* epochs,
                          int64_t* deadlines, void* starts, void* counts, int count_dtype,
                          void* stream);

/* Replaces scatter_committed / scatter_committed_device (expert_queue.py:487-560):
 * valid[q] = (token_ids[q] in [0, rows) and epochs[q] == active_epochs[token_ids[q]])
 * (uint8), and for every row t reduced[t, h] = sum over the valid packets of token t, in
 * ascending queue order, of fp32(float(expert_out[q, h]) * coefficients[q]), accumulated
 * from 0 in that order (the order and roundings of the reference's index_add_; packets are
 * matched to rows by token alone, as there; no atomics in the sum, same bits on every
 * call).  workspace: qs_expert_queue_scatter_workspace_bytes(rows, A) bytes.  A, rows and
 * H below 2^31. */
size_t qs_expert_queue_scatter_workspace_bytes(int64_t rows, int64_t A);
int qs_expert_queue_scatter(const int64_t* token_ids, const float* coefficients, const int64_t* epochs,
                            const int64_t* active_epochs, const void* expert_out, int out_dtype,
                            int64_t ld_out, int64_t A, int64_t rows, int64_t H, void* workspace,
                            size_t workspace_bytes, float* reduced, uint8_t* valid, void* stream);

/* Routed-row quantization (int8 analogue of quantize_fp8_activation,
 * olmoe_cuda.py:1173-1176, with the W8A8 recipe of w8a8.py:118-121):
 * row a of the output is source[rows[a]] (rows nullable = identity). */
int qs_moe_gather_quant(const void* source, int src_dtype, int64_t ld_src, const int64_t* rows,
                        int64_t A, int64_t H, int8_t* q, float* scale, void* stream);

/* Replaces grouped_fp8_mm(_strided) / _grouped_fp8_strided_kernel / grouped_w4_mm_strided
 * (olmoe_cuda.py:1197-1252, qwen3_moe_cuda.py:1910-2470) for int8 experts: for every
 * group g with rows [starts[g], starts[g]+counts[g]) and weights
 * w + slot(g)*w_stride ([N_w, K] int8 rows; slot(g) = slots ? slots[g] : g):
 *   out[row, n] = (float(acc) * a_scale[row]) * w_scale[slot(g)*ws_stride + n]
 * (F32/BF16); swiglu != 0: N_w = 2N, out[row, n] = bf16(bf16(silu(bf16(gate))) * bf16(up))
 * with gate from weight row n and up from row n + N.  K % 64 == 0, K <= 8192 with SwiGLU,
 * K <= 16384 without.  max_rows is the reference's max_rows argument
 * (qwen3_moe_cuda.py:2257-2310, callers pass the routed row count, :2747): a bound on
 * counts[g] used only to size the row tile (0 = unknown); results do not depend on it. */
int qs_moe_grouped_gemm_i8(const int8_t* a, const float* a_scale, const int8_t* w,
                           int64_t w_stride, const float* w_scale, int64_t ws_stride,
                           const int32_t* starts, const int32_t* counts, const int32_t* slots,
                           int G, int64_t N, int64_t K, int64_t max_rows, int swiglu, void* out,
                           int out_dtype, void* stream);

/* qs_moe_grouped_gemm_i8 whose queue row r reads a[row_ids[r]] and a_scale[row_ids[r]]
 * (the gather source.index_select(0, token_ids) of FP8ExpertBackend.moe, olmoe_cuda.py:
 * 1340-1345, folded into the kernel's staging; ids outside [0, src_rows) read zero rows).
 * Needs the streaming kernel: 16 staged rows of K + 28 bytes must fit 144 KiB of LDS. */
int qs_moe_grouped_gemm_i8_rows(const int8_t* a, const float* a_scale, const int64_t* row_ids,
                                int64_t src_rows, const int8_t* w, int64_t w_stride, const float* w_scale,
                                int64_t ws_stride, const int32_t* starts, const int32_t* counts,
                                const int32_t* slots, int G, int64_t N, int64_t K, int64_t max_rows,
                                int swiglu, void* out, int out_dtype, void* stream);

/* Replaces grouped_bf16_mm / _grouped_bf16_kernel (qwen3_moe_cuda.py:2473-2510, 2117-2157)
 * as used by PackedBF16ExpertBackend.moe (:2978-3046), over int8 expert pages (the weight-
 * only W8A16 grouped variant): for every group g with rows [starts[g], starts[g]+counts[g])
 * and weights w + slot(g)*w_stride ([N_w, K] int8 rows, scales w_scale + slot(g)*ws_stride):
 *   out[row, n] = sum_k float(x[row, k]) * float(bf16(float(code[n, k]) * w_scale[n]))
 * (fp32 accumulate, F32 or BF16 out), x bf16.  row_ids nullable: x[row] is source row
 * row_ids[row] of a (the reference's source.index_select(0, token_ids)); ids outside
 * [0, src_rows) read zeros.  swiglu != 0: N_w = 2N, out = bf16(bf16(silu(bf16(gate))) *
 * bf16(up)) with gate from weight row n and up from row n + N (the reference's
 * F.silu(gate) * up on bf16 halves).  K % 64 == 0; max_rows as qs_moe_grouped_gemm_i8. */
int qs_moe_grouped_gemm_w8a16(const void* a, const int64_t* row_ids, int64_t src_rows,
                              const int8_t* w, int64_t w_stride, const float* w_scale,
                              int64_t ws_stride, const int32_t* starts, const int32_t* counts,
                              const int32_t* slots, int G, int64_t N, int64_t K, int64_t max_rows,
                              int swiglu, void* out, int out_dtype, void* stream);

/* Replaces stable_route_reduce / _stable_route_reduce_kernel (qwen3_moe_cuda.py:2561-2664,
 * 2160-2182): out[t, h] = sum over rank r = 0..k-1 (in order) of
 * float(y[inverse[t*k+r], h]) * coef[inverse[t*k+r]], each product rounded to fp32.  A
 * negative inverse entry (a rank qs_moe_route dropped) contributes 0. */
int qs_moe_route_reduce(const void* expert_out, int y_dtype, const float* coef,
                        const int64_t* inverse, int64_t T, int k, int64_t H, float* out,
                        void* stream);

/* qs_moe_route_reduce with the output in out_dtype (QS_F32 or QS_BF16): BF16 rounds each
 * fp32 sum once (RNE), the value of the reference's fp32 reduce followed by its cast to
 * the model dtype (qwen3_moe_cuda.py:2910-2918 then :2936, output.to(self.dtype)). */
int qs_moe_route_reduce_to(const void* expert_out, int y_dtype, const float* coef,
                           const int64_t* inverse, int64_t T, int k, int64_t H, void* out,
                           int out_dtype, void* stream);

/* ---- packed int3 / int2 ("qrow3" / "qrow2") --------------------------------------------
 * packed: uint8 [N, row_bytes], each row an LSB-first bitstream of K codes of `bits` bits
 * (code k at bits [bits*k, bits*k + bits)); scales [N, ceil(K/G)] (F32 or F16); zeros
 * likewise (F16/F32) or nullptr with a fixed `offset`:  w[n,k] = (float(code) - zero) *
 * scale[n, k/G].
 * The reference layout is zeros = nullptr, offset 4 (int3) / 1 (int2), F32 scales, G = 128
 * (src/mrun/engine/kernels/qstore_int3.py:30-56, qstore_int2.py:24-63); the asymmetric
 * G = 64 variant passes F16 scales and F16 zero points. */

/* Replaces _dequant_int3 / _dequant_int2 (src/mrun/engine/kernels/qstore.py:441-456):
 * out[n,k] = (float(code) - zero) * scale in fp32, bit-exact.  bits 2, 3 or 4. */
int qs_lowbit_dequant(const uint8_t* packed, int64_t row_bytes, const void* scales,
                      int scale_dtype, const void* zeros, int zero_dtype, float offset, int bits,
                      int group_size, float* out, int64_t N, int64_t K, void* stream);

/* Workspace bytes qs_lowbit_gemv needs for these dimensions. */
size_t qs_lowbit_workspace_bytes(int x_dtype, int64_t M, int64_t N, int64_t K, int group_size);

/* Replaces QStoreInt3.matmul / QStoreInt2.matmul (qstore.py:1318-1341, 1451-1474):
 * y[m,n] = sum_k x[m,k] * w[n,k] in fp32, y F32 [M, N].  x BF16 or F32; bits 2 or 3; any
 * group size and K (the tiled kernels take G 64 / 128 with whole groups and 4-byte aligned
 * rows, every other layout a scalar-decode kernel).  workspace: device memory of at least
 * qs_lowbit_workspace_bytes(...) bytes, contents clobbered. */
int qs_lowbit_gemv(const void* x, int x_dtype, int64_t ldx, const uint8_t* packed,
                   int64_t row_bytes, const void* scales, int scale_dtype, const void* zeros,
                   int zero_dtype, float offset, int bits, int group_size, float* y, int64_t ldy,
                   int64_t M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes,
                   void* stream);

/* ---- offline codecs (store writer) --------------------------------------------------------
 * Replaces _quant_row_int8 (src/mrun/engine/kernels/qstore_build.py:496-501): per row,
 * s = max|W| / 127 (0 -> 1), q = clip(rint(W / s), +-127); W fp32 [N, K] (ldw), q int8
 * [N, K] (ldq), scales fp32 [N].  Bit-exact with the numpy writer. */
int qs_quant_rows_int8(const float* W, int64_t ldw, int64_t N, int64_t K, int8_t* q, int64_t ldq,
                       float* scales, void* stream);
/* Replaces _quant_row_int3 (qstore_int3.py:42-56, bits 3) and _quant_row_int2
 * (qstore_int2.py:36-63, bits 2, TWN ternary) with their packers (:30-39, :24-33): per row
 * and group of G columns, scales fp32 [N, ceil(K/G)] and LSB-first code streams packed
 * [N, row_bytes = ceil(K*bits/8)].  codes is a workspace of N*K bytes (raw codes).
 * Bit-exact with the numpy writer, including numpy's pairwise summation order in the
 * int2 means and sums. */
int qs_quant_rows_lowbit(const float* W, int64_t ldw, int64_t N, int64_t K, int bits, int G,
                         uint8_t* packed, int64_t row_bytes, float* scales, uint8_t* codes,
                         void* stream);

/* ---- pinned-host -> HBM page streaming -------------------------------------------------
 * Replaces the CUDA prefetch ring _RingSlot / _RingPrefetch (src/mrun/engine/kernels/
 * qstore.py:459-660: pinned staging, side-stream H2D, event + record_stream ordering) at
 * the runtime level.  The ring is caller-owned device memory of slots * slot_bytes bytes
 * (slot_bytes a multiple of 256); host sources must be pinned (hipHostMalloc / torch
 * pin_memory).  A submitted range is a run of contiguous host pages; it goes out as
 * hipMemcpyAsync transfers of at most max_transfer bytes on the pager's own copy stream
 * (default priority).  submit waits on the host for the slot's last release to have
 * fired on the GPU (blocking only while that consumer is still queued, i.e. when the host
 * is a whole ring ahead), seal marks the slot ready, acquire makes a compute stream wait
 * for ready, release marks the slot free once the compute stream's queued work is done. */
typedef struct qs_pager qs_pager;

int qs_pager_create(void* device_arena, size_t slot_bytes, int slots, size_t max_transfer,
                    qs_pager** out);
int qs_pager_destroy(qs_pager* pager);
/* Device address of a slot (nullptr when out of range). */
void* qs_pager_slot_ptr(qs_pager* pager, int slot);
/* Queue host[0..bytes) -> slot[dst_offset..dst_offset+bytes) on the copy stream. */
int qs_pager_submit(qs_pager* pager, int slot, const void* host, size_t bytes, size_t dst_offset);
/* Mark the end of the slot's submissions (records its ready event). */
int qs_pager_seal(qs_pager* pager, int slot);
/* host[0..count * slot_bytes) -> slots [slot, slot + count) (whole slots, contiguous in the
 * arena) on the copy stream, then each slot sealed: submit + seal for a run of slots with
 * the copy in max_transfer pieces.  With qs_pager_submit, replaces the miss path of the MoE
 * page cache (src/mrun/engine/qwen3_moe_cuda.py:1490-1567, _acquire_resident: one H2D of the
 * staged misses, then index_copy_ into the cache slots): here each run of consecutive pages
 * moves straight into its consecutive slots. */
int qs_pager_submit_run(qs_pager* pager, int slot, int count, const void* host);
int qs_pager_acquire(qs_pager* pager, int slot, void* compute_stream);
int qs_pager_release(qs_pager* pager, int slot, void* compute_stream);
/* acquire/release for slots[0..n) in one call (an expert layer's active set).
 * acquire_many enqueues no wait for a slot whose copies have already landed.
 * Replace the per-page event ordering of the MoE page cache,
 * src/mrun/engine/qwen3_moe_cuda.py:1490-1614 (_acquire_resident, acquire_slot_binding). */
int qs_pager_acquire_many(qs_pager* pager, const int* slots, int n, void* compute_stream);
/* release_many refuses (QS_ERR_INVALID, nothing changed) a batch that lists a slot twice. */
int qs_pager_release_many(qs_pager* pager, const int* slots, int n, void* compute_stream);
/* Block the host until every queued copy has landed. */
int qs_pager_sync(qs_pager* pager);
/* Host-side view of one slot's last sealed copies, for a caller that reuses the host
 * buffer a copy read from (the bounded pinned staging of _RingPrefetch._stage,
 * qstore.py:622-659, waits on its slot event for the same reason): slot_landed returns 1
 * when they have landed, 0 when not yet (negative on error); wait_landed blocks until
 * they have. */
int qs_pager_slot_landed(qs_pager* pager, int slot);
int qs_pager_wait_landed(qs_pager* pager, int slot);

#ifdef __cplusplus
}
#endif

#endif /* QSTORE_HIP_H_ */
