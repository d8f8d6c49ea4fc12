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

/* Replaces fused_qrow_swiglu + _qrow_w8a16_paired_swiglu_kernel
 * (dense_qstore_cuda.py:1053-1102, 515-575); reference contract
 * fused_qrow_swiglu_reference (dense_qstore_cuda.py:1037-1050):
 *   g = bf16(x @ Wg^T), u = bf16(x @ Wu^T) (W8A16 each),
 *   y = bf16( float(bf16(g * sigmoid(g))) * float(u) ).  x, y BF16. */
int qs_qrow_swiglu(const void* x, int64_t ldx, const int8_t* gate_codes,
                   const float* gate_scales, const int8_t* up_codes, const float* up_scales,
                   void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* stream);

/* ---- W8A8 (int8 weights x per-token int8 activations) ------------------------------ */

/* Activation quantizer of w8a8_matmul (src/mrun/engine/kernels/w8a8.py:118-121):
 * per row m, v = x*keep (keep nullable, fp32 [K]); s[m] = max|v|/127 (0 -> 1);
 * q[m,k] = clamp(round_half_even(v/s[m]), -127, 127).  IEEE fp32 ops, bit-exact. */
int qs_act_quant_i8(const void* x, int x_dtype, int64_t ldx, const float* keep, int8_t* q,
                    float* scale, int64_t M, int64_t K, void* stream);

/* Outlier column selection of w8a8_matmul (w8a8.py:98-102): colmax[k] = max_m |x[m,k]|,
 * idx = the k largest (1 <= k <= 64, ties -> lower column), keep = 1 except 0 at idx.
 * colmax is caller-provided workspace of K floats. */
int qs_outlier_topk(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int k,
                    float* colmax, int64_t* idx, float* keep, void* stream);

/* Operands of the exact fp32 side path (w8a8.py:108-112): xp[m,p] = float(x[m, idx[p]]),
 * wp[n,p] = float(qw[n, idx[p]]) * sw[n]; 1 <= P <= 64. */
int qs_w8a8_side_gather(const void* x, int x_dtype, int64_t ldx, const int8_t* qw,
                        const float* sw, const int64_t* idx, int P, int64_t M, int64_t N,
                        int64_t K, float* xp, float* wp, void* stream);

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

#ifdef __cplusplus
}
#endif

#endif /* QSTORE_HIP_H_ */
