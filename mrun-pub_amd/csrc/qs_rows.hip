// Row gather + dequant of an int8 qrow block (embedding lookups) on gfx950.
//
//   k_dequant_rows16 : one thread per 16 codes of a selected row (one 16-byte load, four
//                      16-byte fp32 stores); rows with K % 16 == 0 and aligned pointers.
//   k_dequant_rows   : one thread per element, any K.
// Both compute out[i, k] = float(codes[rows[i], k]) * scales[rows[i]] (one IEEE fp32
// multiply, the reference's dequant), and write zeros for a row index outside [0, N) (the
// host rejects those before the launch; the kernel never reads out of bounds either way).
#include "qs_common.h"

namespace qs {
namespace {

__global__ __launch_bounds__(256) void k_dequant_rows16(const int8_t* __restrict__ codes,
                                                        const float* __restrict__ scales,
                                                        const int64_t* __restrict__ rows, int64_t n,
                                                        int64_t N, int64_t K, float* __restrict__ out) {
  const int64_t per_row = K / 16;
  const int64_t total = n * per_row;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += (int64_t)gridDim.x * 256) {
    const int64_t i = t / per_row;
    const int64_t c = t - i * per_row;
    const int64_t r = rows[i];
    f32x4* dst = reinterpret_cast<f32x4*>(out + i * K + c * 16);
    if (r < 0 || r >= N) {
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
      dst[0] = z;
      dst[1] = z;
      dst[2] = z;
      dst[3] = z;
      continue;
    }
    const i32x4 w = *reinterpret_cast<const i32x4*>(codes + r * K + c * 16);
    const float s = scales[r];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f32x4 v;
      v[0] = mul_rn(byte_f32(w[j], 0), s);
      v[1] = mul_rn(byte_f32(w[j], 1), s);
      v[2] = mul_rn(byte_f32(w[j], 2), s);
      v[3] = mul_rn(byte_f32(w[j], 3), s);
      dst[j] = v;
    }
  }
}

__global__ __launch_bounds__(256) void k_dequant_rows(const int8_t* __restrict__ codes,
                                                      const float* __restrict__ scales,
                                                      const int64_t* __restrict__ rows, int64_t n,
                                                      int64_t N, int64_t K, float* __restrict__ out) {
  const int64_t total = n * K;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += (int64_t)gridDim.x * 256) {
    const int64_t i = t / K;
    const int64_t k = t - i * K;
    const int64_t r = rows[i];
    out[t] = (r < 0 || r >= N) ? 0.f : mul_rn(static_cast<float>(codes[r * K + k]), scales[r]);
  }
}

}  // namespace
}  // namespace qs

using namespace qs;

extern "C" int qs_qrow_dequant_rows(const int8_t* codes, const float* scales, int64_t N, int64_t K,
                                    const int64_t* rows, int64_t n_rows, float* out, void* stream) {
  if (!codes || !scales || !out || (n_rows > 0 && !rows)) return fail(QS_ERR_INVALID, "dequant_rows: null pointer");
  if (N <= 0 || K <= 0 || n_rows < 0) return fail(QS_ERR_INVALID, "dequant_rows: bad shape");
  if (n_rows == 0) return QS_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool fast = K % 16 == 0 && aligned(codes, 16) && aligned(out, 16);
  const int64_t work = fast ? n_rows * (K / 16) : n_rows * K;
  const unsigned blocks = (unsigned)(cdiv(work, 256) < 65536 ? cdiv(work, 256) : 65536);
  if (fast)
    hipLaunchKernelGGL(k_dequant_rows16, dim3(blocks), dim3(256), 0, s, codes, scales, rows, n_rows, N, K, out);
  else
    hipLaunchKernelGGL(k_dequant_rows, dim3(blocks), dim3(256), 0, s, codes, scales, rows, n_rows, N, K, out);
  return hip_check(hipGetLastError(), "k_dequant_rows launch");
}
