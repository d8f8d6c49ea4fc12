// Row gather + dequant of an int8 qrow block (embedding lookups) on gfx950.
//
//   k_dequant_rows4  : four pieces of 4 codes per thread, each one lane-contiguous 16-byte
//                      fp32 store; rows with K % 16 == 0 and aligned pointers.
//   k_dequant_rows   : one thread per element, any K.
// Both compute out[i, k] = float(codes[rows[i], k]) * scales[rows[i]] (one IEEE fp32
// multiply, the reference's dequant), and write zeros for a row index outside [0, N) (the
// host rejects those before the launch; the kernel never reads out of bounds either way).
#include "qs_common.h"

namespace qs {
namespace {

// A piece is 4 codes of a selected row and its one 16-byte fp32 store; lane l of a wave
// takes piece base + l, so a store instruction writes 1 KB of consecutive output.  Each
// thread takes U pieces, 256 apart, and issues all their loads before the first store.
constexpr int kRowPieces = 4;

template <int U>
__global__ __launch_bounds__(256) void k_dequant_rows4(const int8_t* __restrict__ codes,
                                                       const float* __restrict__ scales,
                                                       const int64_t* __restrict__ rows, int64_t n,
                                                       int64_t N, int64_t K, float* __restrict__ out) {
  const int64_t per_row = K / 4;
  const int64_t total = n * per_row;
  for (int64_t base = (int64_t)blockIdx.x * 256 * U; base < total; base += (int64_t)gridDim.x * 256 * U) {
    // the chunk's first output row from one division, each piece's from a 32-bit one
    const int64_t i0 = base / per_row;
    const uint32_t c0 = (uint32_t)(base - i0 * per_row);
    int64_t i[U], r[U];
    uint32_t c[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t off = c0 + (uint32_t)(u * 256 + threadIdx.x);  // < per_row + 256 U
      const uint32_t q = off / (uint32_t)per_row;
      ok[u] = base + u * 256 + threadIdx.x < total;
      i[u] = ok[u] ? i0 + q : 0;
      c[u] = ok[u] ? off - q * (uint32_t)per_row : 0u;
      r[u] = rows[i[u]];
    }
    int w[U];
    float sc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t rr = r[u] >= 0 && r[u] < N ? r[u] : 0;
      w[u] = *reinterpret_cast<const int*>(codes + rr * K + 4 * (int64_t)c[u]);
      sc[u] = scales[rr];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!ok[u]) continue;
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (r[u] >= 0 && r[u] < N) {
        v[0] = mul_rn(byte_f32(w[u], 0), sc[u]);
        v[1] = mul_rn(byte_f32(w[u], 1), sc[u]);
        v[2] = mul_rn(byte_f32(w[u], 2), sc[u]);
        v[3] = mul_rn(byte_f32(w[u], 3), sc[u]);
      }
      *reinterpret_cast<f32x4*>(out + i[u] * K + 4 * (int64_t)c[u]) = v;
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
  // per-row pieces must fit the 32-bit column arithmetic of k_dequant_rows4
  const bool fast = K % 16 == 0 && aligned(codes, 16) && aligned(out, 16) && K <= (int64_t(1) << 33);
  const int64_t per = fast ? 256 * kRowPieces : 256;
  const int64_t work = fast ? n_rows * (K / 4) : n_rows * K;
  const unsigned blocks = (unsigned)(cdiv(work, per) < 65536 ? cdiv(work, per) : 65536);
  if (fast)
    hipLaunchKernelGGL(k_dequant_rows4<kRowPieces>, dim3(blocks), dim3(256), 0, s, codes, scales, rows, n_rows, N, K,
                       out);
  else
    hipLaunchKernelGGL(k_dequant_rows, dim3(blocks), dim3(256), 0, s, codes, scales, rows, n_rows, N, K, out);
  return hip_check(hipGetLastError(), "k_dequant_rows launch");
}
