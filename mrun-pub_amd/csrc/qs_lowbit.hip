// Packed int3 / int2 QStore GEMV and dequant on gfx950.
//
// Layout (reference qstore_int3.py:30-56, qstore_int2.py:24-63): every weight row is an
// LSB-first bitstream, code k at bits [b*k, b*k + b) of the row, row_bytes =
// ceil(K*b/8); one scale per (row, group of G codes).  Weight value
//   w[n,k] = (float(code) - zero[n, k/G]) * scale[n, k/G]
// with zero the reference's fixed offset (4 for int3, 1 for int2; scales fp32, G = 128) or
// a per-group zero point (fp16 scale + fp16 zero, G = 64: the asymmetric variant).
//
// GEMV (k_lowbit_mfma): y[m,n] = sum_k x[m,k] w[n,k] in fp32.  Codes are widened to the
// exact bf16 values OFF + code (OFF = 8 for 3-bit, 4 for 2-bit: bf16 bit pattern
// 0x4100 | code << 4, resp. 0x4080 | code << 5 -- one bfe, one 24-bit multiply and one
// and_or per PAIR of codes) and fed to v_mfma_f32_16x16x32_bf16 against bf16 activations
// (products exact in fp32).  Each MFMA covers 32 codes of ONE group, so per group
//   sum_k x (code - z) = R - (OFF + z) * S0,     S0 = sum_{k in group} x[m,k],
// and y += scale * (R - (OFF + z) * S0).  fp32 activations are split exactly into three
// bf16 terms (x = h + m + l) that run as three activation rows and are summed at the end.
#include "qs_common.h"

namespace qs {

struct LowbitParams {
  const uint16_t* x;   // bf16 [M, K] (M <= 16)
  int64_t ldx;
  const float* s0;     // [M, ng] group sums of x
  const uint8_t* packed;
  int64_t row_bytes;
  const void* scales;  // [N, ng] f32 or f16
  const void* zeros;   // [N, ng] f16/f32, nullable
  int scale_f16, zero_f16;
  float offset;        // used when zeros == nullptr
  float* y;            // [M, N]
  int64_t ldy;
  int M, N, K, ng;
};

// Lane code extraction: the lane's G/4 codes (BITS*G/4 bits, at a 2- or 4-byte aligned
// offset) are returned as a 64/96-bit little-endian field.
template <int BITS, int G>
__device__ __forceinline__ void load_codes(const uint8_t* p, uint32_t (&f)[3]) {
  constexpr int NB = BITS * G / 4;  // bits per lane: 48, 96, 32, 64
  if constexpr (NB == 96) {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
    f[0] = __builtin_nontemporal_load(q);
    f[1] = __builtin_nontemporal_load(q + 1);
    f[2] = __builtin_nontemporal_load(q + 2);
  } else if constexpr (NB == 64) {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
    f[0] = __builtin_nontemporal_load(q);
    f[1] = __builtin_nontemporal_load(q + 1);
    f[2] = 0;
  } else if constexpr (NB == 32) {
    f[0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
    f[1] = f[2] = 0;
  } else {  // 48 bits at a 2-byte aligned offset; never reads outside [p, p + 6)
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    if (a & 2) {
      const uint16_t h0 = __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(p));
      const uint32_t d1 = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p + 2));
      f[0] = (uint32_t)h0 | (d1 << 16);
      f[1] = d1 >> 16;
    } else {
      f[0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
      f[1] = __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(p + 4));
    }
    f[2] = 0;
  }
}

// 2 codes starting at bit position bp of the field -> packed bf16 pair (OFF + c).
template <int BITS>
__device__ __forceinline__ uint32_t code_pair(const uint32_t (&f)[3], int bp) {
  const int w = bp >> 5, o = bp & 31;
  uint32_t t;
  if (o + 2 * BITS <= 32)
    t = __builtin_amdgcn_ubfe(f[w], o, 2 * BITS);
  else
    t = __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(f[w + 1], f[w], o), 0, 2 * BITS);
  if constexpr (BITS == 3)
    return ((t * 0x20010u) & 0x00700070u) | 0x41004100u;  // 8 + c at bits 4-6 / 20-22
  else
    return ((t * 0x80020u) & 0x00600060u) | 0x40804080u;  // 4 + c at bits 5-6 / 21-22
}

template <int BITS, int G, int KW>
__global__ __launch_bounds__(KW * 64) void k_lowbit_mfma(LowbitParams p) {
  constexpr int CODES = G / 4;               // codes per lane per group
  constexpr int CB = BITS * G / 8;           // bytes per row per group
  constexpr int LB = BITS * CODES / 8;       // bytes per lane per group (may be 6)
  constexpr int NMMA = G / 32;               // MFMAs per group
  constexpr float OFF = BITS == 3 ? 8.f : 4.f;
  const int lane = threadIdx.x & 63;
  const int ks = threadIdx.x >> 6;
  const int col = lane & 15, g4 = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int n = min(n0 + col, p.N - 1);
  const uint8_t* row = p.packed + (int64_t)n * p.row_bytes + g4 * LB;
  const bool mval = col < p.M;
  const uint16_t* xr = p.x + (int64_t)(mval ? col : 0) * p.ldx + g4 * CODES;
  f32x4 y = {0.f, 0.f, 0.f, 0.f};

  // UG groups per round: their codes, activations and scales are all requested before
  // the first one is consumed.
  constexpr int UG = 4;
  for (int g0 = ks; g0 < p.ng; g0 += UG * KW) {
    uint32_t f[UG][3];
    bf16x8 xa[UG][NMMA];
    float sc[UG], z[UG];
#pragma unroll
    for (int u = 0; u < UG; ++u) {
      const int g = g0 + u * KW;
      if (g < p.ng) {
        load_codes<BITS, G>(row + (int64_t)g * CB, f[u]);
#pragma unroll
        for (int j = 0; j < NMMA; ++j)
          xa[u][j] = mval ? *reinterpret_cast<const bf16x8*>(xr + (int64_t)g * G + 8 * j) : bf16x8{};
        const int64_t si = (int64_t)n * p.ng + g;
        sc[u] = p.scale_f16 ? f16_bits_to_f32(static_cast<const uint16_t*>(p.scales)[si])
                            : static_cast<const float*>(p.scales)[si];
        if (p.zeros)
          z[u] = p.zero_f16 ? f16_bits_to_f32(static_cast<const uint16_t*>(p.zeros)[si])
                            : static_cast<const float*>(p.zeros)[si];
        else
          z[u] = p.offset;
      }
    }
#pragma unroll
    for (int u = 0; u < UG; ++u) {
      const int g = g0 + u * KW;
      if (g >= p.ng) break;
      f32x4 r = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NMMA; ++j) {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        u32x4 b;
#pragma unroll
        for (int d = 0; d < 4; ++d) b[d] = code_pair<BITS>(f[u], BITS * (8 * j + 2 * d));
        r = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[u][j], __builtin_bit_cast(bf16x8, b), r, 0, 0, 0);
      }
      const float c = OFF + z[u];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = 4 * g4 + q;
        const float s0 = m < p.M ? p.s0[(int64_t)m * p.ng + g] : 0.f;
        y[q] = fmaf(sc[u], fmaf(-c, s0, r[q]), y[q]);
      }
    }
  }
  __shared__ f32x4 red[KW][64];
  red[ks][lane] = y;
  __syncthreads();
  if (ks != 0) return;
  f32x4 t = red[0][lane];
#pragma unroll
  for (int w = 1; w < KW; ++w) t += red[w][lane];
  const int no = n0 + col;
  if (no >= p.N) return;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int m = 4 * g4 + q;
    if (m < p.M) p.y[(int64_t)m * p.ldy + no] = t[q];
  }
}

// x (f32 or bf16) -> bf16 activation rows: bf16 x is copied; fp32 row m becomes rows
// 3m, 3m+1, 3m+2 = h, bf16(x - h), bf16(x - h - m) (an exact three-term split).
__global__ __launch_bounds__(256) void k_lowbit_prep(const void* __restrict__ x, int x_dtype,
                                                     int64_t ldx, int M, int K,
                                                     uint16_t* __restrict__ xb) {
  const int64_t i = blockIdx.x * 256ll + threadIdx.x;
  if (i >= (int64_t)M * K) return;
  const int64_t m = i / K, k = i - m * K;
  if (x_dtype == QS_BF16) {
    xb[m * K + k] = static_cast<const uint16_t*>(x)[m * ldx + k];
  } else {
    const float v = static_cast<const float*>(x)[m * ldx + k];
    const uint16_t h = f32_to_bf16_bits(v);
    const float r1 = v - bf16_bits_to_f32(h);
    const uint16_t md = f32_to_bf16_bits(r1);
    const float r2 = r1 - bf16_bits_to_f32(md);
    xb[(3 * m) * K + k] = h;
    xb[(3 * m + 1) * K + k] = md;
    xb[(3 * m + 2) * K + k] = f32_to_bf16_bits(r2);
  }
}

// S0[m, g] = sum of the G bf16 activations of group g, fixed order.  One wave per (m, g).
__global__ __launch_bounds__(256) void k_group_sums(const uint16_t* __restrict__ xb, int M, int K,
                                                    int G, float* __restrict__ s0) {
  const int lane = threadIdx.x & 63;
  const int64_t w = blockIdx.x * 4ll + (threadIdx.x >> 6);
  const int ng = K / G;
  if (w >= (int64_t)M * ng) return;
  const int64_t m = w / ng, g = w - m * ng;
  float v = 0.f;
  for (int k = lane; k < G; k += 64) v += bf16_bits_to_f32(xb[m * K + g * G + k]);
  v = wave_sum(v);
  if (lane == 0) s0[w] = v;
}

// y[m, n] = y3[3m, n] + y3[3m+1, n] + y3[3m+2, n]
__global__ __launch_bounds__(256) void k_lowbit_combine(const float* __restrict__ y3, int M, int N,
                                                        float* __restrict__ y, int64_t ldy) {
  const int64_t i = blockIdx.x * 256ll + threadIdx.x;
  if (i >= (int64_t)M * N) return;
  const int64_t m = i / N, n = i - m * N;
  y[m * ldy + n] = add_rn(add_rn(y3[(3 * m) * N + n], y3[(3 * m + 1) * N + n]), y3[(3 * m + 2) * N + n]);
}

// w[n, k] = (float(code) - zero) * scale, fp32 (reference _dequant_int3/_int2 order).
__global__ __launch_bounds__(256) void k_lowbit_dequant(LowbitParams p, int bits, int G, float* __restrict__ out) {
  const int64_t i = blockIdx.x * 256ll + threadIdx.x;
  if (i >= (int64_t)p.N * p.K) return;
  const int64_t n = i / p.K, k = i - n * p.K;
  const int64_t bit = k * bits;
  const uint8_t* row = p.packed + n * p.row_bytes;
  uint32_t v = row[bit >> 3] >> (bit & 7);
  if ((bit & 7) + bits > 8) v |= (uint32_t)row[(bit >> 3) + 1] << (8 - (bit & 7));
  const uint32_t code = v & ((1u << bits) - 1);
  const int64_t si = n * p.ng + k / G;
  const float sc = p.scale_f16 ? f16_bits_to_f32(static_cast<const uint16_t*>(p.scales)[si])
                               : static_cast<const float*>(p.scales)[si];
  float z = p.offset;
  if (p.zeros)
    z = p.zero_f16 ? f16_bits_to_f32(static_cast<const uint16_t*>(p.zeros)[si])
                   : static_cast<const float*>(p.zeros)[si];
  out[i] = mul_rn(static_cast<float>(code) - z, sc);
}

namespace {
template <int BITS, int G>
void launch_lowbit(const LowbitParams& p, hipStream_t s) {
  const dim3 grid((unsigned)cdiv(p.N, 16));
  if (p.ng >= 64)
    hipLaunchKernelGGL((k_lowbit_mfma<BITS, G, 8>), grid, dim3(8 * 64), 0, s, p);
  else
    hipLaunchKernelGGL((k_lowbit_mfma<BITS, G, 4>), grid, dim3(4 * 64), 0, s, p);
}

int check_lowbit(const void* packed, int64_t row_bytes, const void* scales, int bits, int G,
                 int64_t N, int64_t K) {
  if (!packed || !scales) return fail(QS_ERR_INVALID, "lowbit: null pointer");
  if (bits != 2 && bits != 3) return fail(QS_ERR_UNSUPPORTED, "lowbit: bits must be 2 or 3");
  if (G != 64 && G != 128) return fail(QS_ERR_UNSUPPORTED, "lowbit: group size must be 64 or 128");
  if (N <= 0 || K <= 0 || K % G != 0) return fail(QS_ERR_UNSUPPORTED, "lowbit: K must be a positive multiple of the group size");
  if (row_bytes < (K * bits + 7) / 8) return fail(QS_ERR_INVALID, "lowbit: row_bytes too small");
  if (row_bytes % 4 != 0 || !aligned(packed, 4)) return fail(QS_ERR_UNSUPPORTED, "lowbit: rows must be 4-byte aligned");
  return QS_OK;
}
}  // namespace
}  // namespace qs

using namespace qs;

extern "C" int qs_lowbit_gemv(const void* x, int x_dtype, int64_t ldx, const uint8_t* packed,
                              int64_t row_bytes, const void* scales, int scale_dtype,
                              const void* zeros, int zero_dtype, float offset, int bits,
                              int group_size, float* y, int64_t ldy, int64_t M, int64_t N,
                              int64_t K, void* workspace, size_t workspace_bytes, void* stream) {
  int st = check_lowbit(packed, row_bytes, scales, bits, group_size, N, K);
  if (st) return st;
  if (!x || !y) return fail(QS_ERR_INVALID, "lowbit_gemv: null pointer");
  if (x_dtype != QS_BF16 && x_dtype != QS_F32) return fail(QS_ERR_INVALID, "lowbit_gemv: x must be BF16 or F32");
  if (scale_dtype != QS_F32 && scale_dtype != QS_F16) return fail(QS_ERR_INVALID, "lowbit_gemv: scales F32 or F16");
  if (zeros && zero_dtype != QS_F32 && zero_dtype != QS_F16) return fail(QS_ERR_INVALID, "lowbit_gemv: zeros F32 or F16");
  if (M < 0 || ldx < K || ldy < N) return fail(QS_ERR_INVALID, "lowbit_gemv: bad leading dimension");
  if (M == 0) return QS_OK;
  const int rows_per_x = x_dtype == QS_F32 ? 3 : 1;
  const int mb = x_dtype == QS_F32 ? 5 : 16;  // activation rows per MFMA tile
  const int ng = (int)(K / group_size);
  const size_t need = qs_lowbit_workspace_bytes(x_dtype, M, N, K, group_size);
  if (!workspace || workspace_bytes < need)
    return fail(QS_ERR_INVALID, "lowbit_gemv: workspace of %zu bytes required", need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // workspace: bf16 rows [mb*rows_per_x, K] | s0 [mb*rows_per_x, ng] | y3 [mb*3, N]
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint16_t* xb = reinterpret_cast<uint16_t*>(ws);
  const size_t xb_bytes = ((size_t)16 * K * 2 + 255) / 256 * 256;
  float* s0 = reinterpret_cast<float*>(ws + xb_bytes);
  const size_t s0_bytes = ((size_t)16 * ng * 4 + 255) / 256 * 256;
  float* y3 = reinterpret_cast<float*>(ws + xb_bytes + s0_bytes);
  for (int64_t m0 = 0; m0 < M; m0 += mb) {
    const int mm = (int)((M - m0) < mb ? (M - m0) : mb);
    const int rows = mm * rows_per_x;
    const void* xm = static_cast<const char*>(x) + m0 * ldx * (x_dtype == QS_F32 ? 4 : 2);
    hipLaunchKernelGGL(k_lowbit_prep, dim3((unsigned)cdiv((int64_t)mm * K, 256)), dim3(256), 0, s, xm, x_dtype, ldx, mm, (int)K, xb);
    hipLaunchKernelGGL(k_group_sums, dim3((unsigned)cdiv((int64_t)rows * ng, 4)), dim3(256), 0, s, xb, rows, (int)K, group_size, s0);
    LowbitParams p{};
    p.x = xb;
    p.ldx = K;
    p.s0 = s0;
    p.packed = packed;
    p.row_bytes = row_bytes;
    p.scales = scales;
    p.zeros = zeros;
    p.scale_f16 = scale_dtype == QS_F16;
    p.zero_f16 = zero_dtype == QS_F16;
    p.offset = offset;
    p.M = rows;
    p.N = (int)N;
    p.K = (int)K;
    p.ng = ng;
    if (x_dtype == QS_BF16) {
      p.y = y + m0 * ldy;
      p.ldy = ldy;
    } else {
      p.y = y3;
      p.ldy = N;
    }
    if (bits == 3 && group_size == 64) launch_lowbit<3, 64>(p, s);
    else if (bits == 3) launch_lowbit<3, 128>(p, s);
    else if (group_size == 64) launch_lowbit<2, 64>(p, s);
    else launch_lowbit<2, 128>(p, s);
    if (x_dtype == QS_F32)
      hipLaunchKernelGGL(k_lowbit_combine, dim3((unsigned)cdiv((int64_t)mm * N, 256)), dim3(256), 0, s, y3, mm, (int)N, y + m0 * ldy, ldy);
  }
  return hip_check(hipGetLastError(), "k_lowbit launch");
}

extern "C" size_t qs_lowbit_workspace_bytes(int x_dtype, int64_t M, int64_t N, int64_t K, int group_size) {
  (void)M;
  (void)x_dtype;
  const int64_t ng = group_size > 0 ? K / group_size : 0;
  const size_t xb = ((size_t)16 * K * 2 + 255) / 256 * 256;
  const size_t s0 = ((size_t)16 * ng * 4 + 255) / 256 * 256;
  const size_t y3 = (size_t)15 * N * 4;
  return xb + s0 + y3;
}

extern "C" int qs_lowbit_dequant(const uint8_t* packed, int64_t row_bytes, const void* scales,
                                 int scale_dtype, const void* zeros, int zero_dtype, float offset,
                                 int bits, int group_size, float* out, int64_t N, int64_t K,
                                 void* stream) {
  if (!packed || !scales || !out) return fail(QS_ERR_INVALID, "lowbit_dequant: null pointer");
  if (bits != 2 && bits != 3 && bits != 4) return fail(QS_ERR_UNSUPPORTED, "lowbit_dequant: bits 2, 3 or 4");
  if (group_size <= 0 || N <= 0 || K <= 0 || row_bytes < (K * bits + 7) / 8)
    return fail(QS_ERR_INVALID, "lowbit_dequant: bad shape");
  LowbitParams p{};
  p.packed = packed;
  p.row_bytes = row_bytes;
  p.scales = scales;
  p.zeros = zeros;
  p.scale_f16 = scale_dtype == QS_F16;
  p.zero_f16 = zero_dtype == QS_F16;
  p.offset = offset;
  p.N = (int)N;
  p.K = (int)K;
  p.ng = (int)((K + group_size - 1) / group_size);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_lowbit_dequant, dim3((unsigned)cdiv(N * K, 256)), dim3(256), 0, s, p, bits, group_size, out);
  return hip_check(hipGetLastError(), "k_lowbit_dequant launch");
}
