// Offline QStore codecs on the device: the writer's row quantizers, bit-exact.
//
// Kernels
//   k_quant_int8   : one wave per row: s = max|W| / 127 (0 -> 1), q = clip(rint(W / s), +-127)
//                    (_quant_row_int8, src/mrun/engine/kernels/qstore_build.py:496-501).
//   k_quant_groups : one thread per (row, group) of G columns, raw codes to a workspace:
//                    bits 3: s = max|blk| / 3 (0 -> 1), code = clip(rint(blk / s), -3, 3) + 4
//                    (_quant_row_int3, qstore_int3.py:42-56);
//                    bits 2: TWN ternary, thr = 0.7 * mean|blk|, active = |blk| >= thr,
//                    s = sum(|blk| * active) / count (no active -> 1; 0 -> 1),
//                    code = (active ? sign(blk) : 0) + 1 (_quant_row_int2, qstore_int2.py:36-63).
//   k_pack_codes   : one thread per output byte of the LSB-first row bitstream
//                    (np.packbits(bitorder="little"), qstore_int3.py:30-39, qstore_int2.py:24-33).
//   k_quant_int8_r/_v, k_quant_g128 : the same arithmetic with 16-byte loads, for rows of
//                    whole 4-column pieces (int8; rows up to 4096 held in registers) and for
//                    the writers' default G = 128 with whole groups (int3/int2, codes packed
//                    in the same launch).
//
// Arithmetic follows numpy's exactly:
//   * float32 divisions by the literals 127.0 / 3.0 (numpy keeps float32 for a Python float
//     operand) and by the per-element scale are IEEE single divisions (HIP's default float
//     division is correctly rounded), np.round is round-half-even (rintf);
//   * the float32 sums of mean() and sum() use numpy's pairwise summation order (8
//     interleaved partial sums for n <= 128, combined as ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)),
//     the n % 8 tail added in order; longer runs split at n/2 rounded down to a multiple
//     of 8), starting from the additive identity;
//   * mean = float32(double(sum) / n) and s = float32(double(weighted) / count): numpy
//     divides a float32 array by an integer count in float64 and casts the result back;
//   * 0.7 * mean is a float32 product with 0.7 rounded to float32.
#include "qs_common.h"

namespace qs {

// numpy's float32 pairwise sum of f(0) .. f(n-1) (loops_utils.h: FLOAT_pairwise_sum),
// written as an explicit stack of halves so that it stays iterative on the device.
template <typename F>
__device__ float np_pairwise_sum(int n, F f) {
  // ranges waiting to be summed: [start, len]; results combined in the same tree order
  // through a second stack of partial sums.
  int st_start[32], st_len[32], st_state[32];
  float st_val[32];
  int sp = 0;
  st_start[0] = 0;
  st_len[0] = n;
  st_state[0] = 0;
  float ret = 0.f;
  while (sp >= 0) {
    const int a = st_start[sp], len = st_len[sp];
    if (len <= 128) {
      float res;
      if (len < 8) {
        res = 0.f;
        for (int i = 0; i < len; ++i) res += f(a + i);
      } else {
        float r[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = f(a + j);
        int i = 8;
        for (; i < len - (len % 8); i += 8) {
#pragma unroll
          for (int j = 0; j < 8; ++j) r[j] += f(a + i + j);
        }
        res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        for (; i < len; ++i) res += f(a + i);
      }
      // pop and hand the result to the parent
      --sp;
      while (true) {
        if (sp < 0) {
          ret = res;
          break;
        }
        if (st_state[sp] == 1) {  // left half done: remember it, descend into the right half
          st_val[sp] = res;
          st_state[sp] = 2;
          const int n2 = st_len[sp] / 2 - (st_len[sp] / 2) % 8;
          ++sp;
          st_start[sp] = st_start[sp - 1] + n2;
          st_len[sp] = st_len[sp - 1] - n2;
          st_state[sp] = 0;
          break;
        }
        // both halves done
        res = st_val[sp] + res;
        --sp;
      }
    } else {
      // split: left half first
      st_state[sp] = 1;
      const int n2 = len / 2 - (len / 2) % 8;
      ++sp;
      st_start[sp] = a;
      st_len[sp] = n2;
      st_state[sp] = 0;
    }
  }
  return ret;
}

__global__ __launch_bounds__(256) void k_quant_int8(const float* __restrict__ W, int64_t ldw, int N, int K,
                                                    int8_t* __restrict__ q, int64_t ldq, float* __restrict__ scales) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const float* w = W + (int64_t)n * ldw;
  float mx = 0.f;
  for (int k = lane; k < K; k += 64) mx = fmaxf(mx, fabsf(w[k]));
  mx = wave_max(mx);
  float s = mx / 127.0f;
  if (s == 0.f) s = 1.f;
  if (lane == 0) scales[n] = s;
  for (int k = lane; k < K; k += 64) {
    float r = rintf(w[k] / s);
    r = fminf(fmaxf(r, -127.f), 127.f);
    q[(int64_t)n * ldq + k] = static_cast<int8_t>(r);
  }
}

// k_quant_int8 for rows of whole 4-column pieces (16-byte aligned): 16-byte loads, the
// second pass re-reading the row from L2, four codes per 4-byte store.
__global__ __launch_bounds__(256) void k_quant_int8_v(const float* __restrict__ W, int64_t ldw, int N, int K,
                                                      int8_t* __restrict__ q, int64_t ldq,
                                                      float* __restrict__ scales) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const f32x4* w = reinterpret_cast<const f32x4*>(W + (int64_t)n * ldw);
  const int k4 = K / 4;
  float mx = 0.f;
  for (int i = lane; i < k4; i += 64) {
    const f32x4 v = w[i];
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
  }
  mx = wave_max(mx);
  float s = mx / 127.0f;
  if (s == 0.f) s = 1.f;
  if (lane == 0) scales[n] = s;
  auto code = [&](float x) -> uint32_t {
    float r = rintf(x / s);
    r = fminf(fmaxf(r, -127.f), 127.f);
    return static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(r)));
  };
  uint32_t* qo = reinterpret_cast<uint32_t*>(q + (int64_t)n * ldq);
  for (int i = lane; i < k4; i += 64) {
    const f32x4 v = w[i];
    qo[i] = code(v[0]) | code(v[1]) << 8 | code(v[2]) << 16 | code(v[3]) << 24;
  }
}

// k_quant_int8_v for K <= 4096: the row stays in registers (up to 16 four-column pieces
// per lane), so it is read once; the two-pass form re-read it from HBM (470 MB fetched for
// a 235 MB weight).
__global__ __launch_bounds__(256) void k_quant_int8_r(const float* __restrict__ W, int64_t ldw, int N, int K,
                                                      int8_t* __restrict__ q, int64_t ldq,
                                                      float* __restrict__ scales) {
  constexpr int V = 16;  // pieces per lane: K <= 64 * V * 4
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const f32x4* w = reinterpret_cast<const f32x4*>(W + (int64_t)n * ldw);
  const int k4 = K / 4;
  f32x4 v[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int i = lane + 64 * j;
    v[j] = i < k4 ? w[i] : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float mx = 0.f;
#pragma unroll
  for (int j = 0; j < V; ++j)
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[j][0]), fabsf(v[j][1])), fmaxf(fabsf(v[j][2]), fabsf(v[j][3]))));
  mx = wave_max(mx);
  float s = mx / 127.0f;
  if (s == 0.f) s = 1.f;
  if (lane == 0) scales[n] = s;
  auto code = [&](float x) -> uint32_t {
    float r = rintf(x / s);
    r = fminf(fmaxf(r, -127.f), 127.f);
    return static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(r)));
  };
  uint32_t* qo = reinterpret_cast<uint32_t*>(q + (int64_t)n * ldq);
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int i = lane + 64 * j;
    if (i < k4) qo[i] = code(v[j][0]) | code(v[j][1]) << 8 | code(v[j][2]) << 16 | code(v[j][3]) << 24;
  }
}

// k_quant_groups + k_pack_codes for G = 128 with whole groups (K % 128 == 0) and 16-byte
// aligned rows, in one launch: half a wave per group, lane l of the half holding columns
// 4l .. 4l + 3.  int3: the group maximum over the half, then lane pairs write their 8 codes
// as 3 bytes.  int2: numpy's pairwise sums of 128 terms are 8 interleaved running sums
// (terms j, j + 8, .., j + 120, in order) combined as ((r0 + r1) + (r2 + r3)) + ((r4 + r5) +
// (r6 + r7)); the group goes through LDS so that lane j < 8 of the half forms r_j in that
// order, and an xor butterfly over lanes 0..7 forms the combination bit for bit (IEEE
// addition commutes).  Each lane then writes its 4 codes as one byte.
template <int BITS>
__global__ __launch_bounds__(256) void k_quant_g128(const float* __restrict__ W, int64_t ldw, int N, int K,
                                                    float* __restrict__ scales, uint8_t* __restrict__ packed,
                                                    int64_t row_bytes) {
  __shared__ __attribute__((aligned(16))) float stage[8][128];  // one group per half wave
  const int lane = threadIdx.x & 63, hw = threadIdx.x >> 5, l = lane & 31;
  const int ng = K / 128;
  const int64_t grp = (int64_t)blockIdx.x * 8 + hw;
  const bool valid = grp < (int64_t)N * ng;
  const int n = valid ? (int)(grp / ng) : 0;
  const int g = valid ? (int)(grp - (int64_t)n * ng) : 0;
  const f32x4 v = valid ? *reinterpret_cast<const f32x4*>(W + (int64_t)n * ldw + g * 128 + 4 * l)
                        : f32x4{0.f, 0.f, 0.f, 0.f};
  float* st = stage[hw];
  // numpy's pairwise sum of the 128 staged values.  A half wave reads only what its own
  // wave wrote, and a wave's LDS operations complete in order: waiting for this wave's
  // writes is enough, no workgroup barrier
  auto staged_sum = [&]() -> float {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    float r = 0.f;
    if (l < 8) {
      r = st[l];
      for (int i = 1; i < 16; ++i) r += st[l + 8 * i];
    }
    r += __shfl_xor(r, 1);
    r += __shfl_xor(r, 2);
    r += __shfl_xor(r, 4);
    return __shfl(r, lane & 32);  // lane 0 of the half
  };
  uint8_t* const prow = packed + (int64_t)n * row_bytes;
  float s;
  if constexpr (BITS == 3) {
    float mx = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    for (int o = 1; o < 32; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));  // within the half
    s = mx / 3.0f;
    if (s == 0.f) s = 1.f;
    uint32_t c12 = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float r = rintf(v[t] / s);
      r = fminf(fmaxf(r, -3.f), 3.f);
      c12 |= static_cast<uint32_t>(static_cast<int>(r) + 4) << (3 * t);
    }
    const uint32_t c24 = c12 | static_cast<uint32_t>(__shfl_xor(static_cast<int>(c12), 1)) << 12;
    if (valid && (l & 1) == 0) {
      uint8_t* const o = prow + g * 48 + 3 * (l >> 1);
      o[0] = static_cast<uint8_t>(c24);
      o[1] = static_cast<uint8_t>(c24 >> 8);
      o[2] = static_cast<uint8_t>(c24 >> 16);
    }
  } else {
    const f32x4 a = {fabsf(v[0]), fabsf(v[1]), fabsf(v[2]), fabsf(v[3])};
    *reinterpret_cast<f32x4*>(st + 4 * l) = a;
    const float sum_abs = staged_sum();
    const float mean = static_cast<float>(static_cast<double>(sum_abs) / 128);
    const float thr = 0.7f * mean;
    int cnt = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) cnt += a[t] >= thr;
    for (int o = 1; o < 32; o <<= 1) cnt += __shfl_xor(cnt, o);
    // the first staging's reads have returned (their sums were used above) before the
    // second staging is written
    *reinterpret_cast<f32x4*>(st + 4 * l) =
        f32x4{a[0] >= thr ? a[0] : 0.f, a[1] >= thr ? a[1] : 0.f, a[2] >= thr ? a[2] : 0.f, a[3] >= thr ? a[3] : 0.f};
    const float weighted = staged_sum();
    s = cnt > 0 ? static_cast<float>(static_cast<double>(weighted) / cnt) : 1.f;
    if (s == 0.f) s = 1.f;
    uint32_t b = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int sg = v[t] > 0.f ? 1 : (v[t] < 0.f ? -1 : 0);
      b |= static_cast<uint32_t>((a[t] >= thr ? sg : 0) + 1) << (2 * t);
    }
    if (valid) prow[g * 32 + l] = static_cast<uint8_t>(b);
  }
  if (valid && l == 0) scales[(int64_t)n * ng + g] = s;
}

template <int BITS>
__global__ __launch_bounds__(256) void k_quant_groups(const float* __restrict__ W, int64_t ldw, int N, int K,
                                                      int G, float* __restrict__ scales,
                                                      uint8_t* __restrict__ codes) {
  const int ng = (K + G - 1) / G;
  const int64_t t = blockIdx.x * 256ll + threadIdx.x;
  if (t >= (int64_t)N * ng) return;
  const int n = (int)(t / ng), g = (int)(t - (int64_t)n * ng);
  const int c0 = g * G, len = min(G, K - c0);
  const float* w = W + (int64_t)n * ldw + c0;
  uint8_t* out = codes + (int64_t)n * K + c0;
  float s;
  if constexpr (BITS == 3) {
    float mx = 0.f;
    for (int i = 0; i < len; ++i) mx = fmaxf(mx, fabsf(w[i]));
    s = mx / 3.0f;
    if (s == 0.f) s = 1.f;
    for (int i = 0; i < len; ++i) {
      float r = rintf(w[i] / s);
      r = fminf(fmaxf(r, -3.f), 3.f);
      out[i] = static_cast<uint8_t>(static_cast<int>(r) + 4);
    }
  } else {
    const float sum_abs = np_pairwise_sum(len, [&](int i) { return fabsf(w[i]); });
    const float mean = static_cast<float>(static_cast<double>(sum_abs) / len);
    const float thr = 0.7f * mean;
    int count = 0;
    for (int i = 0; i < len; ++i) count += fabsf(w[i]) >= thr;
    const float weighted = np_pairwise_sum(len, [&](int i) {
      const float a = fabsf(w[i]);
      return a >= thr ? a : 0.f;  // |w| * active (active is 0/1; a * 0 = +0)
    });
    s = count > 0 ? static_cast<float>(static_cast<double>(weighted) / count) : 1.f;
    if (s == 0.f) s = 1.f;
    for (int i = 0; i < len; ++i) {
      const float v = w[i];
      const int sg = v > 0.f ? 1 : (v < 0.f ? -1 : 0);
      out[i] = static_cast<uint8_t>((fabsf(v) >= thr ? sg : 0) + 1);
    }
  }
  scales[(int64_t)n * ng + g] = s;
}

// Output byte b of row n holds bits 8b .. 8b+7 of the row's code stream, code j at bits
// [BITS*j, BITS*j + BITS), least significant bit first.
template <int BITS>
__global__ __launch_bounds__(256) void k_pack_codes(const uint8_t* __restrict__ codes, int N, int K,
                                                    uint8_t* __restrict__ packed, int64_t row_bytes) {
  const int64_t t = blockIdx.x * 256ll + threadIdx.x;
  if (t >= (int64_t)N * row_bytes) return;
  const int n = (int)(t / row_bytes);
  const int64_t b = t - (int64_t)n * row_bytes;
  const uint8_t* c = codes + (int64_t)n * K;
  unsigned v = 0;
  const int64_t bit0 = 8 * b;
  for (int64_t j = bit0 / BITS; j < K && j * BITS < bit0 + 8; ++j) {
    const int64_t sh = j * BITS - bit0;  // may be negative for the code straddling in
    const unsigned code = c[j] & ((1u << BITS) - 1);
    v |= sh >= 0 ? code << sh : code >> (-sh);
  }
  packed[t] = static_cast<uint8_t>(v & 0xffu);
}

}  // namespace qs

using namespace qs;

extern "C" int qs_quant_rows_int8(const float* W, int64_t ldw, int64_t N, int64_t K, int8_t* q,
                                  int64_t ldq, float* scales, void* stream) {
  if (!W || !q || !scales) return fail(QS_ERR_INVALID, "quant_rows_int8: null pointer");
  if (N < 0 || K <= 0 || ldw < K || ldq < K) return fail(QS_ERR_INVALID, "quant_rows_int8: bad shape");
  if (N > INT_MAX || K > INT_MAX) return fail(QS_ERR_LIMIT, "quant_rows_int8: dimension exceeds int32");
  if (N == 0) return QS_OK;
  const bool vec = K % 4 == 0 && ldw % 4 == 0 && ldq % 4 == 0 && aligned(W, 16) && aligned(q, 4);
  if (vec && K <= 4096)
    hipLaunchKernelGGL(k_quant_int8_r, dim3((unsigned)cdiv(N, 4)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       W, ldw, (int)N, (int)K, q, ldq, scales);
  else if (vec)
    hipLaunchKernelGGL(k_quant_int8_v, dim3((unsigned)cdiv(N, 4)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       W, ldw, (int)N, (int)K, q, ldq, scales);
  else
    hipLaunchKernelGGL(k_quant_int8, dim3((unsigned)cdiv(N, 4)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       W, ldw, (int)N, (int)K, q, ldq, scales);
  return hip_check(hipGetLastError(), "k_quant_int8 launch");
}

extern "C" int qs_quant_rows_lowbit(const float* W, int64_t ldw, int64_t N, int64_t K, int bits, int G,
                                    uint8_t* packed, int64_t row_bytes, float* scales, uint8_t* codes,
                                    void* stream) {
  if (!W || !packed || !scales || !codes) return fail(QS_ERR_INVALID, "quant_rows_lowbit: null pointer");
  if (bits != 2 && bits != 3) return fail(QS_ERR_UNSUPPORTED, "quant_rows_lowbit: bits must be 2 or 3");
  if (N < 0 || K <= 0 || G <= 0 || ldw < K) return fail(QS_ERR_INVALID, "quant_rows_lowbit: bad shape");
  if (row_bytes != (K * bits + 7) / 8) return fail(QS_ERR_INVALID, "quant_rows_lowbit: row_bytes must be ceil(K*bits/8)");
  if (N * K > ((int64_t)1 << 40) || K > INT_MAX || G > (1 << 24))
    return fail(QS_ERR_LIMIT, "quant_rows_lowbit: shape too large");
  if (N == 0) return QS_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t ng = cdiv(K, G);
  if (G == 128 && K % 128 == 0 && ldw % 4 == 0 && aligned(W, 16)) {
    const unsigned gg = (unsigned)cdiv(N * ng, 8);  // 8 groups per 256-thread workgroup
    if (bits == 3)
      hipLaunchKernelGGL(k_quant_g128<3>, dim3(gg), dim3(256), 0, s, W, ldw, (int)N, (int)K, scales, packed, row_bytes);
    else
      hipLaunchKernelGGL(k_quant_g128<2>, dim3(gg), dim3(256), 0, s, W, ldw, (int)N, (int)K, scales, packed, row_bytes);
    return hip_check(hipGetLastError(), "k_quant_g128 launch");
  }
  const unsigned gq = (unsigned)cdiv(N * ng, 256), gp = (unsigned)cdiv(N * row_bytes, 256);
  if (bits == 3) {
    hipLaunchKernelGGL(k_quant_groups<3>, dim3(gq), dim3(256), 0, s, W, ldw, (int)N, (int)K, G, scales, codes);
    hipLaunchKernelGGL(k_pack_codes<3>, dim3(gp), dim3(256), 0, s, codes, (int)N, (int)K, packed, row_bytes);
  } else {
    hipLaunchKernelGGL(k_quant_groups<2>, dim3(gq), dim3(256), 0, s, W, ldw, (int)N, (int)K, G, scales, codes);
    hipLaunchKernelGGL(k_pack_codes<2>, dim3(gp), dim3(256), 0, s, codes, (int)N, (int)K, packed, row_bytes);
  }
  return hip_check(hipGetLastError(), "qs_quant_rows_lowbit launch");
}
