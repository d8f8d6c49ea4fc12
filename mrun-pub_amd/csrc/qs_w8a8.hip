// W8A8: per-token int8 activation quantization + int8 x int8 -> int32 MFMA GEMM with a
// fused dequant epilogue, and the fp32 outlier side path (LLM.int8 style).
//
// Kernels
//   k_act_quant      : per row, s = max|x*keep| / 127 (0 -> 1), q = clamp(rint(x*keep / s))
//                      -- one IEEE fp32 multiply/divide per element, round-half-even, the
//                      exact recipe of the reference (bit-exact codes and scales).
//   k_col_absmax(_rows): max over rows of |x[:, k]| (outlier column detection; one pass
//                      without atomics for M <= 1024).
//   k_topk           : the k largest column maxima (ties -> lower column index).
//   k_gather_side    : xp[m, p] = x[m, idx[p]], wp[n, p] = float(qw[n, idx[p]]) * sw[n].
//   k_gemm_i8<...>   : C = A[M,K] . B[N,K]^T with v_mfma_i32_32x32x32_i8, 128/64-byte K
//                      steps staged through padded, double-buffered LDS tiles, an XCD-aware
//                      tile order, and one of three epilogues: raw int32, or
//                      y = side + (float(acc) * a_scale[m]) * b_scale[n] in fp32 / bf16.
//   k_gemm_i8_generic: any shape (one thread per output, exact int32).
//
// MFMA operand mapping (32x32x32 i8, wave64): lane l supplies row (l & 31) of A and
// column (l & 31) of B with 16 int8 of the k half (l >> 5); A and B use the same
// lane -> k assignment, so each lane just loads 16 contiguous bytes at k = 16*(l>>5) of
// its row.  Accumulator register r of lane l holds
// C[8*(r/4) + 4*(l>>5) + (r%4)][l & 31].
#include "qs_common.h"

#include <type_traits>

namespace qs {

typedef int i32x16 __attribute__((ext_vector_type(16)));

// ----------------------------------------------------------------------------------
// activation quantization
// ----------------------------------------------------------------------------------
template <int XT>
__device__ __forceinline__ float load_x(const void* x, int64_t i) {
  if constexpr (XT == QS_F32) return static_cast<const float*>(x)[i];
  else if constexpr (XT == QS_BF16) return bf16_bits_to_f32(static_cast<const uint16_t*>(x)[i]);
  else return f16_bits_to_f32(static_cast<const uint16_t*>(x)[i]);
}

// One workgroup per row.  keep (nullable) multiplies x before everything (protected
// outlier columns carry 0, the rest 1).
template <int XT>
__global__ __launch_bounds__(256) void k_act_quant(const void* __restrict__ x, int64_t ldx,
                                                   const float* __restrict__ keep,
                                                   int8_t* __restrict__ q, int64_t ldq,
                                                   float* __restrict__ scale, int K) {
  const int64_t row = blockIdx.x;
  const void* xr = static_cast<const char*>(x) + row * ldx * (XT == QS_F32 ? 4 : 2);
  float amax = 0.f;
  for (int k = threadIdx.x; k < K; k += 256) {
    float v = load_x<XT>(xr, k);
    if (keep) v = mul_rn(v, keep[k]);
    amax = fmaxf(amax, fabsf(v));
  }
  amax = wave_max(amax);
  __shared__ float red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float s = amax / 127.0f;  // IEEE division
  if (s == 0.f) s = 1.f;
  if (threadIdx.x == 0) scale[row] = s;
  int8_t* qr = q + row * ldq;
  for (int k = threadIdx.x; k < K; k += 256) {
    float v = load_x<XT>(xr, k);
    if (keep) v = mul_rn(v, keep[k]);
    float r = rintf(v / s);  // IEEE division, round half to even
    r = fminf(fmaxf(r, -127.f), 127.f);
    qr[k] = static_cast<int8_t>(r);
  }
}

template <int XT, int CPL, int WPR>
struct QuantRow {
  i32x4 v[CPL];
};

// The row's chunks of this lane into registers (zero loads for rows >= M).
template <int XT, int CPL, int WPR>
__device__ __forceinline__ void act_quant_load(const void* __restrict__ x, int64_t ldx, int row, int M, int K,
                                               QuantRow<XT, CPL, WPR>& qr) {
  constexpr int ES = XT == QS_F32 ? 4 : 2;
  constexpr int E = 16 / ES;
  const int lane = threadIdx.x & 63, wr = (threadIdx.x >> 6) % WPR;
  const bool live = row < M;
  const char* xr = static_cast<const char*>(x) + (int64_t)(live ? row : 0) * ldx * ES;
  const int nch = K / E;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = (c * WPR + wr) * 64 + lane;
    if (live && ch < nch) qr.v[c] = *reinterpret_cast<const i32x4*>(xr + (int64_t)ch * 16);
  }
}

// Scale and codes of the row from the loaded chunks.  keep4(ch, h) gives the keep factors
// of elements 4h..4h+3 of chunk ch (has_keep false: no factors).  Every thread of the
// workgroup reaches the barrier (WPR > 1).
template <int XT, int CPL, int WPR, class KeepF>
__device__ __forceinline__ void act_quant_compute(const QuantRow<XT, CPL, WPR>& qrow, bool has_keep, KeepF keep4,
                                                  int8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale,
                                                  int row, int M, int K) {
  constexpr int ES = XT == QS_F32 ? 4 : 2;
  constexpr int E = 16 / ES;  // elements per 16-byte chunk
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wr = wave % WPR;
  const bool live = row < M;
  const int nch = K / E;
  float amax = 0.f;
  auto widen = [&](const i32x4& c, int e) -> float {
    if constexpr (XT == QS_F32) return __int_as_float(c[e]);
    const uint32_t d = static_cast<uint32_t>(c[e >> 1]);
    const uint32_t h = (e & 1) ? (d >> 16) : (d & 0xffffu);
    if constexpr (XT == QS_BF16) return bf16_bits_to_f32(h);
    return f16_bits_to_f32(static_cast<uint16_t>(h));
  };
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = (c * WPR + wr) * 64 + lane;
    if (live && ch < nch) {
      if (has_keep) {
#pragma unroll
        for (int h = 0; h < E / 4; ++h) {
          const f32x4 kv = keep4(ch, h);
#pragma unroll
          for (int e = 0; e < 4; ++e) amax = fmaxf(amax, fabsf(mul_rn(widen(qrow.v[c], 4 * h + e), kv[e])));
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) amax = fmaxf(amax, fabsf(widen(qrow.v[c], e)));
      }
    }
  }
  amax = wave_max(amax);
  if constexpr (WPR > 1) {  // max is exact in any order
    __shared__ float wmax[4];
    if (lane == 0) wmax[wave] = amax;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < WPR; ++j) amax = fmaxf(amax, wmax[(wave / WPR) * WPR + j]);
  }
  if (!live) return;
  float s = amax / 127.0f;  // IEEE division
  if (s == 0.f) s = 1.f;
  if (lane == 0 && wr == 0) scale[row] = s;
  int8_t* qr = q + (int64_t)row * ldq;
  const float rs = 1.0f / s;  // correctly rounded
  // row-uniform: bf16 rows with s >= 2^-120 take the corrected quotient (the same codes as
  // the IEEE division for every bf16 element, x * keep included), others divide
  const bool fast = XT == QS_BF16 && s >= 0x1p-120f;
  auto quantize = [&](auto fast_tag) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ch = (c * WPR + wr) * 64 + lane;
      if (ch < nch) {
        uint32_t packed[E / 4];
#pragma unroll
        for (int j = 0; j < E / 4; ++j) packed[j] = 0;
        f32x4 kv[E / 4];
#pragma unroll
        for (int h = 0; h < E / 4; ++h) kv[h] = has_keep ? keep4(ch, h) : f32x4{1.f, 1.f, 1.f, 1.f};
#pragma unroll
        for (int e = 0; e < E; ++e) {
          float f = widen(qrow.v[c], e);
          if (has_keep) f = mul_rn(f, kv[e >> 2][e & 3]);
          float r = rintf(decltype(fast_tag)::value ? quot_markstein(f, s, rs) : f / s);  // half to even
          r = fminf(fmaxf(r, -127.f), 127.f);
          packed[e >> 2] |= (static_cast<uint32_t>(static_cast<int>(r)) & 0xffu) << (8 * (e & 3));
        }
        if constexpr (E == 8)
          *reinterpret_cast<uint2*>(qr + (int64_t)ch * 8) = make_uint2(packed[0], packed[1]);
        else
          *reinterpret_cast<uint32_t*>(qr + (int64_t)ch * 4) = packed[0];
      }
    }
  };
  if (fast) quantize(std::true_type{});
  else quantize(std::false_type{});
}

// WPR waves per row (1, or 4 for short batches) with the row held in registers between
// the max pass and the quantize pass: lane l of the row's wave wr owns the 16-byte chunks
// (c * WPR + wr) * 64 + l (each wave instruction reads 1 KiB contiguous); the waves'
// maxima meet in LDS.  Same arithmetic, element by element, as k_act_quant.
// Requires K % E == 0, 16-byte aligned rows of x, 8/4-byte aligned rows of q and
// K <= 64 * WPR * CPL * E.
template <int XT, int CPL, int WPR>
__global__ __launch_bounds__(256) void k_act_quant_w(const void* __restrict__ x, int64_t ldx,
                                                     const float* __restrict__ keep,
                                                     int8_t* __restrict__ q, int64_t ldq,
                                                     float* __restrict__ scale, int M, int K) {
  constexpr int E = XT == QS_F32 ? 4 : 8;
  const int row = blockIdx.x * (4 / WPR) + (int)(threadIdx.x >> 6) / WPR;
  // keep mask of chunk ch: E floats at keep + ch*E (16-byte aligned), read as float4s
  auto keep4 = [&](int ch, int h) -> f32x4 { return reinterpret_cast<const f32x4*>(keep + ch * E)[h]; };
  QuantRow<XT, CPL, WPR> qr;
  act_quant_load<XT, CPL, WPR>(x, ldx, row, M, K, qr);
  act_quant_compute<XT, CPL, WPR>(qr, keep != nullptr, keep4, q, ldq, scale, row, M, K);
}

// Column maxima: block (bx, by) covers 256 columns x 64 rows and folds the max over its
// rows of |x[m, k]| into colmax[k] (zeroed beforehand by k_fill_zero).
template <int XT>
__global__ __launch_bounds__(256) void k_col_absmax(const void* __restrict__ x, int64_t ldx,
                                                    int M, int K, float* __restrict__ part) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  if (k >= K) return;
  const int m0 = blockIdx.y * 64;
  const int m1 = min(M, m0 + 64);
  float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int m = m0;
  for (; m + 8 <= m1; m += 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = fmaxf(a[j], fabsf(load_x<XT>(x, (int64_t)(m + j) * ldx + k)));
  }
  for (; m < m1; ++m) a[0] = fmaxf(a[0], fabsf(load_x<XT>(x, (int64_t)m * ldx + k)));
  float r = a[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) r = fmaxf(r, a[j]);
  // non-negative floats order like their bit patterns: an integer max is the float max,
  // exact and independent of the order in which the row blocks arrive
  atomicMax(reinterpret_cast<unsigned int*>(part) + k, __float_as_uint(r));
}

// Column maxima in one pass for short batches: workgroup (bx, by) covers 64 columns of
// rows [1024 by, 1024 by + 1024) with 16 row groups (rows g, g + 16, ...), combined
// through LDS; writes colmax[by * K + k] directly, so no zero fill and no atomics (one
// row of partial maxima per 1024 rows).
template <int XT>
__global__ __launch_bounds__(1024) void k_col_absmax_rows(const void* __restrict__ x, int64_t ldx,
                                                          int M, int K, float* __restrict__ colmax) {
  __shared__ float red[16][64];
  const int c = blockIdx.x * 64 + (threadIdx.x & 63), g = threadIdx.x >> 6;
  const int r0 = (int)blockIdx.y * 1024;
  M = min(M, r0 + 1024);
  colmax += (int64_t)blockIdx.y * K;
  float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (c < K) {
    int m = r0 + g;
    for (; m + 7 * 16 < M; m += 8 * 16) {
#pragma unroll
      for (int j = 0; j < 8; ++j) a[j] = fmaxf(a[j], fabsf(load_x<XT>(x, (int64_t)(m + 16 * j) * ldx + c)));
    }
    for (; m < M; m += 16) a[0] = fmaxf(a[0], fabsf(load_x<XT>(x, (int64_t)m * ldx + c)));
  }
  float r = a[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) r = fmaxf(r, a[j]);
  red[g][threadIdx.x & 63] = r;
  __syncthreads();
  if (g == 0 && c < K) {
#pragma unroll
    for (int j = 1; j < 16; ++j) r = fmaxf(r, red[j][threadIdx.x]);
    colmax[c] = r;
  }
}

// k_col_absmax_rows with 16-byte loads (rows 16-byte aligned): lane l of wave w holds
// the E columns 64 bx + E (l % CG) of rows w RPI + l / CG + 16 RPI i, four rows' loads in
// flight at a time; lanes of one column group meet by shuffles, the 16 waves through LDS.
template <int XT>
__global__ __launch_bounds__(1024) void k_col_absmax_v(const void* __restrict__ x, int64_t ldx, int M, int K,
                                                       float* __restrict__ colmax) {
  constexpr int ES = XT == QS_F32 ? 4 : 2, E = 16 / ES, CG = 64 / E, RPI = 64 / CG;
  __shared__ float red[16][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int cg = lane % CG, ro = lane / CG;
  const int c0 = (int)blockIdx.x * 64 + cg * E;
  const int r0 = (int)blockIdx.y * 1024, r1 = min(M, r0 + 1024);
  auto widen = [&](const i32x4& c, int e) -> float {
    if constexpr (XT == QS_F32) return __int_as_float(c[e]);
    const uint32_t d = static_cast<uint32_t>(c[e >> 1]);
    const uint32_t h = (e & 1) ? (d >> 16) : (d & 0xffffu);
    if constexpr (XT == QS_BF16) return bf16_bits_to_f32(h);
    return f16_bits_to_f32(static_cast<uint16_t>(h));
  };
  float a[E];
#pragma unroll
  for (int e = 0; e < E; ++e) a[e] = 0.f;
  if (c0 < K) {  // K % E == 0: a lane's E columns are all in range or all out
    const char* xb = static_cast<const char*>(x) + (int64_t)c0 * ES;
    for (int m = r0 + w * RPI + ro; m < r1; m += 4 * 16 * RPI) {
      i32x4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int mu = m + u * 16 * RPI;
        v[u] = mu < r1 ? *reinterpret_cast<const i32x4*>(xb + (int64_t)mu * ldx * ES) : i32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < E; ++e) a[e] = fmaxf(a[e], fabsf(widen(v[u], e)));
    }
  }
#pragma unroll
  for (int off = CG; off < 64; off <<= 1)
#pragma unroll
    for (int e = 0; e < E; ++e) a[e] = fmaxf(a[e], __shfl_xor(a[e], off));
  if (ro == 0)
#pragma unroll
    for (int e = 0; e < E; ++e) red[w][cg * E + e] = a[e];
  __syncthreads();
  if (threadIdx.x < 64) {
    const int c = (int)blockIdx.x * 64 + (int)threadIdx.x;
    float r = red[0][threadIdx.x];
#pragma unroll
    for (int j = 1; j < 16; ++j) r = fmaxf(r, red[j][threadIdx.x]);
    if (c < K) colmax[(int64_t)blockIdx.y * K + c] = r;
  }
}

__global__ __launch_bounds__(256) void k_fill_zero(float* __restrict__ p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// Single workgroup: kk rounds of a block-wide argmax over vals[0..K).  Selected entries
// are excluded by index; ties go to the lower index.  Emits int64 indices (descending
// value order) and the keep mask (1 everywhere, 0 at the selected columns).
// vals holds `parts` partial rows [parts, K]; they are first folded into row 0.
__global__ __launch_bounds__(1024) void k_topk(float* __restrict__ vals, int K, int parts, int kk,
                                               int64_t* __restrict__ idx, float* __restrict__ keep) {
  __shared__ float bv[16];
  __shared__ int bi[16];
  __shared__ int chosen[64];
  for (int k = threadIdx.x; k < K; k += 1024) {
    float v = vals[k];
    for (int p = 1; p < parts; ++p) v = fmaxf(v, vals[(int64_t)p * K + k]);
    vals[k] = v;
    keep[k] = 1.f;
  }
  __syncthreads();
  for (int round = 0; round < kk; ++round) {
    float best = -1.f;
    int besti = 0x7fffffff;
    for (int k = threadIdx.x; k < K; k += 1024) {
      bool taken = false;
      for (int j = 0; j < round; ++j) taken |= chosen[j] == k;
      if (taken) continue;
      const float v = vals[k];
      if (v > best || (v == best && k < besti)) {
        best = v;
        besti = k;
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(best, off, 64);
      const int oi = __shfl_xor(besti, off, 64);
      if (ov > best || (ov == best && oi < besti)) {
        best = ov;
        besti = oi;
      }
    }
    if ((threadIdx.x & 63) == 0) {
      bv[threadIdx.x >> 6] = best;
      bi[threadIdx.x >> 6] = besti;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float b = bv[0];
      int i = bi[0];
      for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
        if (bv[w] > b || (bv[w] == b && bi[w] < i)) {
          b = bv[w];
          i = bi[w];
        }
      chosen[round] = i;
      idx[round] = i;
      keep[i] = 0.f;
    }
    __syncthreads();
  }
}

// One step of a wave argmax over (value desc, index asc) on the DPP network.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void argmax_dpp_step(float& best, int& bi) {
  const int vb = __float_as_int(best);
  const float ov = __int_as_float(__builtin_amdgcn_update_dpp(vb, vb, CTRL, ROW_MASK, 0xf, false));
  const int oi = __builtin_amdgcn_update_dpp(bi, bi, CTRL, ROW_MASK, 0xf, false);
  if (ov > best || (ov == best && oi < bi)) {
    best = ov;
    bi = oi;
  }
}

// Wave argmax: quad swaps, row half-mirror and mirror, then row broadcasts 15 and 31
// carry the winner to lane 63, which is broadcast to all lanes.
__device__ __forceinline__ void wave_argmax_dpp(float& best, int& bi) {
  argmax_dpp_step<0xB1, 0xf>(best, bi);   // quad_perm [1,0,3,2]
  argmax_dpp_step<0x4E, 0xf>(best, bi);   // quad_perm [2,3,0,1]
  argmax_dpp_step<0x141, 0xf>(best, bi);  // row_half_mirror
  argmax_dpp_step<0x140, 0xf>(best, bi);  // row_mirror
  argmax_dpp_step<0x142, 0xa>(best, bi);  // row_bcast:15
  argmax_dpp_step<0x143, 0xc>(best, bi);  // row_bcast:31
  best = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(best), 63));
  bi = __builtin_amdgcn_readlane(bi, 63);
}

// Single workgroup of 16 waves.  The partial maxima are folded into registers (wave w
// owns columns [w*S, (w+1)*S), lane l the columns w*S + l + 64*e); every wave selects the
// kk largest of its slice with kk rounds of a wave argmax, and wave 0 merges the 16
// candidate lists the same way.  Ties go to the lower column index at every step, so the
// result equals kk rounds of a global argmax.  K <= 16 * 64 * kTopkVpl.
constexpr int kTopkVpl = 16;
__global__ __launch_bounds__(1024) void k_topk_w(const float* __restrict__ vals, int K, int parts,
                                                 int kk, int64_t* __restrict__ idx,
                                                 float* __restrict__ keep) {
  __shared__ float cv[16 * 64];
  __shared__ int ci[16 * 64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int S = (K + 15) / 16;
  const int base = wave * S;
  const float NEG = -__builtin_inff();
  float v[kTopkVpl];
#pragma unroll
  for (int e = 0; e < kTopkVpl; ++e) {
    const int off = e * 64 + lane;
    const int k = base + off;
    v[e] = NEG;
    if (off < S && k < K) {
      float m = vals[k];
      for (int pp = 1; pp < parts; ++pp) m = fmaxf(m, vals[(int64_t)pp * K + k]);
      v[e] = m;
      keep[k] = 1.f;
    }
  }
  auto argmax = [&](float& best, int& bi) { wave_argmax_dpp(best, bi); };
  for (int r = 0; r < kk; ++r) {
    float best = NEG;
    int bi = 0x7fffffff;
#pragma unroll
    for (int e = 0; e < kTopkVpl; ++e) {
      const int k = base + e * 64 + lane;
      if (v[e] > best || (v[e] == best && k < bi)) {
        best = v[e];
        bi = k;
      }
    }
    argmax(best, bi);
    if (lane == 0) {
      cv[wave * 64 + r] = best;
      ci[wave * 64 + r] = bi;
    }
#pragma unroll
    for (int e = 0; e < kTopkVpl; ++e)
      if (base + e * 64 + lane == bi) v[e] = NEG;
  }
  __syncthreads();
  if (wave != 0) return;
  // wave 0: merge 16 lists of kk candidates (entry j = w * kk + r, lane owns j = lane + 64 t)
  float c[16];
  int cidx[16];
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    const int j = lane + 64 * t;
    c[t] = NEG;
    cidx[t] = 0x7fffffff;
    if (j < 16 * kk) {
      const int w = j / kk, r = j - (j / kk) * kk;
      c[t] = cv[w * 64 + r];
      cidx[t] = ci[w * 64 + r];
    }
  }
  for (int r = 0; r < kk; ++r) {
    float best = NEG;
    int bi = 0x7fffffff;
#pragma unroll
    for (int t = 0; t < 16; ++t)
      if (c[t] > best || (c[t] == best && cidx[t] < bi)) {
        best = c[t];
        bi = cidx[t];
      }
    argmax(best, bi);
    if (lane == 0) {
      idx[r] = bi;
      keep[bi] = 0.f;
    }
#pragma unroll
    for (int t = 0; t < 16; ++t)
      if (cidx[t] == bi) c[t] = NEG;
  }
}

// Top-k by radix selection (single workgroup, 1024 threads, K <= 1024 * kRadixVpt).
// Every column gets the 64-bit key (value bits << 32) | ~index: values are >= 0, so the
// key order is value descending, then index ascending, and all keys are distinct.  The
// kk-th largest key T is found one byte at a time from the top (histogram of the byte
// among the keys that match the prefix found so far, then a suffix scan over the 256
// bins); the selection is every key >= T, exactly kk columns.  The value bytes settle T
// unless the value at the threshold is tied, in which case the index bytes follow.  The
// kk selected keys are finally ranked against each other to emit idx in order.
constexpr int kRadixVpt = 16;
// Adds one count per active lane to hist[bin].  Lanes that share the leader's bin are
// combined into one LDS atomic per round; the rounds stop once a round combines fewer
// than 8 lanes (spread bins), and the remaining lanes add one atomic each.  The first
// digit of float keys lands in one or two bins, where per-lane atomics serialise.
__device__ __forceinline__ void hist_add_wave(unsigned* hist, bool active, unsigned bin) {
  unsigned long long act = __ballot(active);
  const int lane = threadIdx.x & 63;
  while (act) {
    const int leader = __builtin_ctzll(act);
    const unsigned lb = __builtin_amdgcn_readlane(bin, leader);
    const unsigned long long same = __ballot(((act >> lane) & 1ull) && bin == lb);
    const int n = __popcll(same);
    if (lane == leader) atomicAdd(&hist[lb], (unsigned)n);
    act &= ~same;
    if (n < 8) break;
  }
  if ((act >> lane) & 1ull) atomicAdd(&hist[bin], 1u);
}

// One step of a wave-wide 64-bit maximum through DPP: lanes whose source lane is outside
// the pattern (or whose row is masked off) keep their own value.
template <int CTRL, int ROWS>
__device__ __forceinline__ unsigned long long dpp_max_u64(unsigned long long v) {
  const int lo = (int)(unsigned)v, hi = (int)(unsigned)(v >> 32);
  const unsigned olo = (unsigned)__builtin_amdgcn_update_dpp(lo, lo, CTRL, ROWS, 0xf, false);
  const unsigned ohi = (unsigned)__builtin_amdgcn_update_dpp(hi, hi, CTRL, ROWS, 0xf, false);
  const unsigned long long o = ((unsigned long long)ohi << 32) | olo;
  return o > v ? o : v;
}

// Maximum over the wave, returned to every lane: row_shr 1, 2, 4, 8 leave each 16-lane
// row's maximum in its lane 15; row_bcast 15 (rows 1, 3) and row_bcast 31 (rows 2, 3)
// carry it to lane 63, which is read back as a scalar.
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
  v = dpp_max_u64<0x111, 0xf>(v);
  v = dpp_max_u64<0x112, 0xf>(v);
  v = dpp_max_u64<0x114, 0xf>(v);
  v = dpp_max_u64<0x118, 0xf>(v);
  v = dpp_max_u64<0x142, 0xa>(v);
  v = dpp_max_u64<0x143, 0xc>(v);
  const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)v, 63);
  const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(v >> 32), 63);
  return ((unsigned long long)hi << 32) | lo;
}

// Small k (kk <= 16): the same 64-bit keys as k_topk_radix ((value bits << 32) | ~column:
// larger value first, lower column on ties; keys are unique, and real keys are > 0).
// Filter: the 16 wave maxima are 16 distinct keys, so with kk <= 16 every top-kk key is
// >= T, the smallest wave maximum.  The keys >= T (a few dozen for ordinary data) are
// compacted into LDS and wave 0 selects from them by kk rounds of a wave-wide maximum.
// When more than 256 pass (ties across many columns), each wave first takes its own top
// kk the same way and wave 0 selects from those 16 * kk candidates.  Emits idx in
// descending key order and the keep mask.
template <int VPT>
__global__ __launch_bounds__(1024) void k_topk_small(const float* __restrict__ vals, int K, int kk,
                                                     int64_t* __restrict__ idx, float* __restrict__ keep) {
  constexpr int kCand = 256;
  __shared__ unsigned long long cand[kCand];
  __shared__ unsigned long long sel[16];
  __shared__ unsigned long long wmax[16];
  __shared__ int ncand;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid == 0) ncand = 0;
  unsigned long long key[VPT];
  unsigned long long mine = 0ull;
#pragma unroll
  for (int e = 0; e < VPT; ++e) {
    const int k = tid + 1024 * e;
    key[e] = k < K ? (((unsigned long long)__float_as_uint(vals[k]) << 32) | (unsigned)(~(unsigned)k)) : 0ull;
    if (k < K) keep[k] = 1.f;
    mine = key[e] > mine ? key[e] : mine;
  }
  auto wave_top = [&](unsigned long long* keys, int n) {
    unsigned long long best = 0ull;
    for (int e = 0; e < n; ++e) best = keys[e] > best ? keys[e] : best;
    best = wave_max_u64(best);
    for (int e = 0; e < n; ++e)
      if (keys[e] == best) keys[e] = 0ull;
    return best;
  };
  // wave 0: the final kk from 4 candidates per lane
  auto final_select = [&](unsigned long long (&c)[4]) {
    for (int r = 0; r < kk; ++r) {
      const unsigned long long b = wave_top(c, 4);
      if (lane == 0) {
        sel[r] = b;
        idx[r] = (int64_t)(~(unsigned)(b & 0xffffffffull));
      }
    }
  };
  const unsigned long long wm = wave_max_u64(mine);
  if (lane == 0) wmax[wave] = wm;
  __syncthreads();
  unsigned long long T = wmax[0];
#pragma unroll
  for (int w = 1; w < 16; ++w) T = wmax[w] < T ? wmax[w] : T;
#pragma unroll
  for (int e = 0; e < VPT; ++e)
    if (key[e] != 0ull && key[e] >= T) {
      const int pos = atomicAdd(&ncand, 1);
      if (pos < kCand) cand[pos] = key[e];
    }
  __syncthreads();
  const int n = ncand;  // the same for every thread: the branch below is uniform
  if (n <= kCand) {
    if (wave == 0) {
      unsigned long long c[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = lane + 64 * j < n ? cand[lane + 64 * j] : 0ull;
      final_select(c);
    }
  } else {
    __syncthreads();  // every thread has read ncand before cand is reused
    for (int r = 0; r < kk; ++r) {
      const unsigned long long b = wave_top(key, VPT);
      if (lane == 0) cand[wave * 16 + r] = b;
    }
    __syncthreads();
    if (wave == 0) {
      unsigned long long c[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = lane + 64 * j;  // candidate (wave i / 16, rank i % 16)
        c[j] = (i % 16) < kk ? cand[i] : 0ull;
      }
      final_select(c);
    }
  }
  __syncthreads();  // every keep = 1 store precedes the zeros
  if (tid < kk) keep[~(unsigned)(sel[tid] & 0xffffffffull)] = 0.f;
}

__global__ __launch_bounds__(1024) void k_topk_radix(const float* __restrict__ vals, int K, int kk,
                                                     int64_t* __restrict__ idx, float* __restrict__ keep) {
  __shared__ unsigned hist[256];
  __shared__ unsigned long long s_prefix;  // bytes of T found so far (top bytes)
  __shared__ unsigned s_need;               // keys still to take inside the prefix bucket
  __shared__ unsigned s_bucket;             // keys in the prefix bucket
  __shared__ unsigned wsum[4];
  __shared__ int s_nsel;
  __shared__ unsigned long long sel[64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  unsigned long long key[kRadixVpt];
#pragma unroll
  for (int e = 0; e < kRadixVpt; ++e) {
    const int k = tid + 1024 * e;
    // columns past K are never counted or selected
    const unsigned v = k < K ? __float_as_uint(vals[k]) : 0u;
    key[e] = ((unsigned long long)v << 32) | (unsigned)(~(unsigned)k);
    if (k < K) keep[k] = 1.f;
  }
  if (tid == 0) {
    s_prefix = 0ull;
    s_need = (unsigned)kk;
    s_nsel = 0;
  }
  unsigned long long mask = 0ull;
  for (int pass = 0; pass < 8; ++pass) {
    const int shift = 56 - 8 * pass;
    if (tid < 256) hist[tid] = 0u;
    __syncthreads();
    const unsigned long long prefix = s_prefix;
#pragma unroll
    for (int e = 0; e < kRadixVpt; ++e)
      if (1024 * e < K)  // block-uniform: skip register rows that hold no column
        hist_add_wave(hist, tid + 1024 * e < K && (key[e] & mask) == prefix,
                      (unsigned)(key[e] >> shift) & 255u);
    __syncthreads();
    // suffix scan: thread t < 256 takes bin 255 - t; inclusive prefix over t
    unsigned h = 0, c = 0;
    if (tid < 256) {
      h = hist[255 - tid];
      c = h;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const unsigned o = __shfl_up(c, off, 64);
        if (lane >= off) c += o;
      }
      if (lane == 63) wsum[wave] = c;
    }
    __syncthreads();
    if (tid < 256) {
      unsigned base = 0;
      for (int w = 0; w < wave; ++w) base += wsum[w];
      const unsigned incl = base + c, excl = incl - h;
      const unsigned need = s_need;
      if (excl < need && incl >= need) {  // exactly one bin holds the need-th key
        s_prefix = prefix | ((unsigned long long)(255 - tid) << shift);
        s_need = need - excl;
        s_bucket = h;
      }
    }
    __syncthreads();
    mask |= 0xffull << shift;
    // the whole bucket is taken: T is its smallest key, no further bytes needed
    if (s_need == s_bucket) break;
  }
  // T: the smallest selected key; with a full bucket, every key of the bucket qualifies
  const unsigned long long prefix = s_prefix;
  const bool full = s_need == s_bucket;
#pragma unroll
  for (int e = 0; e < kRadixVpt; ++e) {
    const bool take = tid + 1024 * e < K && (full ? ((key[e] & mask) >= prefix) : (key[e] >= prefix));
    if (take) {
      const int slot = atomicAdd(&s_nsel, 1);
      if (slot < 64) sel[slot] = key[e];
    }
  }
  __syncthreads();
  if (tid < kk) {
    const unsigned long long my = sel[tid];
    int rank = 0;
    for (int j = 0; j < kk; ++j) rank += sel[j] > my;
    const int col = (int)(~(unsigned)my);
    idx[rank] = col;
    keep[col] = 0.f;
  }
}

// The protect_k front end of w8a8_matmul in one launch after the column maxima.  Every
// workgroup takes the kk largest column maxima (the keys and order of k_topk_small:
// value bits above ~column, kk rounds of a block-wide maximum over the maxima staged in
// LDS), quantizes its activation rows with those columns' keep factor 0 (act_quant_*,
// the factors read from an LDS bitmap), gathers its rows' side activations
// xp[m, p] = x[m, idx[p]] and a 1 / gridDim.x slice of the side weights
// wp[n, p] = float(qw[n, idx[p]]) * sw[n]; workgroup 0 also stores idx, keep and the
// column maxima when asked.  Needs K <= kProtectMaxK (the maxima sit in LDS).
constexpr int kProtectMaxK = 8192;
constexpr int kProtectMaxP = 16;

struct ProtectParams {
  const void* x;
  int64_t ldx;
  int M, K, N;
  const float* colpart;  // [R][K] partial column maxima
  int R;
  int kk;  // protected columns
  const int8_t* qw;
  const float* sw;
  int8_t* q;
  float* scale;
  float* xp;  // [M][kk]
  float* wp;  // [N][kk]
  int64_t* idx;  // optional outputs (workgroup 0)
  float* keep;
  float* colmax;
};

template <int XT, int CPL, int WPR, int VM>
__global__ __launch_bounds__(256) void k_protect_quant(ProtectParams p) {
  static_assert(VM % 4 == 0 && VM * 256 <= kProtectMaxK, "keys per thread");  // K <= 256 VM
  __shared__ uint32_t selbits[kProtectMaxK / 32];
  __shared__ unsigned long long gmax[16];
  __shared__ unsigned long long cand[256];
  __shared__ unsigned long long wbest[2][4];
  __shared__ int sel[kProtectMaxP];
  __shared__ int ncand;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int K = p.K;
  const int row0 = (int)blockIdx.x * (4 / WPR);
  const int row = row0 + wave / WPR;
  if (tid == 0) ncand = 0;
  for (int w = tid; w < (K + 31) / 32; w += 256) selbits[w] = 0u;
  // 1. keys of the column maxima (over the R partial rows): thread tid holds columns
  //    4 tid + 1024 j + e, read as 16-byte vectors (all of a partial row's loads in flight
  //    at once); value bits above ~column, so larger values first, lower column on ties,
  //    and every real key > 0
  f32x4 cv[VM / 4];
#pragma unroll
  for (int j = 0; j < VM / 4; ++j) {
    const int k0 = 4 * tid + 1024 * j;
    cv[j] = k0 < K ? *reinterpret_cast<const f32x4*>(p.colpart + k0) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // 0. this workgroup's activation rows into registers, requested right behind the first
  //    row of maxima (loads complete in order, so the keys wait for the maxima only) and
  //    landing during the selection
  QuantRow<XT, CPL, WPR> qrow;
  act_quant_load<XT, CPL, WPR>(p.x, p.ldx, row, p.M, K, qrow);
  for (int r = 1; r < p.R; ++r) {
    f32x4 w[VM / 4];
#pragma unroll
    for (int j = 0; j < VM / 4; ++j) {
      const int k0 = 4 * tid + 1024 * j;
      w[j] = k0 < K ? *reinterpret_cast<const f32x4*>(p.colpart + (int64_t)r * K + k0) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < VM / 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) cv[j][e] = fmaxf(cv[j][e], w[j][e]);
  }
  unsigned long long key[VM];
  unsigned long long mine = 0ull;
#pragma unroll
  for (int j = 0; j < VM / 4; ++j) {
    const int k0 = 4 * tid + 1024 * j;
    if (k0 < K && p.colmax && blockIdx.x == 0) *reinterpret_cast<f32x4*>(p.colmax + k0) = cv[j];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k = k0 + e;
      key[4 * j + e] = k < K ? ((unsigned long long)__float_as_uint(cv[j][e]) << 32) | (unsigned)(~(unsigned)k) : 0ull;
      mine = key[4 * j + e] > mine ? key[4 * j + e] : mine;
    }
  }
  // 2. the 16 maxima of 16-lane groups are 16 distinct keys (or 0 where a group holds no
  //    column).  T, the smallest of those with fewer than kk larger ones, is the kk-th
  //    largest group maximum (0 when fewer than kk groups hold a column): at least kk keys
  //    are >= T, so each of the kk <= 16 largest keys is >= T.  The keys >= T (about kk
  //    to 2 kk for ordinary data) go to LDS, and each candidate's rank (the candidates
  //    above it) places it: rank < kk is selected, at position rank.
  //    The barriers of the selection wait for LDS only (s_waitcnt lgkmcnt(0) + s_barrier):
  //    the activation rows requested above stay in flight through it.
  unsigned long long g = dpp_max_u64<0x111, 0xf>(mine);
  g = dpp_max_u64<0x112, 0xf>(g);
  g = dpp_max_u64<0x114, 0xf>(g);
  g = dpp_max_u64<0x118, 0xf>(g);
  if ((lane & 15) == 15) gmax[wave * 4 + (lane >> 4)] = g;
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  unsigned long long T;
  {
    const unsigned long long v = gmax[lane & 15];
    int larger = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) larger += gmax[w] > v ? 1 : 0;
    unsigned long long t = larger < p.kk ? ~v : 0ull;  // the row maximum of ~v is ~(min v)
    t = dpp_max_u64<0x111, 0xf>(t);
    t = dpp_max_u64<0x112, 0xf>(t);
    t = dpp_max_u64<0x114, 0xf>(t);
    t = dpp_max_u64<0x118, 0xf>(t);
    const unsigned tlo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)t, 15);
    const unsigned thi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(t >> 32), 15);
    T = ~(((unsigned long long)thi << 32) | tlo);
  }
#pragma unroll
  for (int j = 0; j < VM; ++j)
    if (key[j] != 0ull && key[j] >= T) {  // rare: one LDS atomic per candidate
      const int pos = atomicAdd(&ncand, 1);
      if (pos < 256) cand[pos] = key[j];
    }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  const int n = ncand;  // uniform
  if (n <= 256) {
    if (tid < n) {  // each candidate's rank counts the larger ones
      const unsigned long long my = cand[tid];
      int rank = 0;
#pragma unroll 8
      for (int j = 0; j < n; ++j) rank += cand[j] > my;
      if (rank < p.kk) {
        const int col = (int)(~(unsigned)(my & 0xffffffffull));
        sel[rank] = col;
        atomicOr(&selbits[col >> 5], 1u << (col & 31));
      }
    }
  } else {
    // many ties across columns: kk rounds of a block-wide maximum over the keys
    for (int r = 0; r < p.kk; ++r) {
      unsigned long long best = 0ull;
#pragma unroll
      for (int j = 0; j < VM; ++j) best = key[j] > best ? key[j] : best;
      best = wave_max_u64(best);
      if (lane == 0) wbest[r & 1][wave] = best;
      __syncthreads();
      unsigned long long b = wbest[r & 1][0];
#pragma unroll
      for (int w = 1; w < 4; ++w) b = wbest[r & 1][w] > b ? wbest[r & 1][w] : b;
#pragma unroll
      for (int j = 0; j < VM; ++j)
        if (key[j] == b) key[j] = 0ull;
      if (tid == 0) {
        const int col = (int)(~(unsigned)(b & 0xffffffffull));
        sel[r] = col;
        selbits[col >> 5] |= 1u << (col & 31);
      }
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  // 3. side operands requested now, stored after the quantization (their gathers land
  //    while it runs): the side activations of the workgroup's rows and a slice of the
  //    side weights (kWpPrefetch per thread; a remainder, if any, afterwards)
  const bool xside = tid < (4 / WPR) * p.kk;
  const int xrow = row0 + tid / p.kk, xpp = tid % p.kk;
  float xv = 0.f;
  if (xside && xrow < p.M) xv = load_x<XT>(p.x, (int64_t)xrow * p.ldx + sel[xpp]);
  const int nper = (p.N + (int)gridDim.x - 1) / (int)gridDim.x;
  const int nb = (int)blockIdx.x * nper;
  const int wtot = nper * p.kk;
  constexpr int kWpPrefetch = 4;
  int wqv[kWpPrefetch];
  float wsv[kWpPrefetch];
#pragma unroll
  for (int u = 0; u < kWpPrefetch; ++u) {
    const int i = tid + 256 * u;
    const int n = nb + i / p.kk, pp = i % p.kk;
    wqv[u] = 0;
    wsv[u] = 0.f;
    if (i < wtot && n < p.N) {
      wqv[u] = p.qw[(int64_t)n * K + sel[pp]];
      wsv[u] = p.sw[n];
    }
  }
  // 4. the workgroup's rows, quantized with keep factor 0 at the selected columns
  constexpr int E = XT == QS_F32 ? 4 : 8;
  auto keep4 = [&](int ch, int h) -> f32x4 {
    const int c0 = ch * E + 4 * h;  // a multiple of 4: the 4 bits share a word
    const uint32_t w = selbits[c0 >> 5] >> (c0 & 31);
    return f32x4{(w & 1u) ? 0.f : 1.f, (w & 2u) ? 0.f : 1.f, (w & 4u) ? 0.f : 1.f, (w & 8u) ? 0.f : 1.f};
  };
  act_quant_compute<XT, CPL, WPR>(qrow, true, keep4, p.q, K, p.scale, row, p.M, K);
  // 5. the side operands
  if (xside && xrow < p.M) p.xp[(int64_t)xrow * p.kk + xpp] = xv;
#pragma unroll
  for (int u = 0; u < kWpPrefetch; ++u) {
    const int i = tid + 256 * u;
    const int n = nb + i / p.kk, pp = i % p.kk;
    if (i < wtot && n < p.N) p.wp[(int64_t)n * p.kk + pp] = static_cast<float>(wqv[u]) * wsv[u];
  }
  for (int i = tid + 256 * kWpPrefetch; i < wtot; i += 256) {
    const int n = nb + i / p.kk, pp = i % p.kk;
    if (n < p.N) p.wp[(int64_t)n * p.kk + pp] = static_cast<float>(p.qw[(int64_t)n * K + sel[pp]]) * p.sw[n];
  }
  // 6. the selection itself, when asked
  if (blockIdx.x == 0) {
    if (p.idx && tid < p.kk) p.idx[tid] = sel[tid];
    if (p.keep)
      for (int k = tid; k < K; k += 256) p.keep[k] = ((selbits[k >> 5] >> (k & 31)) & 1u) ? 0.f : 1.f;
  }
}

template <int XT>
__global__ __launch_bounds__(256) void k_gather_side(const void* __restrict__ x, int64_t ldx,
                                                     const int8_t* __restrict__ qw, int64_t ldw,
                                                     const float* __restrict__ sw,
                                                     const int64_t* __restrict__ idx, int P,
                                                     int M, int N, float* __restrict__ xp,
                                                     float* __restrict__ wp) {
  const int64_t i = blockIdx.x * 256ll + threadIdx.x;
  const int64_t nx = (int64_t)M * P;
  if (i < nx) {
    const int64_t m = i / P, pp = i - m * P;
    xp[i] = load_x<XT>(x, m * ldx + idx[pp]);
  } else if (i < nx + (int64_t)N * P) {
    const int64_t j = i - nx;
    const int64_t n = j / P, pp = j - n * P;
    wp[j] = static_cast<float>(qw[n * ldw + idx[pp]]) * sw[n];
  }
}

// ----------------------------------------------------------------------------------
// int8 MFMA GEMM
// ----------------------------------------------------------------------------------
struct GemmParams {
  const int8_t* a;  // [M, K]
  const int8_t* b;  // [N, K]
  int64_t lda, ldb;
  int M, N, K;
  void* c;
  int64_t ldc;
  const float* as;  // [M]   (epilogue 1/2)
  const float* bs;  // [N]
  const float* xp;  // [M, P] side-path activations (nullable)
  const float* wp;  // [N, P] side-path weights
  int P;
};

enum { EPI_I32 = 0, EPI_F32 = 1, EPI_BF16 = 2 };

constexpr int kBK = 64;        // default k bytes per step; LDS rows padded by 16 bytes
constexpr int kSideLds = 16;   // side-path columns per LDS staging in the epilogue
// Epilogue operands fetched by the DMA GEMM ahead of its epilogue ("tail", floats):
// act scales [256], weight scales [256], side activations [BM][P] and weights [BN][P]
// for P <= kTailSide.
constexpr int kTailSide = 8;
constexpr int kTailAs = 0, kTailBs = 256, kTailXp = 512;
template <int BM, int BN>
constexpr int tail_floats() { return kTailXp + (BM + BN) * kTailSide; }

// Epilogue shared by the GEMM kernels: scales, the optional fp32 side path and the store.
// `ws0` is the workgroup's LDS (at least (BM + BN) * (kSideLds + 1) floats), free once the
// main loop's last barrier has passed.  PRE: the scales, and the side operands when
// P <= kTailSide, already sit in LDS at `tail` (layout above), visible to every wave.
template <int BM, int BN, int WM, int WN, int EPI, int NT, int PRE = 0>
__device__ __forceinline__ void gemm_epilogue(const GemmParams& p, i32x16 (&acc)[WM / 32][WN / 32], float* ws0,
                                              int bm, int bn, int wm, int wn, int tid, int lane,
                                              const float* tail = nullptr) {
  constexpr int FM = WM / 32, FN = WN / 32;
  static_assert(!PRE || (EPI != EPI_I32 && BM <= 256 && BN <= 256), "tail layout");
  const bool tside = PRE && p.P > 0 && p.P <= kTailSide;
  // Epilogue.  The side path (P protected columns, fp32) runs on the matrix cores:
  // side[32x32 tile] = xs[rows][P] . ws[P][cols] with v_mfma_f32_32x32x2_f32, whose
  // accumulator layout is the int32 one, so each lane adds side[r] to its own outputs.
  // Operands go through LDS in chunks of kSideLds columns (zero padded); with
  // P <= kSideLds one staging serves every tile.
  const int nsc = (EPI != EPI_I32 && p.P > 0 && !tside) ? (p.P + kSideLds - 1) / kSideLds : 0;
  float* xs = ws0;  // [BM][kSideLds]
  float* ws = xs + BM * kSideLds;                     // [kSideLds][BN]
  auto stage_side = [&](int q0) {
    for (int t = tid; t < BM * kSideLds; t += NT) {
      const int r = t / kSideLds, q = q0 + (t - (t / kSideLds) * kSideLds);
      xs[t] = (bm + r < p.M && q < p.P) ? p.xp[(int64_t)(bm + r) * p.P + q] : 0.f;
    }
    for (int t = tid; t < BN * kSideLds; t += NT) {
      const int c = t / kSideLds, qq = t - (t / kSideLds) * kSideLds, q = q0 + qq;
      ws[qq * BN + c] = (bn + c < p.N && q < p.P) ? p.wp[(int64_t)(bn + c) * p.P + q] : 0.f;
    }
  };
  // the block's activation and weight scales, staged once: read per output from LDS
  // instead of one dependent L2 round trip per output row
  const float* asl = PRE ? tail + kTailAs : ws + kSideLds * BN;  // [BM]
  const float* bsl = PRE ? tail + kTailBs : ws + kSideLds * BN + BM;  // [BN]
  if constexpr (EPI != EPI_I32 && !PRE) {
    float* as_st = ws + kSideLds * BN;
    for (int t = tid; t < BM; t += NT) as_st[t] = bm + t < p.M ? p.as[bm + t] : 0.f;
    for (int t = tid; t < BN; t += NT) as_st[BM + t] = bn + t < p.N ? p.bs[bn + t] : 0.f;
  }
  if (nsc == 1) stage_side(0);
  if ((EPI != EPI_I32 && !PRE) || nsc == 1) __syncthreads();
  typedef float f32x16 __attribute__((ext_vector_type(16)));
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int lr = wm * WM + 32 * i;  // tile row / column offsets within the block
      const int lc = wn * WN + 32 * j;
      f32x16 side = {};
      if (tside) {
        // the same MFMAs, in the same order, as the staged path below
        const float* txp = tail + kTailXp;             // [BM][P]
        const float* twp = tail + kTailXp + BM * kTailSide;  // [BN][P]
        for (int s2 = 0; s2 < p.P; s2 += 2) {
          const int q = s2 + (lane >> 5);
          const float xa = q < p.P ? txp[(lr + (lane & 31)) * p.P + q] : 0.f;
          const float wb = q < p.P ? twp[(lc + (lane & 31)) * p.P + q] : 0.f;
          side = __builtin_amdgcn_mfma_f32_32x32x2f32(xa, wb, side, 0, 0, 0);
        }
      }
      for (int c = 0; c < nsc; ++c) {
        if (nsc > 1) {
          __syncthreads();
          stage_side(c * kSideLds);
          __syncthreads();
        }
        const int qn = min(kSideLds, p.P - c * kSideLds);
        for (int s2 = 0; s2 < qn; s2 += 2) {
          const float xa = xs[(lr + (lane & 31)) * kSideLds + s2 + (lane >> 5)];
          const float wb = ws[(s2 + (lane >> 5)) * BN + lc + (lane & 31)];
          side = __builtin_amdgcn_mfma_f32_32x32x2f32(xa, wb, side, 0, 0, 0);
        }
      }
      const int col = bn + lc + (lane & 31);
      float bsc = 0.f;
      if constexpr (EPI != EPI_I32) bsc = bsl[lc + (lane & 31)];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lrow = lr + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int row = bm + lrow;
        if (row < p.M && col < p.N) {
          if constexpr (EPI == EPI_I32) {
            static_cast<int32_t*>(p.c)[(int64_t)row * p.ldc + col] = acc[i][j][r];
          } else {
            // reference order: (float(acc) * act_scale) * w_scale, added to the side path
            float v = mul_rn(mul_rn(static_cast<float>(acc[i][j][r]), asl[lrow]), bsc);
            if (nsc || tside) v = add_rn(side[r], v);
            if constexpr (EPI == EPI_F32)
              static_cast<float*>(p.c)[(int64_t)row * p.ldc + col] = v;
            else
              static_cast<uint16_t*>(p.c)[(int64_t)row * p.ldc + col] = f32_to_bf16_bits(v);
          }
        }
      }
    }
}

// Epilogue of the DMA GEMM, whose MFMAs take the weight fragment as A and the activation
// fragment as B: accumulator register r of lane l then holds
// C[row (l & 31)][col 8 * (r / 4) + 4 * (l >> 5) + (r % 4)] of the 32 x 32 tile, i.e. four
// consecutive columns of one row per register group, stored with one 16-byte (int32 /
// fp32) or 8-byte (bf16) instruction instead of four scalar ones.  The side path's
// MFMAs swap their operands the same way and keep their order, so every value equals the
// one gemm_epilogue computes.  PRE as in gemm_epilogue.
//
// LDSB is the size of the tile LDS at ws0.  When it also holds a 32 x WN block per wave
// beyond the side-path staging, each wave passes its block of row tile i through that
// wave-private area (16-byte chunks XOR-swizzled by block row) and stores it with 16
// bytes per lane, 8 (bf16) or 16 (fp32 / int32) lanes per block row: every store
// instruction then writes whole 128-byte lines instead of 16- or 32-byte pieces of 32
// rows.  A wave whose block is ragged or whose rows are not 16-byte aligned stores from
// registers.
template <int BM, int BN, int WM, int WN, int EPI, int NT, int PRE, int LDSB = 0>
__device__ __forceinline__ void gemm_epilogue_t(const GemmParams& p, i32x16 (&acc)[WM / 32][WN / 32], float* ws0,
                                                int bm, int bn, int wm, int wn, int tid, int lane,
                                                const float* tail) {
  constexpr int FM = WM / 32, FN = WN / 32;
  static_assert(!PRE || (EPI != EPI_I32 && BM <= 256 && BN <= 256), "tail layout");
  constexpr int ES = EPI == EPI_BF16 ? 2 : 4;                // output bytes per element
  constexpr int RB = WN * ES, NCH = RB / 16;                 // block row bytes, 16-byte chunks
  constexpr int SIDE_B = (BM + BN) * (kSideLds + 1) * 4;     // side-path staging at ws0
  constexpr bool kRowStore = WN == 64 && LDSB >= SIDE_B + (NT / 64) * 32 * RB;
  const int h = lane >> 5, l32 = lane & 31;
  const bool tside = PRE && p.P > 0 && p.P <= kTailSide;
  const int nsc = (EPI != EPI_I32 && p.P > 0 && !tside) ? (p.P + kSideLds - 1) / kSideLds : 0;
  float* xs = ws0;                 // [BM][kSideLds]
  float* ws = xs + BM * kSideLds;  // [kSideLds][BN]
  auto stage_side = [&](int q0) {
    for (int t = tid; t < BM * kSideLds; t += NT) {
      const int r = t / kSideLds, q = q0 + (t - (t / kSideLds) * kSideLds);
      xs[t] = (bm + r < p.M && q < p.P) ? p.xp[(int64_t)(bm + r) * p.P + q] : 0.f;
    }
    for (int t = tid; t < BN * kSideLds; t += NT) {
      const int c = t / kSideLds, qq = t - (t / kSideLds) * kSideLds, q = q0 + qq;
      ws[qq * BN + c] = (bn + c < p.N && q < p.P) ? p.wp[(int64_t)(bn + c) * p.P + q] : 0.f;
    }
  };
  const float* asl = PRE ? tail + kTailAs : ws + kSideLds * BN;       // [BM]
  const float* bsl = PRE ? tail + kTailBs : ws + kSideLds * BN + BM;  // [BN]
  if constexpr (EPI != EPI_I32 && !PRE) {
    float* as_st = ws + kSideLds * BN;
    for (int t = tid; t < BM; t += NT) as_st[t] = bm + t < p.M ? p.as[bm + t] : 0.f;
    for (int t = tid; t < BN; t += NT) as_st[BM + t] = bn + t < p.N ? p.bs[bn + t] : 0.f;
  }
  if (nsc == 1) stage_side(0);
  if ((EPI != EPI_I32 && !PRE) || nsc == 1) __syncthreads();
  // 4-wide stores need 16-byte aligned rows (ldc % 4 == 0, y 16-byte aligned)
  const bool vec = p.ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(p.c) & 15) == 0;
  const bool rowst = kRowStore && ((int64_t)p.ldc * ES) % 16 == 0 && (reinterpret_cast<uintptr_t>(p.c) & 15) == 0 &&
                     bn + wn * WN + WN <= p.N;
  int8_t* const tb = reinterpret_cast<int8_t*>(ws0) + SIDE_B + __builtin_amdgcn_readfirstlane(tid >> 6) * 32 * RB;
  typedef float f32x16 __attribute__((ext_vector_type(16)));
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int lrow = wm * WM + 32 * i + l32;
    const int row = bm + lrow;
    const bool tr = rowst && bm + wm * WM + 32 * i + 32 <= p.M;  // wave-uniform
    // the side operands of this lane's row (P == 8 tail: two 16-byte LDS reads)
    float xr[kTailSide];
    if (tside) {
      const float* txp = tail + kTailXp;
      if (p.P == kTailSide) {
        const f32x4 a0 = *reinterpret_cast<const f32x4*>(txp + lrow * kTailSide);
        const f32x4 a1 = *reinterpret_cast<const f32x4*>(txp + lrow * kTailSide + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) xr[e] = a0[e], xr[4 + e] = a1[e];
      } else {
#pragma unroll
        for (int e = 0; e < kTailSide; ++e) xr[e] = e < p.P ? txp[lrow * p.P + e] : 0.f;
      }
    }
    float asc = 0.f;
    if constexpr (EPI != EPI_I32) asc = asl[lrow];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int lc = wn * WN + 32 * j;
      f32x16 side = {};
      if (tside) {
        const float* twp = tail + kTailXp + BM * kTailSide;  // [BN][P]
        const int lcol = lc + l32;
        float wr[kTailSide];
        if (p.P == kTailSide) {
          const f32x4 b0 = *reinterpret_cast<const f32x4*>(twp + lcol * kTailSide);
          const f32x4 b1 = *reinterpret_cast<const f32x4*>(twp + lcol * kTailSide + 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) wr[e] = b0[e], wr[4 + e] = b1[e];
        } else {
#pragma unroll
          for (int e = 0; e < kTailSide; ++e) wr[e] = e < p.P ? twp[lcol * p.P + e] : 0.f;
        }
        // steps of two columns (2s, 2s + 1), half h of the wave supplying column 2s + h
#pragma unroll
        for (int s2 = 0; s2 < kTailSide; s2 += 2) {
          if (s2 < p.P) {
            const float xa = h ? xr[s2 + 1] : xr[s2];
            const float wb = h ? wr[s2 + 1] : wr[s2];
            side = __builtin_amdgcn_mfma_f32_32x32x2f32(wb, xa, side, 0, 0, 0);
          }
        }
      }
      for (int c = 0; c < nsc; ++c) {
        if (nsc > 1) {
          __syncthreads();
          stage_side(c * kSideLds);
          __syncthreads();
        }
        const int qn = min(kSideLds, p.P - c * kSideLds);
        for (int s2 = 0; s2 < qn; s2 += 2) {
          const float xa = xs[lrow * kSideLds + s2 + h];
          const float wb = ws[(s2 + h) * BN + lc + l32];
          side = __builtin_amdgcn_mfma_f32_32x32x2f32(wb, xa, side, 0, 0, 0);
        }
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int lcol0 = lc + 8 * g + 4 * h;
        const int col0 = bn + lcol0;
        if (row >= p.M || col0 >= p.N) continue;
        const int64_t o = (int64_t)row * p.ldc + col0;
        const bool full = vec && col0 + 3 < p.N;
        // this lane's four values in the wave's block: row l32, 16-byte chunk q (bf16: its
        // half h), at the chunk's swizzled place
        const int q = ES == 2 ? 4 * j + g : 8 * j + 2 * g + h;
        int8_t* const tw = tb + l32 * RB + 16 * (q ^ (l32 & (NCH - 1))) + (ES == 2 ? 8 * h : 0);
        if constexpr (EPI == EPI_I32) {
          const i32x4 v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
          if (tr) {
            *reinterpret_cast<i32x4*>(tw) = v;
          } else if (full) {
            *reinterpret_cast<i32x4*>(static_cast<int32_t*>(p.c) + o) = v;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (col0 + e < p.N) static_cast<int32_t*>(p.c)[o + e] = v[e];
          }
        } else {
          const f32x4 bsc = *reinterpret_cast<const f32x4*>(bsl + lcol0);
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            // reference order: (float(acc) * act_scale) * w_scale, added to the side path
            v[e] = mul_rn(mul_rn(static_cast<float>(acc[i][j][4 * g + e]), asc), bsc[e]);
            if (nsc || tside) v[e] = add_rn(side[4 * g + e], v[e]);
          }
          if constexpr (EPI == EPI_F32) {
            if (tr) {
              *reinterpret_cast<f32x4*>(tw) = f32x4{v[0], v[1], v[2], v[3]};
            } else if (full) {
              *reinterpret_cast<f32x4*>(static_cast<float*>(p.c) + o) = f32x4{v[0], v[1], v[2], v[3]};
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (col0 + e < p.N) static_cast<float*>(p.c)[o + e] = v[e];
            }
          } else {
            uint16_t b[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) b[e] = f32_to_bf16_bits(v[e]);
            const uint2 pk = make_uint2(b[0] | (uint32_t)b[1] << 16, b[2] | (uint32_t)b[3] << 16);
            if (tr) {
              *reinterpret_cast<uint2*>(tw) = pk;
            } else if (full) {
              *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.c) + o) = pk;
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (col0 + e < p.N) static_cast<uint16_t*>(p.c)[o + e] = b[e];
            }
          }
        }
      }
    }
    if (tr) {
      // the block's rows, 16 bytes per lane: lane l reads chunk l % NCH of block row
      // RPI s + l / NCH (its swizzled place) and stores it where the row lies in C
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's block writes landed
      constexpr int RPI = 64 / NCH;
      const int c = lane & (NCH - 1);
      char* const cb = static_cast<char*>(p.c) +
                       ((int64_t)(bm + wm * WM + 32 * i) * p.ldc + bn + wn * WN) * ES + 16 * c;
#pragma unroll
      for (int s = 0; s < 32 / RPI; ++s) {
        const int r = RPI * s + lane / NCH;
        const i32x4 v = *reinterpret_cast<const i32x4*>(tb + r * RB + 16 * (c ^ (r & (NCH - 1))));
        *reinterpret_cast<i32x4*>(cb + (int64_t)r * p.ldc * ES) = v;
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, int EPI, int BK = kBK>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void k_gemm_i8(GemmParams p) {
  constexpr int WAVES_M = BM / WM, WAVES_N = BN / WN;
  constexpr int NT = WAVES_M * WAVES_N * 64;
  constexpr int FM = WM / 32, FN = WN / 32;
  constexpr int LROW = BK + 16;                            // padded LDS row
  constexpr int RC = BK / 16;                              // 16-byte chunks per tile row
  constexpr int A_CH = BM * RC / NT, B_CH = BN * RC / NT;  // 16-byte chunks per thread
  static_assert(A_CH >= 1 && B_CH >= 1 && BM * RC % NT == 0 && BN * RC % NT == 0,
                "tile too small for the thread count");
  static_assert(2 * (BM + BN) * LROW >= (BM + BN) * (kSideLds + 1) * 4, "epilogue staging needs the tile LDS");
  __shared__ __attribute__((aligned(16))) int8_t lds[2][(BM + BN) * LROW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;

  // XCD-aware tile order: consecutive workgroup ids are dealt round-robin to the 8 XCDs,
  // so regroup them such that the workgroups of one XCD walk consecutive M tiles of the
  // same N tile (its B tile is then served from that XCD's L2).
  const int tiles_m = (p.M + BM - 1) / BM;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int G = tiles_m * tiles_n;
  const int bid = blockIdx.x;
  int lid = bid;
  if ((G & 7) == 0) lid = (bid & 7) * (G >> 3) + (bid >> 3);
  const int tm = lid % tiles_m, tn = lid / tiles_m;
  const int bm = tm * BM, bn = tn * BN;

  // global -> register staging
  const int8_t* ga[A_CH];
  const int8_t* gb[B_CH];
  int la[A_CH], lb[B_CH];
#pragma unroll
  for (int i = 0; i < A_CH; ++i) {
    const int c = tid + i * NT;
    const int r = c / RC, col = (c % RC) * 16;
    const int gr = bm + r < p.M ? bm + r : p.M - 1;
    ga[i] = p.a + (int64_t)gr * p.lda + col;
    la[i] = r * LROW + col;
  }
#pragma unroll
  for (int i = 0; i < B_CH; ++i) {
    const int c = tid + i * NT;
    const int r = c / RC, col = (c % RC) * 16;
    const int gr = bn + r < p.N ? bn + r : p.N - 1;
    gb[i] = p.b + (int64_t)gr * p.ldb + col;
    lb[i] = (BM + r) * LROW + col;
  }
  i32x4 ra[A_CH], rb[B_CH];
  auto gload = [&](int kt) {
    const int64_t ko = (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < A_CH; ++i) ra[i] = *reinterpret_cast<const i32x4*>(ga[i] + ko);
#pragma unroll
    for (int i = 0; i < B_CH; ++i) rb[i] = *reinterpret_cast<const i32x4*>(gb[i] + ko);
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) *reinterpret_cast<i32x4*>(&lds[buf][la[i]]) = ra[i];
#pragma unroll
    for (int i = 0; i < B_CH; ++i) *reinterpret_cast<i32x4*>(&lds[buf][lb[i]]) = rb[i];
  };

  i32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  const int KT = p.K / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  const int arow = wm * WM + (lane & 31);
  const int brow = BM + wn * WN + (lane & 31);
  const int kh = 16 * (lane >> 5);
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      i32x4 fa[FM], fb[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        fa[i] = *reinterpret_cast<const i32x4*>(&lds[buf][(arow + 32 * i) * LROW + 32 * ks + kh]);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        fb[j] = *reinterpret_cast<const i32x4*>(&lds[buf][(brow + 32 * j) * LROW + 32 * ks + kh]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) lstore(buf ^ 1);
    __syncthreads();
  }

  gemm_epilogue<BM, BN, WM, WN, EPI, NT>(p, acc, reinterpret_cast<float*>(&lds[0][0]), bm, bn, wm, wn, tid, lane);
}

// LDS row swizzle of the DMA-fed tiles: 16-byte chunk c of tile row r sits in slot
// c ^ dma_swz(r).  gfx950 serves a ds_read_b128 in four passes of 16 lanes over 64 banks
// (16 groups of 16 bytes); measured with SQ_LDS_BANK_CONFLICT, the passes are lanes
// {0-3, 12-15, 20-23, 24-27}, {4-7, 8-11, 16-19, 28-31} and the same sets + 32, not 16
// consecutive lanes.  A fragment read puts row r = lane & 31 (one chunk index per half
// wave) in bank group 4 (r & 3) + slot, so the four rows of a pass that share r & 3 need
// distinct slots: their r >> 2 are {0, 3, 5, 6} or {1, 2, 4, 7}, and (r >> 2) & 3 is a
// bijection on each set.
__device__ __forceinline__ int dma_swz(int r) { return (r >> 2) & 3; }

// One wave's 1 KiB global -> LDS copy: lane l's 16 bytes at buffer offset voff + soff land
// at dst + 16 l.  Kept out of the kernel template: in template-dependent code the host
// compilation pass drops the kernel's launch stub over this builtin.
__device__ __forceinline__ void lds_copy16(__amdgpu_buffer_rsrc_t r, int8_t* dst, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, soff, 0, 0);
}

// int8 GEMM with LDS fed by DMA: BM x BN blocks of 8 waves (256 x 256 with 128 x 64 per
// wave for large products, 256 x 128 with 64 x 64 otherwise -- 14% faster than 128 x 128
// at M=512), 64-byte K steps, a ring of four LDS stages.  Tile kt + 3 is
// requested (buffer_load ... lds: global memory straight into LDS, 1 KiB per wave
// instruction) while tile kt is multiplied, so loads have three steps to land and
// neither staging registers nor ds_write instructions sit in the loop.  A DMA instruction
// writes its 64 lanes' 16 bytes contiguously, so a wave instruction fills 16 tile rows
// and the lane -> global chunk map carries the row swizzle.  One barrier per step: each
// wave waits for its own copies of tile kt (vmcnt), then the barrier makes every wave's
// copies visible and retires the stage read in step kt - 1, which the next copy reuses.
// Needs K % 64 == 0, 16-byte aligned rows and 256 * ld < 2^31.
template <int BM, int BN, int WM, int WN, int EPI, int PRE = 0>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void k_gemm_i8_dma(GemmParams p) {
  constexpr int BK = 64, S = 4;
  constexpr int WAVES_M = BM / WM, NW = WAVES_M * (BN / WN), NT = NW * 64;
  constexpr int FM = WM / 32, FN = WN / 32;
  constexpr int TILE_A = BM * BK, TILE_B = BN * BK;  // bytes per operand per stage
  constexpr int STAGE = TILE_A + TILE_B;
  constexpr int JA = BM / 16 / NW, JB = BN / 16 / NW;  // 1 KiB copies per wave per stage
  static_assert(JA >= 1 && JB >= 1 && JA * 16 * NW == BM && JB * 16 * NW == BN, "whole copies per wave");
  static_assert(S * STAGE >= (BM + BN) * (kSideLds + 1) * 4, "epilogue staging needs the tile LDS");
  constexpr int TAIL = PRE ? 4 * tail_floats<BM, BN>() : 0;  // bytes
  __shared__ __attribute__((aligned(1024))) int8_t lds[S * STAGE + TAIL];
  int8_t* const tail = lds + S * STAGE;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int tiles_m = (p.M + BM - 1) / BM;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int G = tiles_m * tiles_n;
  const int bid = blockIdx.x;
  int lid = bid;
  if ((G & 7) == 0) lid = (bid & 7) * (G >> 3) + (bid >> 3);
  const int tm = lid % tiles_m, tn = lid / tiles_m;
  const int bm = tm * BM, bn = tn * BN;

  const int64_t arem = (int64_t)(p.M - bm) * p.lda, brem = (int64_t)(p.N - bn) * p.ldb;
  const int alim = (int)(arem < INT_MAX ? arem : INT_MAX), blim = (int)(brem < INT_MAX ? brem : INT_MAX);
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t*>(p.a + (int64_t)bm * p.lda), (short)0, alim, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t*>(p.b + (int64_t)bn * p.ldb), (short)0, blim, 0x00020000);
  // DMA roles: copy j of this wave covers tile rows 16 * (J * wave + j) + 0..15 of its
  // operand; lane l lands in row + (l >> 2), slot l & 3, and fetches chunk slot ^ swizzle.
  int aoff[JA], boff[JB];
#pragma unroll
  for (int j = 0; j < JA; ++j) {
    const int r = 16 * (JA * wave + j) + (lane >> 2);
    aoff[j] = r * (int)p.lda + 16 * ((lane & 3) ^ dma_swz(r));
  }
#pragma unroll
  for (int j = 0; j < JB; ++j) {
    const int r = 16 * (JB * wave + j) + (lane >> 2);
    boff[j] = r * (int)p.ldb + 16 * ((lane & 3) ^ dma_swz(r));
  }
  const int KT = p.K / BK;
  // PRE: the copy slots of step KT, which loads nothing otherwise, fetch the epilogue's
  // operands into the tail instead -- act / weight scales (1 KiB each) and, for
  // P <= kTailSide, the side operands' row slices (BM * P and BN * P floats, 1 KiB per
  // copy, zero past M / N).  Every wave still issues JA + JB copies per step, so the wait
  // counts hold; the step is waited for only by the loop's final vmcnt(0), and the copies
  // land while the last steps multiply.
  auto tail_copies = [&](int8_t* st) {
    const int tp = p.P > 0 && p.P <= kTailSide ? p.P : 0;
    const int ncx = (BM * tp + 255) / 256, ncw = (BN * tp + 255) / 256;
    auto rs = [](const float* base, int64_t n) {  // n floats readable from base
      return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0,
                                               (int)(4 * n < INT_MAX ? 4 * n : INT_MAX), 0x00020000);
    };
    static_assert(2 + (BM + BN) * kTailSide / 256 <= (JA + JB) * NW, "tail copies fit the step's slots");
#pragma unroll
    for (int j = 0; j < JA + JB; ++j) {
      const int c = j * NW + wave;  // wave-uniform
      if (c == 0)
        lds_copy16(rs(p.as + bm, p.M - bm), tail + 4 * kTailAs, 16 * lane, 0);
      else if (c == 1)
        lds_copy16(rs(p.bs + bn, p.N - bn), tail + 4 * kTailBs, 16 * lane, 0);
      else if (c < 2 + ncx)
        lds_copy16(rs(p.xp + (int64_t)bm * tp, (int64_t)(p.M - bm) * tp), tail + 4 * kTailXp + 1024 * (c - 2),
                   16 * lane + 1024 * (c - 2), 0);
      else if (c < 2 + ncx + ncw)
        lds_copy16(rs(p.wp + (int64_t)bn * tp, (int64_t)(p.N - bn) * tp),
                   tail + 4 * (kTailXp + BM * kTailSide) + 1024 * (c - 2 - ncx), 16 * lane + 1024 * (c - 2 - ncx), 0);
      else
        lds_copy16(rsa, st + 1024 * c, alim, 0);  // nothing to fetch: out of range, no access
    }
  };
  // rows past M / N read as zero; steps past K load out of the buffer's range (zero, no
  // memory access) into a stage that is not read again
  // chk: this step's copies may be step KT's (false in the main loop, so that its body
  // stays one straight block)
  auto dma = [&](int kt, bool chk) {
    const bool live = kt < KT;
    const int ko = live ? kt * BK : 0;
    int8_t* st = lds + (kt & (S - 1)) * STAGE;
    if constexpr (PRE) {
      if (chk && kt == KT) {
        tail_copies(st);
        return;
      }
    }
#pragma unroll
    for (int j = 0; j < JA; ++j) lds_copy16(rsa, st + 1024 * (JA * wave + j), live ? aoff[j] : alim, ko);
#pragma unroll
    for (int j = 0; j < JB; ++j) lds_copy16(rsb, st + TILE_A + 1024 * (JB * wave + j), live ? boff[j] : blim, ko);
  };

  i32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
  // fragment rows are 32-aligned bases + (lane & 31), so one swizzle serves them all
  const int sl = dma_swz(lane & 31);
  const int arow = (wm * WM + (lane & 31)) * BK, brow = TILE_A + (wn * WN + (lane & 31)) * BK;

  static_assert(BK == 64, "the loop below takes two 32-byte slices per step");
  auto frag = [&](i32x4 (&f)[FM + FN], int kt, int ks) {
    const int8_t* st = lds + (kt & (S - 1)) * STAGE;
    const int co = 16 * ((2 * ks + (lane >> 5)) ^ sl);
#pragma unroll
    for (int i = 0; i < FM; ++i) f[i] = *reinterpret_cast<const i32x4*>(st + arow + 32 * BK * i + co);
#pragma unroll
    for (int j = 0; j < FN; ++j) f[FM + j] = *reinterpret_cast<const i32x4*>(st + brow + 32 * BK * j + co);
  };
  auto mma = [&](const i32x4 (&f)[FM + FN]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f[FM + j], f[i], acc[i][j], 0, 0, 0);  // C^T tile
  };
  // Step kt: read slice 1 of tile kt, multiply slice 0 (read one step earlier), then the
  // barrier for tile kt + 1 -- this wave's copies of kt + 1 done (vmcnt) and its reads of
  // tile kt done (lgkmcnt), so the stage may be refilled -- the copy of tile kt + 4, the
  // reads of slice 0 of tile kt + 1, and the MFMAs of slice 1 of tile kt, which cover the
  // barrier and those reads.
  i32x4 fa[FM + FN], fb[FM + FN];
  dma(0, true);
  dma(1, true);
  dma(2, true);
  constexpr int NEWER = 2 * (JA + JB);  // this wave's copies of the two newer stages
  static_assert(NEWER == 8 || NEWER == 6 || NEWER == 4, "wait counts below");
  if constexpr (NEWER == 8)
    asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
  else if constexpr (NEWER == 6)
    asm volatile("s_waitcnt vmcnt(6)\n\ts_barrier" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(4)\n\ts_barrier" ::: "memory");
  dma(3, true);
  // The prologue's copies may take the tail path (K <= 3 * BK), whose kernel-argument
  // loads count in lgkmcnt; settle them here, visibly to the compiler, so that the loop
  // keeps its partial LDS waits.
  if constexpr (PRE) __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt / expcnt unconstrained
  frag(fa, 0, 0);
  // last: kt may be the final step (no next tile).  The main loop's steps never are, so
  // their body has no branch: the compiler cannot see the LDS wait inside the barrier
  // asm, and at a join with a path that skips it, it would wait for the next tile's
  // fragment reads before the MFMAs of slice 1 instead of letting them overlap.
  // sched_barrier keeps the phases in this order (reads ahead of the MFMAs that hide them)
  auto step = [&](int kt, bool chk, bool last) {
    frag(fb, kt, 1);
    __builtin_amdgcn_sched_barrier(0);
    mma(fa);
    __builtin_amdgcn_sched_barrier(0);
    if (!last || kt + 1 < KT) {
      if constexpr (NEWER == 8)
        asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      else if constexpr (NEWER == 6)
        asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      dma(kt + 4, chk);
      frag(fa, kt + 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    mma(fb);
    __builtin_amdgcn_sched_barrier(0);
  };
  // PRE: the last four steps, whose copies may be step KT's, run in a loop of their own;
  // otherwise the last step alone
  const int kmain = !PRE ? KT - 1 : (KT > 4 ? KT - 4 : 0);
  int kt = 0;
  for (; kt < kmain; ++kt) step(kt, false, false);
  for (; kt < KT; ++kt) step(kt, true, true);
  // every copy (including the ones past K) has landed before the epilogue reuses LDS
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  gemm_epilogue_t<BM, BN, WM, WN, EPI, NT, PRE, S * STAGE>(p, acc, reinterpret_cast<float*>(lds), bm, bn, wm, wn,
                                                           tid, lane, reinterpret_cast<const float*>(tail));
}

// s_waitcnt vmcnt(N) (lgkmcnt(0) too with LGK), then s_barrier; N is a compile-time count
// of this wave's newer copies that may stay in flight.
template <int N, bool LGK>
__device__ __forceinline__ void vm_wait_barrier() {
  static_assert(N == 0 || N == 4 || N == 6 || N == 8 || N == 12 || N == 18, "wait counts");
  if constexpr (LGK) {
    if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else if constexpr (N == 4) asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else if constexpr (N == 6) asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else if constexpr (N == 8) asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else if constexpr (N == 12) asm volatile("s_waitcnt vmcnt(12) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(18) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  } else {
    if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    else if constexpr (N == 4) asm volatile("s_waitcnt vmcnt(4)\n\ts_barrier" ::: "memory");
    else if constexpr (N == 6) asm volatile("s_waitcnt vmcnt(6)\n\ts_barrier" ::: "memory");
    else if constexpr (N == 8) asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
    else if constexpr (N == 12) asm volatile("s_waitcnt vmcnt(12)\n\ts_barrier" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(18)\n\ts_barrier" ::: "memory");
  }
}

// k_gemm_i8_dma with 128-byte K steps in S LDS stages (k_gemm_i8_p2; S = 2 for the large
// tiles, 4 for the small ones).  A copy instruction then takes whole 128-byte lines (8 rows
// x 128 bytes) instead of half lines (16 rows x 64 bytes): a probe of this copy ring on 448
// workgroups measured 69.8 GB/s of LDS fill per CU with 64 KB in flight, against 42-43 GB/s
// for the half-line copies with 64 or 96 KB in flight.  Stage p & (S - 1) holds the pair
// of 64-k steps p; the copies of pair p + S go out after the barrier that ends pair p, so
// S - 1 pairs are in flight while one is multiplied.  One barrier per 128 k.  Rows are 128
// bytes; 16-byte chunk c of row r sits at slot c ^ dma_swz8(r), which puts the 16 rows of
// each ds_read_b128 pass (see dma_swz) in 16 distinct bank groups: a pass reads rows of
// both parities, and within a parity its 8 rows have distinct (r >> 1) & 7.  Needs
// K % 128 == 0, 16-byte aligned rows and 256 * ld < 2^31.
__device__ __forceinline__ int dma_swz8(int r) { return (r >> 1) & 7; }

template <int BM, int BN, int WM, int WN, int EPI, int PRE = 0>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void k_gemm_i8_p2(GemmParams p) {
  constexpr int BK = 128;
  // stages: two for the large tiles (a third measured no faster on 256 x 128); the small
  // tiles of few-row products, a weight stream, keep three stages of copies in flight
  // (14336 x 4096, one box: M = 64 on 64 x 64 tiles 19.2 -> 13.1 us, M = 256 on 128 x 128
  // tiles 25.4 -> 24.3 us)
  constexpr int S = BM + BN <= 256 ? 4 : 2;
  static_assert((S & (S - 1)) == 0, "stage index by mask");
  constexpr int WAVES_M = BM / WM, NW = WAVES_M * (BN / WN), NT = NW * 64;
  constexpr int FM = WM / 32, FN = WN / 32;
  constexpr int TILE_A = BM * BK, TILE_B = BN * BK;  // bytes per operand per stage
  constexpr int STAGE = TILE_A + TILE_B;
  constexpr int JA = BM / 8 / NW, JB = BN / 8 / NW;  // 1 KiB copies per wave per stage
  static_assert(JA >= 1 && JB >= 1 && JA * 8 * NW == BM && JB * 8 * NW == BN, "whole copies per wave");
  static_assert(S * STAGE >= (BM + BN) * (kSideLds + 1) * 4, "epilogue staging needs the tile LDS");
  constexpr int TAIL = PRE ? 4 * tail_floats<BM, BN>() : 0;  // bytes
  __shared__ __attribute__((aligned(1024))) int8_t lds[S * STAGE + TAIL];
  int8_t* const tail = lds + S * STAGE;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int tiles_m = (p.M + BM - 1) / BM;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int G = tiles_m * tiles_n;
  const int bid = blockIdx.x;
  int lid = bid;
  if ((G & 7) == 0) lid = (bid & 7) * (G >> 3) + (bid >> 3);
  const int tm = lid % tiles_m, tn = lid / tiles_m;
  const int bm = tm * BM, bn = tn * BN;

  const int64_t arem = (int64_t)(p.M - bm) * p.lda, brem = (int64_t)(p.N - bn) * p.ldb;
  const int alim = (int)(arem < INT_MAX ? arem : INT_MAX), blim = (int)(brem < INT_MAX ? brem : INT_MAX);
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t*>(p.a + (int64_t)bm * p.lda), (short)0, alim, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t*>(p.b + (int64_t)bn * p.ldb), (short)0, blim, 0x00020000);
  // copy j of this wave covers tile rows 8 * (J * wave + j) + 0..7 of its operand; lane l
  // lands in row + (l >> 3), slot l & 7, and fetches chunk slot ^ swizzle
  int aoff[JA], boff[JB];
#pragma unroll
  for (int j = 0; j < JA; ++j) {
    const int r = 8 * (JA * wave + j) + (lane >> 3);
    aoff[j] = r * (int)p.lda + 16 * ((lane & 7) ^ dma_swz8(r));
  }
#pragma unroll
  for (int j = 0; j < JB; ++j) {
    const int r = 8 * (JB * wave + j) + (lane >> 3);
    boff[j] = r * (int)p.ldb + 16 * ((lane & 7) ^ dma_swz8(r));
  }
  const int KP = p.K / BK;  // pairs of 64-k steps
  // PRE: the copy slots of pair KP, which loads nothing otherwise, fetch the epilogue's
  // operands into the tail (as in k_gemm_i8_dma)
  auto tail_copies = [&](int8_t* st) {
    const int tp = p.P > 0 && p.P <= kTailSide ? p.P : 0;
    const int ncx = (BM * tp + 255) / 256, ncw = (BN * tp + 255) / 256;
    auto rs = [](const float* base, int64_t n) {  // n floats readable from base
      return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0,
                                               (int)(4 * n < INT_MAX ? 4 * n : INT_MAX), 0x00020000);
    };
    static_assert(2 + (BM + BN) * kTailSide / 256 <= (JA + JB) * NW, "tail copies fit the pair's slots");
#pragma unroll
    for (int j = 0; j < JA + JB; ++j) {
      const int c = j * NW + wave;  // wave-uniform
      if (c == 0)
        lds_copy16(rs(p.as + bm, p.M - bm), tail + 4 * kTailAs, 16 * lane, 0);
      else if (c == 1)
        lds_copy16(rs(p.bs + bn, p.N - bn), tail + 4 * kTailBs, 16 * lane, 0);
      else if (c < 2 + ncx)
        lds_copy16(rs(p.xp + (int64_t)bm * tp, (int64_t)(p.M - bm) * tp), tail + 4 * kTailXp + 1024 * (c - 2),
                   16 * lane + 1024 * (c - 2), 0);
      else if (c < 2 + ncx + ncw)
        lds_copy16(rs(p.wp + (int64_t)bn * tp, (int64_t)(p.N - bn) * tp),
                   tail + 4 * (kTailXp + BM * kTailSide) + 1024 * (c - 2 - ncx), 16 * lane + 1024 * (c - 2 - ncx), 0);
      else
        lds_copy16(rsa, st + 1024 * c, alim, 0);  // nothing to fetch: out of range, no access
    }
  };
  // pair kp -> stage kp & (S - 1); pairs past K load out of the buffer's range (zero, no
  // memory access) into a stage that is not read again
  auto dma = [&](int kp) {
    const bool live = kp < KP;
    const int ko = live ? kp * BK : 0;
    int8_t* st = lds + (kp & (S - 1)) * STAGE;
    if constexpr (PRE) {
      if (kp == KP) {
        tail_copies(st);
        return;
      }
    }
#pragma unroll
    for (int j = 0; j < JA; ++j) lds_copy16(rsa, st + 1024 * (JA * wave + j), live ? aoff[j] : alim, ko);
#pragma unroll
    for (int j = 0; j < JB; ++j) lds_copy16(rsb, st + TILE_A + 1024 * (JB * wave + j), live ? boff[j] : blim, ko);
  };

  i32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
  const int sl = dma_swz8(lane & 31);  // fragment rows are 32-aligned bases + (lane & 31)
  const int arow = (wm * WM + (lane & 31)) * BK, brow = TILE_A + (wn * WN + (lane & 31)) * BK;
  // slice ks (0..3) of pair kp: 32 k; lanes 0-31 take chunk 2 ks, lanes 32-63 chunk 2 ks + 1
  auto frag = [&](i32x4 (&f)[FM + FN], int kp, int ks) {
    const int8_t* st = lds + (kp & (S - 1)) * STAGE;
    const int co = 16 * ((2 * ks + (lane >> 5)) ^ sl);
#pragma unroll
    for (int i = 0; i < FM; ++i) f[i] = *reinterpret_cast<const i32x4*>(st + arow + 32 * BK * i + co);
#pragma unroll
    for (int j = 0; j < FN; ++j) f[FM + j] = *reinterpret_cast<const i32x4*>(st + brow + 32 * BK * j + co);
  };
  auto mma = [&](const i32x4 (&f)[FM + FN]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f[FM + j], f[i], acc[i][j], 0, 0, 0);  // C^T tile
  };
  i32x4 fa[FM + FN], fb[FM + FN];
#pragma unroll
  for (int i = 0; i < S; ++i) dma(i);
  constexpr int NEWER = JA + JB;  // this wave's copies of one stage
  vm_wait_barrier<(S - 1) * NEWER, false>();  // stage 0 landed
  // a prologue copy that took the tail path issued argument loads (lgkmcnt); settle them
  // here, visibly to the compiler, so that the loop keeps its partial LDS waits
  if constexpr (PRE) __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt / expcnt unconstrained
  frag(fa, 0, 0);
  // Pair kp: slices 0..3, each read one slice ahead of its MFMAs; after the last slice's
  // reads, this wave's copies of pair kp + 1 have landed (only the S - 2 newer stages'
  // copies may still be out) and its reads of stage kp & (S - 1) are done (lgkmcnt(0)), so
  // after the barrier the stage takes the copies of pair kp + S while slice 3 is multiplied.
  // With S > 2 every pair issues its copies, past K too (out of range), so that the wait
  // counts stay exact.
  auto pair = [&](int kp) {
    frag(fb, kp, 1);
    __builtin_amdgcn_sched_barrier(0);
    mma(fa);
    __builtin_amdgcn_sched_barrier(0);
    frag(fa, kp, 2);
    __builtin_amdgcn_sched_barrier(0);
    mma(fb);
    __builtin_amdgcn_sched_barrier(0);
    frag(fb, kp, 3);
    __builtin_amdgcn_sched_barrier(0);
    mma(fa);
    __builtin_amdgcn_sched_barrier(0);
    if (kp + 1 < KP) {
      vm_wait_barrier<(S - 2) * NEWER, true>();
      if constexpr (S == 2) {
        if (kp + 2 <= KP) dma(kp + 2);
      } else {
        dma(kp + S);
      }
      frag(fa, kp + 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    mma(fb);
    __builtin_amdgcn_sched_barrier(0);
  };
  for (int kp = 0; kp < KP; ++kp) pair(kp);
  // every copy (including the ones past K) has landed before the epilogue reuses LDS
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  gemm_epilogue_t<BM, BN, WM, WN, EPI, NT, PRE, S * STAGE>(p, acc, reinterpret_cast<float*>(lds), bm, bn, wm, wn,
                                                           tid, lane, reinterpret_cast<const float*>(tail));
}

// Any shape: one thread per output, exact int32 accumulation.
__global__ __launch_bounds__(256) void k_gemm_i8_generic(GemmParams p, int epi) {
  const int64_t i = blockIdx.x * 256ll + threadIdx.x;
  if (i >= (int64_t)p.M * p.N) return;
  const int row = (int)(i / p.N), col = (int)(i % p.N);
  const int8_t* a = p.a + (int64_t)row * p.lda;
  const int8_t* b = p.b + (int64_t)col * p.ldb;
  int acc = 0;
  for (int k = 0; k < p.K; ++k) acc += (int)a[k] * (int)b[k];
  if (epi == EPI_I32) {
    static_cast<int32_t*>(p.c)[(int64_t)row * p.ldc + col] = acc;
    return;
  }
  float v = mul_rn(mul_rn(static_cast<float>(acc), p.as[row]), p.bs[col]);
  if (p.P > 0) {
    float side = 0.f;
    for (int q = 0; q < p.P; ++q) side = fmaf(p.xp[(int64_t)row * p.P + q], p.wp[(int64_t)col * p.P + q], side);
    v = add_rn(side, v);
  }
  if (epi == EPI_F32)
    static_cast<float*>(p.c)[(int64_t)row * p.ldc + col] = v;
  else
    static_cast<uint16_t*>(p.c)[(int64_t)row * p.ldc + col] = f32_to_bf16_bits(v);
}

namespace {

// Tile shapes (measured on MI355X, 14336 x 4096 weights): 256 x 256 blocks of 8 waves
// (128 x 64 each) for large products, 128 x 128 blocks of 8 waves (64 x 32) otherwise;
// 128-byte K steps when K allows, else 64.
#ifndef QS_GEMM_DMA
#define QS_GEMM_DMA 1
#endif
constexpr bool kGemmDma = QS_GEMM_DMA != 0;  // large products take k_gemm_i8_dma

template <int EPI, int BK>
void launch_gemm_bk(const GemmParams& p, hipStream_t s) {
  const bool big = (int64_t)p.M * p.N >= (int64_t)1024 * 8192;
  if (big) {
    constexpr int BM = 256, BN = 256;
    const int G = (int)(cdiv(p.M, BM) * cdiv(p.N, BN));
    hipLaunchKernelGGL((k_gemm_i8<BM, BN, 128, 64, EPI, BK>), dim3(G), dim3(8 * 64), 0, s, p);
  } else {
    constexpr int BM = 128, BN = 128;
    const int G = (int)(cdiv(p.M, BM) * cdiv(p.N, BN));
    hipLaunchKernelGGL((k_gemm_i8<BM, BN, 64, 32, EPI, BK>), dim3(G), dim3(8 * 64), 0, s, p);
  }
}

template <int EPI>
void launch_gemm(const GemmParams& p, hipStream_t s) {
  const bool big = (int64_t)p.M * p.N >= (int64_t)1024 * 8192;
  const bool dma_ok = p.K % 64 == 0 && p.lda % 16 == 0 && p.ldb % 16 == 0 && aligned(p.a, 16) &&
                      aligned(p.b, 16) && 256 * p.lda < INT_MAX && 256 * p.ldb < INT_MAX;
  if (kGemmDma && dma_ok) {
    // epilogue operands by DMA (PRE) when their row slices are whole 16-byte chunks and
    // 16-byte aligned: a copy's range check then never splits a chunk
    const bool side_tail = p.P > 0 && p.P <= kTailSide;
    const bool pre = EPI != EPI_I32 && p.M % 4 == 0 && p.N % 4 == 0 && aligned(p.as, 16) && aligned(p.bs, 16) &&
                     (!side_tail || (aligned(p.xp, 16) && aligned(p.wp, 16) && ((int64_t)p.M * p.P) % 4 == 0 &&
                                     ((int64_t)p.N * p.P) % 4 == 0));
    const bool p2 = p.K % 128 == 0;  // whole 128-byte lines per copy (k_gemm_i8_p2)
    if (big) {
      const int G = (int)(cdiv(p.M, 256) * cdiv(p.N, 256));
      if (p2) {
        if (pre) hipLaunchKernelGGL((k_gemm_i8_p2<256, 256, 128, 64, EPI, EPI == EPI_I32 ? 0 : 1>), dim3(G), dim3(512), 0, s, p);
        else hipLaunchKernelGGL((k_gemm_i8_p2<256, 256, 128, 64, EPI>), dim3(G), dim3(512), 0, s, p);
      } else if (pre) {
        hipLaunchKernelGGL((k_gemm_i8_dma<256, 256, 128, 64, EPI, EPI == EPI_I32 ? 0 : 1>), dim3(G), dim3(512), 0, s, p);
      } else {
        hipLaunchKernelGGL((k_gemm_i8_dma<256, 256, 128, 64, EPI>), dim3(G), dim3(512), 0, s, p);
      }
    } else if (p2 && p.M <= 64) {
      // a weight stream: 64 x 64 tiles (4 waves of 32 x 32) put twice the tiles of 128-row
      // tiles on the CUs, with no copies for absent rows (14336 x 4096, two stages: M = 64
      // 24.0 -> 19.2 us; M = 128 on 128 x 64 tiles 25.6 -> 22.4 us)
      const int G = (int)(cdiv(p.M, 64) * cdiv(p.N, 64));
      if (pre) hipLaunchKernelGGL((k_gemm_i8_p2<64, 64, 32, 32, EPI, EPI == EPI_I32 ? 0 : 1>), dim3(G), dim3(256), 0, s, p);
      else hipLaunchKernelGGL((k_gemm_i8_p2<64, 64, 32, 32, EPI>), dim3(G), dim3(256), 0, s, p);
    } else if (p2 && p.M <= 128) {
      const int G = (int)(cdiv(p.M, 128) * cdiv(p.N, 64));
      if (pre) hipLaunchKernelGGL((k_gemm_i8_p2<128, 64, 32, 64, EPI, EPI == EPI_I32 ? 0 : 1>), dim3(G), dim3(256), 0, s, p);
      else hipLaunchKernelGGL((k_gemm_i8_p2<128, 64, 32, 64, EPI>), dim3(G), dim3(256), 0, s, p);
    } else if (p2 && cdiv(p.M, 256) * cdiv(p.N, 128) <= 128) {
      // few rows (M <= 256 at N <= 16384): 256 x 128 tiles would fill at most half the CUs,
      // each with a full tile of copies; 128 x 128 tiles (8 waves of 32 x 64) double the
      // tiles and cut each one's copies by a third
      const int G = (int)(cdiv(p.M, 128) * cdiv(p.N, 128));
      if (pre) hipLaunchKernelGGL((k_gemm_i8_p2<128, 128, 32, 64, EPI, EPI == EPI_I32 ? 0 : 1>), dim3(G), dim3(512), 0, s, p);
      else hipLaunchKernelGGL((k_gemm_i8_p2<128, 128, 32, 64, EPI>), dim3(G), dim3(512), 0, s, p);
    } else {
      const int G = (int)(cdiv(p.M, 256) * cdiv(p.N, 128));
      if (p2) {
        if (pre) hipLaunchKernelGGL((k_gemm_i8_p2<256, 128, 64, 64, EPI, EPI == EPI_I32 ? 0 : 1>), dim3(G), dim3(512), 0, s, p);
        else hipLaunchKernelGGL((k_gemm_i8_p2<256, 128, 64, 64, EPI>), dim3(G), dim3(512), 0, s, p);
      } else if (pre) {
        hipLaunchKernelGGL((k_gemm_i8_dma<256, 128, 64, 64, EPI, EPI == EPI_I32 ? 0 : 1>), dim3(G), dim3(512), 0, s, p);
      } else {
        hipLaunchKernelGGL((k_gemm_i8_dma<256, 128, 64, 64, EPI>), dim3(G), dim3(512), 0, s, p);
      }
    }
    return;
  }
  if (p.K % 128 == 0) launch_gemm_bk<EPI, 128>(p, s);
  else launch_gemm_bk<EPI, 64>(p, s);
}

int run_gemm(const GemmParams& p, int epi, hipStream_t s) {
  if (p.M == 0 || p.N == 0) return QS_OK;
  const bool fast = p.K % kBK == 0 && p.lda % 16 == 0 && p.ldb % 16 == 0 && aligned(p.a, 16) &&
                    aligned(p.b, 16);
  if (fast) {
    if (epi == EPI_I32) launch_gemm<EPI_I32>(p, s);
    else if (epi == EPI_F32) launch_gemm<EPI_F32>(p, s);
    else launch_gemm<EPI_BF16>(p, s);
    return hip_check(hipGetLastError(), "k_gemm_i8 launch");
  }
  const int64_t outs = (int64_t)p.M * p.N;
  hipLaunchKernelGGL(k_gemm_i8_generic, dim3((unsigned)cdiv(outs, 256)), dim3(256), 0, s, p, epi);
  return hip_check(hipGetLastError(), "k_gemm_i8_generic launch");
}

int check_mnk(int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N <= 0 || K <= 0) return fail(QS_ERR_INVALID, "bad GEMM shape M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30)) return fail(QS_ERR_LIMIT, "GEMM dimension exceeds 2^30");
  return QS_OK;
}

}  // namespace
}  // namespace qs

using namespace qs;

static constexpr int kQuantCpl = 16;  // 16-byte chunks per lane held by k_act_quant_w

extern "C" int qs_act_quant_i8(const void* x, int x_dtype, int64_t ldx, const float* keep,
                               int8_t* q, float* scale, int64_t M, int64_t K, void* stream) {
  if (!x || !q || !scale) return fail(QS_ERR_INVALID, "act_quant: null pointer");
  if (M < 0 || K <= 0 || ldx < K) return fail(QS_ERR_INVALID, "act_quant: bad shape");
  if (M > (1 << 30) || K > (1 << 30)) return fail(QS_ERR_LIMIT, "act_quant: dimension exceeds 2^30");
  if (M == 0) return QS_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int es = x_dtype == QS_F32 ? 4 : 2;
  const int E = 16 / es;
  const bool wave_path = (x_dtype == QS_F32 || x_dtype == QS_BF16 || x_dtype == QS_F16) && K % E == 0 &&
                         K / E <= 64 * kQuantCpl && aligned(x, 16) && (ldx * es) % 16 == 0 &&
                         (!keep || aligned(keep, 16)) && aligned(q, E == 8 ? 8 : 4);
  if (wave_path) {
    // up to 4096 rows, four waves share a row (more waves in flight: M=512 7.2 -> 5.0 us,
    // M=2048 9.7 -> 8.4 us)
    if (M <= 4096 && K / E <= 4 * 64 * (kQuantCpl / 4)) {
      const dim3 grid((unsigned)M);
      if (x_dtype == QS_F32)
        hipLaunchKernelGGL((k_act_quant_w<QS_F32, kQuantCpl / 4, 4>), grid, dim3(256), 0, s, x, ldx, keep, q, K, scale, (int)M, (int)K);
      else if (x_dtype == QS_BF16)
        hipLaunchKernelGGL((k_act_quant_w<QS_BF16, kQuantCpl / 4, 4>), grid, dim3(256), 0, s, x, ldx, keep, q, K, scale, (int)M, (int)K);
      else
        hipLaunchKernelGGL((k_act_quant_w<QS_F16, kQuantCpl / 4, 4>), grid, dim3(256), 0, s, x, ldx, keep, q, K, scale, (int)M, (int)K);
      return hip_check(hipGetLastError(), "k_act_quant_w launch");
    }
    const dim3 grid((unsigned)cdiv(M, 4));
    if (x_dtype == QS_F32)
      hipLaunchKernelGGL((k_act_quant_w<QS_F32, kQuantCpl, 1>), grid, dim3(256), 0, s, x, ldx, keep, q, K, scale, (int)M, (int)K);
    else if (x_dtype == QS_BF16)
      hipLaunchKernelGGL((k_act_quant_w<QS_BF16, kQuantCpl, 1>), grid, dim3(256), 0, s, x, ldx, keep, q, K, scale, (int)M, (int)K);
    else
      hipLaunchKernelGGL((k_act_quant_w<QS_F16, kQuantCpl, 1>), grid, dim3(256), 0, s, x, ldx, keep, q, K, scale, (int)M, (int)K);
    return hip_check(hipGetLastError(), "k_act_quant_w launch");
  }
  if (x_dtype == QS_F32)
    hipLaunchKernelGGL(k_act_quant<QS_F32>, dim3((unsigned)M), dim3(256), 0, s, x, ldx, keep, q, K, scale, (int)K);
  else if (x_dtype == QS_BF16)
    hipLaunchKernelGGL(k_act_quant<QS_BF16>, dim3((unsigned)M), dim3(256), 0, s, x, ldx, keep, q, K, scale, (int)K);
  else if (x_dtype == QS_F16)
    hipLaunchKernelGGL(k_act_quant<QS_F16>, dim3((unsigned)M), dim3(256), 0, s, x, ldx, keep, q, K, scale, (int)K);
  else
    return fail(QS_ERR_INVALID, "act_quant: dtype must be F32, BF16 or F16");
  return hip_check(hipGetLastError(), "k_act_quant launch");
}

extern "C" int qs_outlier_topk(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K,
                               int k, float* colmax, int64_t* idx, float* keep, void* stream) {
  if (!x || !colmax || !idx || !keep) return fail(QS_ERR_INVALID, "outlier_topk: null pointer");
  if (M <= 0 || K <= 0 || ldx < K) return fail(QS_ERR_INVALID, "outlier_topk: bad shape");
  if (k < 1 || k > 64 || k > K) return fail(QS_ERR_LIMIT, "outlier_topk: k must be in 1..min(64, K)");
  if (M > (int64_t)65535 * 64) return fail(QS_ERR_LIMIT, "outlier_topk: too many rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (x_dtype != QS_F32 && x_dtype != QS_BF16 && x_dtype != QS_F16)
    return fail(QS_ERR_INVALID, "outlier_topk: dtype must be F32, BF16 or F16");
  if (M <= 1024) {
    // one pass, one launch: up to 64 rows per thread
    const dim3 grid((unsigned)cdiv(K, 64));
    if (x_dtype == QS_F32)
      hipLaunchKernelGGL(k_col_absmax_rows<QS_F32>, grid, dim3(1024), 0, s, x, ldx, (int)M, (int)K, colmax);
    else if (x_dtype == QS_BF16)
      hipLaunchKernelGGL(k_col_absmax_rows<QS_BF16>, grid, dim3(1024), 0, s, x, ldx, (int)M, (int)K, colmax);
    else
      hipLaunchKernelGGL(k_col_absmax_rows<QS_F16>, grid, dim3(1024), 0, s, x, ldx, (int)M, (int)K, colmax);
  } else {
    const int parts = (int)cdiv(M, 64);
    const dim3 grid((unsigned)cdiv(K, 256), (unsigned)parts);
    hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)cdiv(K, 256)), dim3(256), 0, s, colmax, (int)K);
    if (x_dtype == QS_F32)
      hipLaunchKernelGGL(k_col_absmax<QS_F32>, grid, dim3(256), 0, s, x, ldx, (int)M, (int)K, colmax);
    else if (x_dtype == QS_BF16)
      hipLaunchKernelGGL(k_col_absmax<QS_BF16>, grid, dim3(256), 0, s, x, ldx, (int)M, (int)K, colmax);
    else
      hipLaunchKernelGGL(k_col_absmax<QS_F16>, grid, dim3(256), 0, s, x, ldx, (int)M, (int)K, colmax);
  }
  if (k <= 16 && K <= 1024 * 4)
    hipLaunchKernelGGL(k_topk_small<4>, dim3(1), dim3(1024), 0, s, colmax, (int)K, k, idx, keep);
  else if (k <= 16 && K <= 1024 * 16)
    hipLaunchKernelGGL(k_topk_small<16>, dim3(1), dim3(1024), 0, s, colmax, (int)K, k, idx, keep);
  else if (K <= 1024 * kRadixVpt)
    hipLaunchKernelGGL(k_topk_radix, dim3(1), dim3(1024), 0, s, colmax, (int)K, k, idx, keep);
  else
    hipLaunchKernelGGL(k_topk, dim3(1), dim3(1024), 0, s, colmax, (int)K, 1, k, idx, keep);
  return hip_check(hipGetLastError(), "outlier_topk launch");
}

extern "C" int qs_w8a8_side_gather(const void* x, int x_dtype, int64_t ldx, const int8_t* qw,
                                   const float* sw, const int64_t* idx, int P, int64_t M,
                                   int64_t N, int64_t K, float* xp, float* wp, void* stream) {
  if (!x || !qw || !sw || !idx || !xp || !wp) return fail(QS_ERR_INVALID, "side_gather: null pointer");
  if (P < 1 || P > 64) return fail(QS_ERR_LIMIT, "side_gather: 1..64 protected columns");
  if (M < 0 || N <= 0 || K <= 0 || ldx < K) return fail(QS_ERR_INVALID, "side_gather: bad shape");
  const int64_t total = (M + N) * P;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned blocks = (unsigned)cdiv(total, 256);
  if (x_dtype == QS_F32)
    hipLaunchKernelGGL(k_gather_side<QS_F32>, dim3(blocks), dim3(256), 0, s, x, ldx, qw, K, sw, idx, P, (int)M, (int)N, xp, wp);
  else if (x_dtype == QS_BF16)
    hipLaunchKernelGGL(k_gather_side<QS_BF16>, dim3(blocks), dim3(256), 0, s, x, ldx, qw, K, sw, idx, P, (int)M, (int)N, xp, wp);
  else if (x_dtype == QS_F16)
    hipLaunchKernelGGL(k_gather_side<QS_F16>, dim3(blocks), dim3(256), 0, s, x, ldx, qw, K, sw, idx, P, (int)M, (int)N, xp, wp);
  else
    return fail(QS_ERR_INVALID, "side_gather: dtype must be F32, BF16 or F16");
  return hip_check(hipGetLastError(), "k_gather_side launch");
}

namespace {
template <int CPL, int WPR, int VM>
void launch_protect(int x_dtype, dim3 grid, const ProtectParams& p, hipStream_t s) {
  if (x_dtype == QS_F32) hipLaunchKernelGGL((k_protect_quant<QS_F32, CPL, WPR, VM>), grid, dim3(256), 0, s, p);
  else if (x_dtype == QS_BF16) hipLaunchKernelGGL((k_protect_quant<QS_BF16, CPL, WPR, VM>), grid, dim3(256), 0, s, p);
  else hipLaunchKernelGGL((k_protect_quant<QS_F16, CPL, WPR, VM>), grid, dim3(256), 0, s, p);
}
}  // namespace

extern "C" int qs_w8a8_protect_quant(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int k,
                                     const int8_t* qw, const float* sw, int64_t N, float* colmax_ws,
                                     int8_t* q, float* act_scale, float* xp, float* wp, int64_t* idx,
                                     float* keep, void* stream) {
  if (!x || !qw || !sw || !colmax_ws || !q || !act_scale || !xp || !wp)
    return fail(QS_ERR_INVALID, "protect_quant: null pointer");
  if (!aligned(colmax_ws, 16) || (keep && !aligned(keep, 16)))
    return fail(QS_ERR_INVALID, "protect_quant: colmax_ws and keep must be 16-byte aligned");
  if (M < 1 || N < 1 || K < 1 || ldx < K) return fail(QS_ERR_INVALID, "protect_quant: bad shape");
  if (k < 1 || k > kProtectMaxP || k > K) return fail(QS_ERR_LIMIT, "protect_quant: k must be in 1..min(%d, K)", kProtectMaxP);
  if (M > (1 << 30) || N > (1 << 30)) return fail(QS_ERR_LIMIT, "protect_quant: dimension exceeds 2^30");
  if (x_dtype != QS_F32 && x_dtype != QS_BF16 && x_dtype != QS_F16)
    return fail(QS_ERR_INVALID, "protect_quant: dtype must be F32, BF16 or F16");
  const int es = x_dtype == QS_F32 ? 4 : 2;
  const int E = 16 / es;
  if (K > kProtectMaxK || K % E || K / E > 64 * kQuantCpl || !aligned(x, 16) || (ldx * es) % 16 ||
      !aligned(q, E == 8 ? 8 : 4))
    return fail(QS_ERR_UNSUPPORTED, "protect_quant: needs K <= %d, K %% %d == 0 and 16-byte aligned rows",
                kProtectMaxK, E);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int R = (int)cdiv(M, 1024);
  if (R > 65535) return fail(QS_ERR_LIMIT, "protect_quant: too many rows");
  const dim3 cgrid((unsigned)cdiv(K, 64), (unsigned)R);
  if (x_dtype == QS_F32)
    hipLaunchKernelGGL(k_col_absmax_v<QS_F32>, cgrid, dim3(1024), 0, s, x, ldx, (int)M, (int)K, colmax_ws);
  else if (x_dtype == QS_BF16)
    hipLaunchKernelGGL(k_col_absmax_v<QS_BF16>, cgrid, dim3(1024), 0, s, x, ldx, (int)M, (int)K, colmax_ws);
  else
    hipLaunchKernelGGL(k_col_absmax_v<QS_F16>, cgrid, dim3(1024), 0, s, x, ldx, (int)M, (int)K, colmax_ws);
  int st = hip_check(hipGetLastError(), "k_col_absmax_v launch");
  if (st) return st;
  ProtectParams p{};
  p.x = x;
  p.ldx = ldx;
  p.M = (int)M;
  p.K = (int)K;
  p.N = (int)N;
  p.colpart = colmax_ws;
  p.R = R;
  p.kk = k;
  p.qw = qw;
  p.sw = sw;
  p.q = q;
  p.scale = act_scale;
  p.xp = xp;
  p.wp = wp;
  p.idx = idx;
  p.keep = keep;
  // 4 waves per row up to 1024 rows, else 4 rows per workgroup: the selection is repeated
  // per workgroup, and the grid stays within one resident round.  K <= 4096 takes the
  // instantiation with 16 keys per thread and half the row registers: every wave runs
  // once through the kernel's fully unrolled code, and the smaller form is 1.3 µs
  // (M = 512) and 2.3 µs (M = 2048) faster for K = 4096.
  const bool half = K <= 4096;
  if (M <= 1024 && K / E <= 4 * 64 * (kQuantCpl / 4)) {
    const dim3 grid((unsigned)M);
    if (half && K / E <= 4 * 64 * (kQuantCpl / 8)) launch_protect<kQuantCpl / 8, 4, 16>(x_dtype, grid, p, s);
    else launch_protect<kQuantCpl / 4, 4, kProtectMaxK / 256>(x_dtype, grid, p, s);
  } else {
    const dim3 grid((unsigned)cdiv(M, 4));
    if (half && K / E <= 64 * (kQuantCpl / 2)) launch_protect<kQuantCpl / 2, 1, 16>(x_dtype, grid, p, s);
    else launch_protect<kQuantCpl, 1, kProtectMaxK / 256>(x_dtype, grid, p, s);
  }
  return hip_check(hipGetLastError(), "k_protect_quant launch");
}

extern "C" int qs_gemm_i8i8_i32(const int8_t* qx, const int8_t* qw, int32_t* acc, int64_t M,
                                int64_t N, int64_t K, void* stream) {
  if (!qx || !qw || !acc) return fail(QS_ERR_INVALID, "gemm_i8: null pointer");
  int st = check_mnk(M, N, K);
  if (st) return st;
  GemmParams p{};
  p.a = qx;
  p.b = qw;
  p.lda = K;
  p.ldb = K;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.c = acc;
  p.ldc = N;
  return run_gemm(p, EPI_I32, static_cast<hipStream_t>(stream));
}

extern "C" int qs_w8a8_gemm(const int8_t* qx, const float* act_scale, const int8_t* qw,
                            const float* w_scale, const float* side_x, const float* side_w,
                            int P, void* y, int y_dtype, int64_t M, int64_t N, int64_t K,
                            void* stream) {
  if (!qx || !act_scale || !qw || !w_scale || !y) return fail(QS_ERR_INVALID, "w8a8_gemm: null pointer");
  if (P < 0 || P > 64 || (P > 0 && (!side_x || !side_w)))
    return fail(QS_ERR_INVALID, "w8a8_gemm: side path needs 1..64 columns and both operands");
  if (y_dtype != QS_F32 && y_dtype != QS_BF16) return fail(QS_ERR_INVALID, "w8a8_gemm: y dtype must be F32 or BF16");
  int st = check_mnk(M, N, K);
  if (st) return st;
  GemmParams p{};
  p.a = qx;
  p.b = qw;
  p.lda = K;
  p.ldb = K;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.c = y;
  p.ldc = N;
  p.as = act_scale;
  p.bs = w_scale;
  p.xp = side_x;
  p.wp = side_w;
  p.P = P;
  return run_gemm(p, y_dtype == QS_F32 ? EPI_F32 : EPI_BF16, static_cast<hipStream_t>(stream));
}
