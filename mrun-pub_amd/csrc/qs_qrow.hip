// int8 row-scaled ("qrow") QStore linears on gfx950.
//
// Kernels
//   k_dequant_v / k_dequant_any : W = float(code) * scale -> f32 / bf16 / f16.
//   k_w8a16<...>                : y = x @ W^T for bf16/f16 activations.  Weights stream
//                                 straight from HBM into VGPRs with 128-bit loads, are
//                                 dequantized in registers (bf16(float(code)*scale), the
//                                 W8A16 contract) and fed to v_mfma_f32_16x16x32_{bf16,f16}
//                                 with the activations as the A operand (M <= 32 rows
//                                 padded to 16-row tiles).  MFMA replaces the per-element
//                                 multiply-add, so the VALU only pays for the dequant
//                                 (cvt_sdwa + mul + half a cvt_pk per weight byte).
//                                 K is split across the waves of a workgroup and reduced
//                                 through LDS in a fixed order.  Used for 5 <= M.
//   k_w8a16_s<...>              : the same contract as a streaming kernel -- one wave per
//                                 (tile, K slice) with a sliding window of chunks in
//                                 flight, SwiGLU planes sharing a wave, activations in LDS
//                                 when they are small.  Used for SwiGLU at 5 <= M and for
//                                 long rows (K >= 4096) while the activations fit in LDS.
//   k_gemv_valu<...>            : M <= 4 bf16/f16 decode rows and every fp32-activation
//                                 call: one wave per weight row, 1 KiB
//                                 contiguous row segments per instruction issued in row
//                                 order through a 4-chunk window, exact-width tail,
//                                 VALU dequant + fma / v_dot2, fixed-order DPP wave sum.
//                                 One bf16/f16 row: each lane loads the activations of
//                                 its own weight bytes into registers; otherwise the
//                                 activations are staged in LDS.  Also the row-stable
//                                 (batch invariant) lane.
//   k_gemv_xg / k_gemv_xg_swi : k_gemv_valu's register-activation path (up to 4 bf16/f16
//                                 rows) with scalar kernel arguments, the ones its first
//                                 loads need leading, so the hardware preloads them into
//                                 SGPRs before the wave starts (no argument load round).
//   k_gemv_top2_xg / k_gemv_top2: the same row work with a running top-2 per wave
//                                 instead of stores (fused head + top-2), persistent.
//   k_generic                   : any shape / alignment, one wave per output row.
//
// MFMA operand mapping (16x16x32, wave64): lane l supplies row (l & 15) of A and
// column (l & 15) of B, holding 8 consecutive k of the k-block (l >> 4).  The k order
// inside the block is irrelevant as long as A and B agree, so lane l simply loads the
// 32 contiguous bytes at k = 128*c + 32*(l>>4) of weight row (l & 15) and the matching
// 32 activations; each 8 of them feed one MFMA (4 per 128-k chunk).  The accumulator of
// lane l holds D[4*(l>>4) + q][l & 15], q = 0..3.
#include "qs_common.h"

#include <mutex>
#include <type_traits>

namespace qs {

struct QrowLin {
  const int8_t* codes;
  const float* scales;
  void* y;
  int64_t ldy;
  int N;
  int tile_begin;  // first workgroup index of this linear
};

struct QrowParams {
  const void* x;
  int64_t ldx;
  int M;
  int K;
  int n_lin;
  QrowLin lin[4];
};

// ----------------------------------------------------------------------------------
// dequant
// ----------------------------------------------------------------------------------
// Lane-contiguous stores: a thread widens E codes (4 for fp32 output, 8 for bf16 / fp16)
// into one 16-byte store, so a wave's store instruction writes 1 KB of consecutive output.
// (Sixteen codes per thread wrote 64 or 32 bytes per lane as 16-byte pieces strided
// across the wave: 79.4 against 60.7 us for a 14336 x 4096 fp32 dequant, same box.)
// Each thread takes U such pieces, 256 apart: all U code loads are issued first and
// waited for once, then the U stores follow, and the wave ends without waiting for them
// (stores and loads share one completion counter, so a load issued behind a store would
// wait for that store too).  The chunk's first row comes from one division per chunk;
// each piece's row and column from a 32-bit division of its offset within the chunk.
constexpr int kDequantPieces = 4;  // 16-byte pieces per thread

template <int OUT, int U>
__global__ __launch_bounds__(256) void k_dequant_v(const int8_t* __restrict__ codes,
                                                   const float* __restrict__ scales,
                                                   void* __restrict__ out, int64_t N,
                                                   int64_t K, int64_t ld_out) {
  constexpr int E = OUT == QS_F32 ? 4 : 8;
  typedef int i32x2 __attribute__((ext_vector_type(2)));
  using CW = typename std::conditional<E == 4, int, i32x2>::type;
  const int64_t per_row = K / E;
  const int64_t total = N * per_row;
  for (int64_t base = (int64_t)blockIdx.x * 256 * U; base < total; base += (int64_t)gridDim.x * 256 * U) {
    const int64_t n0 = base / per_row;
    const uint32_t c0 = (uint32_t)(base - n0 * per_row);
    int64_t n[U];
    uint32_t c[U];
    bool ok[U];
    CW w[U];
    float s[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t off = c0 + (uint32_t)(u * 256 + threadIdx.x);  // < per_row + 256 U
      const uint32_t q = off / (uint32_t)per_row;
      n[u] = n0 + q;
      c[u] = off - q * (uint32_t)per_row;
      ok[u] = base + u * 256 + threadIdx.x < total;
      const int64_t nn = ok[u] ? n[u] : 0;
      const uint32_t cc = ok[u] ? c[u] : 0u;
      w[u] = *reinterpret_cast<const CW*>(codes + nn * K + (int64_t)cc * E);
      s[u] = scales[nn];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!ok[u]) continue;
      if constexpr (OUT == QS_F32) {
        f32x4 v;
        v[0] = sbyte_f32<0>(w[u]) * s[u];
        v[1] = sbyte_f32<1>(w[u]) * s[u];
        v[2] = sbyte_f32<2>(w[u]) * s[u];
        v[3] = sbyte_f32<3>(w[u]) * s[u];
        *reinterpret_cast<f32x4*>(static_cast<float*>(out) + n[u] * ld_out + (int64_t)c[u] * 4) = v;
      } else if constexpr (OUT == QS_BF16) {
        bf16x8 o;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          o[4 * j + 0] = static_cast<__bf16>(sbyte_f32<0>(w[u][j]) * s[u]);
          o[4 * j + 1] = static_cast<__bf16>(sbyte_f32<1>(w[u][j]) * s[u]);
          o[4 * j + 2] = static_cast<__bf16>(sbyte_f32<2>(w[u][j]) * s[u]);
          o[4 * j + 3] = static_cast<__bf16>(sbyte_f32<3>(w[u][j]) * s[u]);
        }
        *reinterpret_cast<bf16x8*>(static_cast<uint16_t*>(out) + n[u] * ld_out + (int64_t)c[u] * 8) = o;
      } else {
        f16x8 o;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          o[4 * j + 0] = static_cast<_Float16>(sbyte_f32<0>(w[u][j]) * s[u]);
          o[4 * j + 1] = static_cast<_Float16>(sbyte_f32<1>(w[u][j]) * s[u]);
          o[4 * j + 2] = static_cast<_Float16>(sbyte_f32<2>(w[u][j]) * s[u]);
          o[4 * j + 3] = static_cast<_Float16>(sbyte_f32<3>(w[u][j]) * s[u]);
        }
        *reinterpret_cast<f16x8*>(static_cast<uint16_t*>(out) + n[u] * ld_out + (int64_t)c[u] * 8) = o;
      }
    }
  }
}

__global__ __launch_bounds__(256) void k_dequant_any(const int8_t* __restrict__ codes,
                                                     const float* __restrict__ scales,
                                                     void* __restrict__ out, int out_dtype,
                                                     int64_t N, int64_t K, int64_t ld_out) {
  const int64_t total = N * K;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i / K;
    const int64_t k = i - n * K;
    const float v = static_cast<float>(codes[i]) * scales[n];
    if (out_dtype == QS_F32)
      static_cast<float*>(out)[n * ld_out + k] = v;
    else if (out_dtype == QS_BF16)
      static_cast<uint16_t*>(out)[n * ld_out + k] = f32_to_bf16_bits(v);
    else
      static_cast<uint16_t*>(out)[n * ld_out + k] = f32_to_f16_bits(v);
  }
}

// ----------------------------------------------------------------------------------
// W8A16 MFMA kernel
// ----------------------------------------------------------------------------------
template <bool F16>
struct HalfOps;

template <>
struct HalfOps<false> {
  typedef bf16x8 vec;
  static __device__ __forceinline__ void deq(i32x4 w, float s, vec& lo, vec& hi) {
    deq16_bf16(w, s, lo, hi);
  }
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t out(float v) { return f32_to_bf16_bits(v); }
};

template <>
struct HalfOps<true> {
  typedef f16x8 vec;
  static __device__ __forceinline__ void deq(i32x4 w, float s, vec& lo, vec& hi) {
    deq16_f16(w, s, lo, hi);
  }
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t out(float v) { return f32_to_f16_bits(v); }
};

__device__ __forceinline__ float silu_f32(float g) { return g * (1.0f / (1.0f + expf(-g))); }

// One round of the K loop for one wave.  A chunk is 128 k of 16 weight rows: lane l
// reads the 32 contiguous bytes at k = 128*c + 32*(l>>4) of row (l & 15) with two
// back-to-back 128-bit loads, so the wave's two instructions cover whole 128-byte lines
// of all 16 rows (no line is shared with another wave).  Order of requests: the
// activations of U chunks (L2-resident, they return first), the U weight chunks
// (nontemporal HBM loads), then -- on the first round -- the row scale; only then
// dequantize and feed 4 MFMAs per chunk, so one round costs one memory latency.
template <int MT, int U, int KW, bool F16>
__device__ __forceinline__ void w8a16_round(int c0, int C, const int8_t* wrow,
                                            const float* srow, float& sc, bool first,
                                            const uint16_t* const (&xrow)[MT],
                                            const bool (&mval)[MT], f32x4 (&acc)[MT]) {
  typedef HalfOps<F16> H;
  typedef typename H::vec hvec;
  hvec xa[U][MT][4];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int cc = c0 + u * KW;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        xa[u][t][j] = (cc < C && mval[t])
                          ? *reinterpret_cast<const hvec*>(xrow[t] + (int64_t)cc * 128 + 8 * j)
                          : hvec{};
    }
  }
  i32x4 wv[U][2];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int cc = c0 + u * KW;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      wv[u][h] = cc < C ? __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(
                              wrow + (int64_t)cc * 128 + 16 * h))
                        : i32x4{0, 0, 0, 0};
  }
  if (first) sc = *srow;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (c0 + u * KW < C) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        hvec b0, b1;
        H::deq(wv[u][h], sc, b0, b1);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          acc[t] = H::mma(xa[u][t][2 * h], b0, acc[t]);
          acc[t] = H::mma(xa[u][t][2 * h + 1], b1, acc[t]);
        }
      }
    }
  }
}

// One workgroup = one 16-row weight tile of P planes (P = 1: a plain linear; P = 2: the
// gate and up projections of one SwiGLU tile).  Its P*KW waves split the work as
// plane = wave % P, K slice = wave / P; each wave owns chunks ks, ks+KW, ks+2*KW, ...
// The per-row accumulation order depends only on (K, KW) -- chosen from (N, K), never
// from M -- so batched rows are bit-identical to B = 1 rows.
// MT: 16-row activation tiles (M <= 16 * MT).  U: chunks in flight per wave per round.
template <int P, int MT, int KW, int U, bool F16>
__global__ __launch_bounds__(P * KW * 64) void k_w8a16(QrowParams p) {
  typedef HalfOps<F16> H;
  constexpr int WAVES = P * KW;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int plane = wave % P;
  const int ks = wave / P;
  const int col = lane & 15;
  const int grp = lane >> 4;

  int li = 0;
  if (P == 1) {
#pragma unroll
    for (int j = 1; j < 4; ++j)
      if (j < p.n_lin && (int)blockIdx.x >= p.lin[j].tile_begin) li = j;
  }
  const int tile = (int)blockIdx.x - p.lin[li].tile_begin;
  const QrowLin& L = p.lin[P == 2 ? plane : li];
  const int N = p.lin[li].N;
  const int K = p.K;
  const int M = p.M;
  const int n0 = tile * 16;
  int n = n0 + col;
  n = n < N ? n : N - 1;  // clamp: the lane's outputs are not stored
  const int8_t* wrow = L.codes + (int64_t)n * K + 32 * grp;
  const float* srow = L.scales + n;

  const uint16_t* xrow[MT];
  bool mval[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = 16 * t + col;
    mval[t] = m < M;
    xrow[t] = static_cast<const uint16_t*>(p.x) + (int64_t)(mval[t] ? m : 0) * p.ldx + 32 * grp;
  }
  f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int C = K / 128;
  float sc = 0.f;
  // first round peeled so that the scale load trails the first weight loads
  w8a16_round<MT, U, KW, F16>(ks, C, wrow, srow, sc, true, xrow, mval, acc);
  for (int c0 = ks + U * KW; c0 < C; c0 += U * KW)
    w8a16_round<MT, U, KW, F16>(c0, C, wrow, srow, sc, false, xrow, mval, acc);

  // cross-wave reduction: per plane, K slices summed in fixed order
  __shared__ f32x4 red[WAVES][MT][64];
#pragma unroll
  for (int t = 0; t < MT; ++t) red[wave][t][lane] = acc[t];
  __syncthreads();
  if (wave != 0) return;
  f32x4 out[P][MT];
#pragma unroll
  for (int pl = 0; pl < P; ++pl)
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      f32x4 s = red[pl][t][lane];
#pragma unroll
      for (int k2 = 1; k2 < KW; ++k2) s += red[k2 * P + pl][t][lane];
      out[pl][t] = s;
    }

  // store: lane holds D[m = 16t + 4*grp + q][n = n0 + col]
  const int no = n0 + col;
  if (no >= N) return;
  if (P == 2) {
    uint16_t* y = static_cast<uint16_t*>(p.lin[0].y);
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = 16 * t + 4 * grp + q;
        if (m < M) {
          const float gt = bf16_bits_to_f32(f32_to_bf16_bits(out[0][t][q]));
          const float ut = bf16_bits_to_f32(f32_to_bf16_bits(out[P - 1][t][q]));
          const float sl = bf16_bits_to_f32(f32_to_bf16_bits(silu_f32(gt)));
          y[(int64_t)m * p.lin[0].ldy + no] = f32_to_bf16_bits(sl * ut);
        }
      }
  } else {
    uint16_t* y = static_cast<uint16_t*>(p.lin[li].y);
    const int64_t ldy = p.lin[li].ldy;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = 16 * t + 4 * grp + q;
        if (m < M) y[(int64_t)m * ldy + no] = H::out(out[0][t][q]);
      }
  }
}

// Streaming W8A16 MFMA kernel (3 <= M <= 32).  One wave per (16-row tile, K slice); the
// P planes of a SwiGLU tile share the wave, so each activation fragment is loaded once
// for both.  A wave walks its chunks ks, ks + KW, ks + 2*KW, ... (128 k each, the lane
// mapping of k_w8a16) through a window of W chunks in flight: chunk i + W is requested
// as soon as chunk i has been consumed, so the wave waits for memory once per slice
// rather than once per batch of chunks.  Window slots past the slice load out of the
// buffer's range (zero, no memory access), which keeps every wait count static.
// Activation rows m >= M are zero and never stored.  The KW
// slices of a tile are summed through LDS in a fixed order and KW depends on (N, K)
// only, so within this kernel a row does not depend on the other rows of the batch.
template <int P, int MT, int KW, int W, bool F16, bool XL>
__global__ __launch_bounds__(KW * 64) void k_w8a16_s(QrowParams p) {
  typedef HalfOps<F16> H;
  typedef typename H::vec hvec;
  const int lane = threadIdx.x & 63;
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, grp = lane >> 4;

  int li = 0;
  if (P == 1) {
#pragma unroll
    for (int j = 1; j < 4; ++j)
      if (j < p.n_lin && (int)blockIdx.x >= p.lin[j].tile_begin) li = j;
  }
  const int tile = (int)blockIdx.x - p.lin[li].tile_begin;
  const int N = p.lin[li].N;
  const int K = p.K;
  const int M = p.M;
  const int n0 = tile * 16;
  const int n = min(n0 + col, N - 1);  // clamped lanes compute a row that is not stored
  // Buffer loads: a 32-bit lane offset plus a uniform chunk offset (the host checks that
  // N*K and M*ldx*2 fit in 31 bits).  A slot past the slice loads at lane offset `wlim` /
  // `xlim` with chunk offset 0: that lane offset alone is outside the buffer's range, so
  // the load returns zero without touching memory.
  __amdgpu_buffer_rsrc_t wr[P];
  const float* srow[P];
  const int wlim = N * K;
#pragma unroll
  for (int pl = 0; pl < P; ++pl) {
    const QrowLin& L = p.lin[P == 2 ? pl : li];
    wr[pl] = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(L.codes), (short)0, wlim, 0x00020000);
    srow[pl] = L.scales + n;
  }
  const int wlane = n * K + 32 * grp;
  const int xlim = M * (int)p.ldx * 2;
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.x), (short)0, xlim, 0x00020000);
  int xlane[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) xlane[t] = (min(16 * t + col, M - 1) * (int)p.ldx + 32 * grp) * 2;
  const int C = K / 128;
  const int nch = ks < C ? (C - 1 - ks) / KW + 1 : 0;  // chunks of this wave's slice

  // XL: the M activation rows sit in LDS (row stride 2K + 16 bytes: the 16 rows of a
  // fragment read fall in distinct banks), copied once per workgroup right after the
  // weight window has been requested (the copy lands behind those loads, about when the
  // first chunk can be consumed), and each chunk's fragments are read from LDS while the
  // previous chunk is multiplied -- the vector-memory queue then carries only the HBM
  // weight stream.
  extern __shared__ __attribute__((aligned(16))) uint8_t xl[];
  const int xstride = 2 * K + 16;

  static_assert(!XL || W % 2 == 0, "the activation double buffer follows the slot parity");
  i32x4 wv[W][P][2];
  hvec xa[XL ? 2 : W][MT][4];
  auto issue = [&](int slot, int i) {
    const bool live = i < nch;
    const int koff = (ks + i * KW) * 128;
    if constexpr (!XL) {
      const int xs = live ? 2 * koff : 0;
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // only the lanes of existing rows fetch; padded rows are zero
          xa[slot][t][j] = hvec{};
          if (16 * t + col < M)
            xa[slot][t][j] = __builtin_bit_cast(
                hvec, __builtin_amdgcn_raw_buffer_load_b128(xr, live ? xlane[t] + 16 * j : xlim, xs, 0));
        }
    }
    const int ws = live ? koff : 0;
#pragma unroll
    for (int pl = 0; pl < P; ++pl)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        wv[slot][pl][h] = __builtin_bit_cast(
            i32x4, __builtin_amdgcn_raw_buffer_load_b128(wr[pl], live ? wlane + 16 * h : wlim, ws, 0));
  };
  float sc[P];
  f32x4 acc[P][MT];
#pragma unroll
  for (int pl = 0; pl < P; ++pl)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[pl][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  // activation fragments of chunk i from LDS into buffer b (XL)
  auto xfrag = [&](int b, int i) {
    const int koff = (ks + min(i, nch - 1) * KW) * 128;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = 16 * t + col;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xa[b][t][j] = hvec{};
        if (m < M) xa[b][t][j] = *reinterpret_cast<const hvec*>(xl + m * xstride + 2 * (koff + 32 * grp + 8 * j));
      }
    }
  };
  auto consume = [&](int slot, int i) {
    // chunk i = (multiple of W) + slot with W even: the buffer parity is static
    const int xs = XL ? (slot & 1) : slot;
    if constexpr (XL) xfrag(xs ^ 1, i + 1);
#pragma unroll
    for (int pl = 0; pl < P; ++pl)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        hvec b0, b1;
        H::deq(wv[slot][pl][h], sc[pl], b0, b1);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          acc[pl][t] = H::mma(xa[xs][t][2 * h], b0, acc[pl][t]);
          acc[pl][t] = H::mma(xa[xs][t][2 * h + 1], b1, acc[pl][t]);
        }
      }
  };

  // W chunks in flight first, the row scales behind them
#pragma unroll
  for (int s = 0; s < W; ++s) {
    issue(s, s);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int pl = 0; pl < P; ++pl) sc[pl] = *srow[pl];
  if constexpr (XL) {
    const int pieces = K / 8;  // 16-byte pieces per row
    for (int q = threadIdx.x; q < M * pieces; q += KW * 64) {
      const int m = q / pieces, c = q - m * pieces;
      *reinterpret_cast<i32x4*>(xl + m * xstride + 16 * c) =
          *reinterpret_cast<const i32x4*>(static_cast<const uint16_t*>(p.x) + (int64_t)m * p.ldx + 8 * c);
    }
    __syncthreads();
    if (nch > 0) xfrag(0, 0);
  }
  for (int base = 0; base < nch; base += W) {
#pragma unroll
    for (int s = 0; s < W; ++s) {
      if (base + s < nch) consume(s, base + s);
      __builtin_amdgcn_sched_barrier(0);
      issue(s, base + s + W);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  if constexpr (KW > 1) {
    __shared__ f32x4 red[KW][P][MT][64];
#pragma unroll
    for (int pl = 0; pl < P; ++pl)
#pragma unroll
      for (int t = 0; t < MT; ++t) red[ks][pl][t][lane] = acc[pl][t];
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int pl = 0; pl < P; ++pl)
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        f32x4 s = red[0][pl][t][lane];
#pragma unroll
        for (int k2 = 1; k2 < KW; ++k2) s += red[k2][pl][t][lane];
        acc[pl][t] = s;
      }
  }

  // store: lane holds D[m = 16t + 4*grp + q][n = n0 + col]
  const int no = n0 + col;
  if (no >= N) return;
  if constexpr (P == 2) {
    uint16_t* y = static_cast<uint16_t*>(p.lin[0].y);
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = 16 * t + 4 * grp + q;
        if (m < M) {
          const float gt = bf16_bits_to_f32(f32_to_bf16_bits(acc[0][t][q]));
          const float ut = bf16_bits_to_f32(f32_to_bf16_bits(acc[1][t][q]));
          const float sl = bf16_bits_to_f32(f32_to_bf16_bits(silu_f32(gt)));
          y[(int64_t)m * p.lin[0].ldy + no] = f32_to_bf16_bits(sl * ut);
        }
      }
  } else {
    uint16_t* y = static_cast<uint16_t*>(p.lin[li].y);
    const int64_t ldy = p.lin[li].ldy;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = 16 * t + 4 * grp + q;
        if (m < M) y[(int64_t)m * ldy + no] = H::out(acc[0][t][q]);
      }
  }
}

// ----------------------------------------------------------------------------------
// VALU GEMV for small M (and every fp32-activation call)
// ----------------------------------------------------------------------------------
// One wave per weight row: lane l reads the 16 contiguous codes at k = 1024*c + 16*l
// (one wave instruction = one 1 KiB contiguous row segment).  The M <= MB activation
// rows are staged in LDS per workgroup while the codes are in flight.
//   fp32 x : w = float(code)*scale, fma per element        (QStore fp32 contract)
//   bf16 x : w = bf16(float(code)*scale), v_dot2_f32_bf16   (W8A16 contract)
//   fp16 x : w = fp16(float(code)*scale), v_dot2_f32_f16
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

template <int XT>
struct XElem {
  static constexpr int size = XT == QS_F32 ? 4 : 2;
};

// Dot of NW code words (4 codes each, in registers) at k .. k + 4*NW with the
// activations of the MB rows staged in LDS.
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x3 __attribute__((ext_vector_type(3)));

template <int XT, int MB, int NW>
__device__ __forceinline__ void valu_words(const int (&w)[4], float sc, const uint8_t* xs, int K,
                                           int k, int M, float (&acc)[MB]) {
  constexpr int ES = XElem<XT>::size;
#pragma unroll
  for (int j = 0; j < NW; ++j) {
    const int d = w[j];
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      if (m >= M) continue;
      const uint8_t* xp = xs + ((int64_t)m * K + k + 4 * j) * ES;
      if constexpr (XT == QS_F32) {
        const f32x4 xv = *reinterpret_cast<const f32x4*>(xp);
        const float w4[4] = {sbyte_f32<0>(d) * sc, sbyte_f32<1>(d) * sc, sbyte_f32<2>(d) * sc,
                             sbyte_f32<3>(d) * sc};
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[m] = fmaf(xv[e], w4[e], acc[m]);
      } else {
        const u32x2 xv = *reinterpret_cast<const u32x2*>(xp);
        // copy the elements out first: a bit_cast of an element expression of an
        // ext_vector can read element 0
        const unsigned x0 = xv[0], x1 = xv[1];
        if constexpr (XT == QS_BF16) {
          bf16x2 a, b;
          a[0] = static_cast<__bf16>(sbyte_f32<0>(d) * sc);
          a[1] = static_cast<__bf16>(sbyte_f32<1>(d) * sc);
          b[0] = static_cast<__bf16>(sbyte_f32<2>(d) * sc);
          b[1] = static_cast<__bf16>(sbyte_f32<3>(d) * sc);
          acc[m] = __builtin_amdgcn_fdot2_f32_bf16(a, __builtin_bit_cast(bf16x2, x0), acc[m], false);
          acc[m] = __builtin_amdgcn_fdot2_f32_bf16(b, __builtin_bit_cast(bf16x2, x1), acc[m], false);
        } else {
          f16x2 a, b;
          a[0] = static_cast<_Float16>(sbyte_f32<0>(d) * sc);
          a[1] = static_cast<_Float16>(sbyte_f32<1>(d) * sc);
          b[0] = static_cast<_Float16>(sbyte_f32<2>(d) * sc);
          b[1] = static_cast<_Float16>(sbyte_f32<3>(d) * sc);
          acc[m] = __builtin_amdgcn_fdot2(a, __builtin_bit_cast(f16x2, x0), acc[m], false);
          acc[m] = __builtin_amdgcn_fdot2(b, __builtin_bit_cast(f16x2, x1), acc[m], false);
        }
      }
    }
  }
}

// Decode GEMV, one wave per output row (SWI: gate row n and up row n).  Load order per
// wave: its share of the activations, then the row's tail (K mod 1024 bytes as one
// exact-width 4/8/12-byte load per lane; 16 = a ragged tail read by the lanes it
// covers), then the full 1 KiB chunks in row order, at most kGemvWindow of them in
// flight; each later chunk is requested after the chunk kGemvWindow before it has been
// consumed.  Scheduling barriers keep that issue order, so the wait before chunk c
// covers chunks <= c only and the dequant/dot work of early chunks runs while later
// ones are still arriving.  Chunk slots past the row (U is a bucket >= K/1024) load
// one uniform address and are not consumed, which keeps every wait count static.
// Sums are lane-local in a fixed order (tail, then chunks), then reduced with
// wave_sum_dpp: a row's result never depends on M or on the other rows.
template <bool SWI, int MB>
struct GemvShape {
  // 8 waves share one staged activation copy; the paired SwiGLU grid is larger than
  // one resident round and drains with less tail in small workgroups.
  static constexpr int waves = SWI ? (MB == 1 ? 2 : 4) : 8;
};
constexpr int kGemvWindow = 4;
constexpr int kGemvXgWindow = 4;  // chunks (weights + activations) in flight

// The row work of one wave, shared by the store and top-2 launches: every thread of the
// workgroup calls it (it stages the activations and passes one barrier).  On return the
// wave's row sums are in acc (wave-uniform), n / li name the row and its linear, and the
// result says whether the wave had a row.
// blk is the 8-row (SWI: 2-row) block of this call; stage = false skips the activation
// staging when an earlier call of the same workgroup has already filled xs.
template <int XT, int MB, int U, int TB, bool SWI>
__device__ __forceinline__ bool gemv_wave_rows(const QrowParams& p, int rows, uint8_t* xs,
                                               float (&acc)[SWI ? 2 : 1][MB], int& n_out,
                                               int& li_out, int blk, bool stage) {
  constexpr int WPB = GemvShape<SWI, MB>::waves;
  constexpr int NT = WPB * 64;
  constexpr int ES = XElem<XT>::size;
  constexpr int P = SWI ? 2 : 1;
  constexpr int XMAX16 = MB * (U * 1024 + (TB ? 1024 : 0)) * ES / 16;
  constexpr int XL = (XMAX16 + NT - 1) / NT;
  constexpr bool XREG = XL <= 6;  // activations fit a few registers: load them first
  const int tid = threadIdx.x, lane = tid & 63;
  const int K = p.K, M = p.M;
  const int F = K >> 10;
  const int r0 = blk * WPB + __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool live = r0 < rows;
  const int rr = live ? r0 : 0;
  int li = 0;
  if (!SWI) {
#pragma unroll
    for (int j = 1; j < 4; ++j)
      if (j < p.n_lin && rr >= p.lin[j].tile_begin) li = j;
  }
  const int n = rr - p.lin[li].tile_begin;
  const int row16 = K * ES / 16;
  const uint8_t* xg = static_cast<const uint8_t*>(p.x);

  i32x4 xr[XREG ? XL : 1];
  if (XREG && stage) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      int idx = tid + i * NT;
      idx = idx < M * row16 ? idx : 0;
      const int m = idx / row16, c = idx - m * row16;
      xr[i] = *reinterpret_cast<const i32x4*>(xg + ((int64_t)m * p.ldx * ES + (int64_t)c * 16));
    }
  }
  const int8_t* wrow[P];
  float sc[P];
#pragma unroll
  for (int pl = 0; pl < P; ++pl) {
    const QrowLin& L = p.lin[SWI ? pl : li];
    wrow[pl] = L.codes + (int64_t)n * K;
    sc[pl] = L.scales[n];
  }
  const int rem = K - (F << 10);
  int tw[P][4];
  if constexpr (TB != 0) {
#pragma unroll
    for (int pl = 0; pl < P; ++pl) {
      const int8_t* t = wrow[pl] + (F << 10);
      if constexpr (TB == 16) {
        const i32x4 v = __builtin_nontemporal_load(
            reinterpret_cast<const i32x4*>(16 * lane < rem ? t + 16 * lane : wrow[pl]));
        tw[pl][0] = v[0]; tw[pl][1] = v[1]; tw[pl][2] = v[2]; tw[pl][3] = v[3];
      } else if constexpr (TB == 12) {
        const u32x3 v = __builtin_nontemporal_load(reinterpret_cast<const u32x3*>(t + 12 * lane));
        tw[pl][0] = v[0]; tw[pl][1] = v[1]; tw[pl][2] = v[2]; tw[pl][3] = 0;
      } else if constexpr (TB == 8) {
        const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(t + 8 * lane));
        tw[pl][0] = v[0]; tw[pl][1] = v[1]; tw[pl][2] = 0; tw[pl][3] = 0;
      } else {
        const unsigned v = __builtin_nontemporal_load(reinterpret_cast<const unsigned*>(t + 4 * lane));
        tw[pl][0] = v; tw[pl][1] = 0; tw[pl][2] = 0; tw[pl][3] = 0;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  int wv[P][U][4];
  auto load_chunk = [&](int c) {
#pragma unroll
    for (int pl = 0; pl < P; ++pl) {
      const int8_t* a = c < F ? wrow[pl] + c * 1024 + 16 * lane : wrow[pl];
      const i32x4 v = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(a));
      wv[pl][c][0] = v[0]; wv[pl][c][1] = v[1]; wv[pl][c][2] = v[2]; wv[pl][c][3] = v[3];
      __builtin_amdgcn_sched_barrier(0);
    }
  };
#pragma unroll
  for (int c = 0; c < (kGemvWindow < U ? kGemvWindow : U); ++c) load_chunk(c);

  if (stage) {
    if constexpr (XREG) {
#pragma unroll
      for (int i = 0; i < XL; ++i) {
        const int idx = tid + i * NT;
        if (idx < M * row16) reinterpret_cast<i32x4*>(xs)[idx] = xr[i];
      }
    } else {
      for (int i = tid; i < M * row16; i += NT) {
        const int m = i / row16, c = i - m * row16;
        reinterpret_cast<i32x4*>(xs)[i] =
            *reinterpret_cast<const i32x4*>(xg + ((int64_t)m * p.ldx * ES + (int64_t)c * 16));
      }
    }
    __syncthreads();
  }
  n_out = n;
  li_out = li;
#pragma unroll
  for (int pl = 0; pl < P; ++pl)
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[pl][m] = 0.f;
  if (!live) return false;
  if constexpr (TB == 16) {
    if (16 * lane < rem) {
#pragma unroll
      for (int pl = 0; pl < P; ++pl) valu_words<XT, MB, 4>(tw[pl], sc[pl], xs, K, (F << 10) + 16 * lane, M, acc[pl]);
    }
  } else if constexpr (TB != 0) {
#pragma unroll
    for (int pl = 0; pl < P; ++pl) valu_words<XT, MB, TB / 4>(tw[pl], sc[pl], xs, K, (F << 10) + TB * lane, M, acc[pl]);
  }
#pragma unroll
  for (int c = 0; c < U; ++c) {
    if (c < F) {
#pragma unroll
      for (int pl = 0; pl < P; ++pl) valu_words<XT, MB, 4>(wv[pl][c], sc[pl], xs, K, c * 1024 + 16 * lane, M, acc[pl]);
    }
    if (c + kGemvWindow < U) load_chunk(c + kGemvWindow);
  }
#pragma unroll
  for (int pl = 0; pl < P; ++pl)
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[pl][m] = wave_sum_dpp(acc[pl][m]);
  return true;
}

// k_gemv_valu takes gemv_wave_xg (activations in registers, no LDS) for up to 4 bf16/f16
// rows.
template <int XT, int MB, int U>
constexpr bool kGemvXg = MB <= 4 && XT != QS_F32;

// Waves per workgroup of k_gemv_valu.  Without the shared activation copy a workgroup is
// only a dispatch unit: long rows (K >= 3072, few of them) spread over more CUs in small
// workgroups, short rows keep 8.
#ifndef QS_GEMV_WG_LONG
#define QS_GEMV_WG_LONG 2
#endif
template <int XT, int MB, int U, bool SWI>
constexpr int kGemvWaves = kGemvXg<XT, MB, U> && !SWI && U > 2 ? QS_GEMV_WG_LONG : GemvShape<SWI, MB>::waves;

// One weight word (4 codes) -> two packed bf16/f16 pairs, exact (the W8A16 contract).
template <int XT>
__device__ __forceinline__ void deq_word(int d, float sc, uint32_t& a, uint32_t& b) {
  if constexpr (XT == QS_BF16) {
    bf16x2 u, v;
    u[0] = static_cast<__bf16>(sbyte_f32<0>(d) * sc);
    u[1] = static_cast<__bf16>(sbyte_f32<1>(d) * sc);
    v[0] = static_cast<__bf16>(sbyte_f32<2>(d) * sc);
    v[1] = static_cast<__bf16>(sbyte_f32<3>(d) * sc);
    a = __builtin_bit_cast(uint32_t, u);
    b = __builtin_bit_cast(uint32_t, v);
  } else {
    f16x2 u, v;
    u[0] = static_cast<_Float16>(sbyte_f32<0>(d) * sc);
    u[1] = static_cast<_Float16>(sbyte_f32<1>(d) * sc);
    v[0] = static_cast<_Float16>(sbyte_f32<2>(d) * sc);
    v[1] = static_cast<_Float16>(sbyte_f32<3>(d) * sc);
    a = __builtin_bit_cast(uint32_t, u);
    b = __builtin_bit_cast(uint32_t, v);
  }
}

// acc += a . x0 + b . x1 in the order of valu_words (two v_dot2 with fp32 accumulation).
template <int XT>
__device__ __forceinline__ float dot_word(uint32_t a, uint32_t b, uint32_t x0, uint32_t x1, float acc) {
  if constexpr (XT == QS_BF16) {
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, x0), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, b), __builtin_bit_cast(bf16x2, x1), acc, false);
  } else {
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, x0), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, b), __builtin_bit_cast(f16x2, x1), acc, false);
  }
  return acc;
}

// Up to MB = 4 bf16/f16 activation rows: a lane only ever multiplies the activations of
// its own weight bytes -- 16 per 1 KiB chunk at c * 1024 + 16 * lane, TB at the tail --
// so it loads exactly those straight into registers (after the first wave of a CU they
// come from its L1), each chunk's with the chunk's weights.  No LDS copy and no workgroup
// barrier: every wave runs on its own.  Each weight word is dequantized once and meets
// every row; each row sees the products and order of gemv_wave_rows, whatever MB is.
// Rows m >= M read row M - 1 and are never stored.
template <int XT, int MB, int U, int TB, bool SWI>
__device__ __forceinline__ bool gemv_wave_xg(const QrowParams& p, int rows, float (&acc)[SWI ? 2 : 1][MB],
                                             int& n_out, int& li_out) {
  constexpr int WPB = kGemvWaves<XT, MB, U, SWI>;
  constexpr int P = SWI ? 2 : 1;
  constexpr int W = U < kGemvXgWindow ? U : kGemvXgWindow;  // chunks in flight
  const int lane = threadIdx.x & 63;
  // Every argument the loads below need, requested in one batch: left to itself the
  // compiler asks for them in three dependent rounds (the row bound, the activation row,
  // then past the issue-order barriers the weight rows), one scalar-cache miss each,
  // before the first weight byte is requested.
  if constexpr (SWI) {
    asm volatile("" ::"s"(p.x), "s"(p.ldx), "s"(p.M), "s"(p.K), "s"(rows), "s"(p.lin[0].codes),
                 "s"(p.lin[0].scales), "s"(p.lin[1].codes), "s"(p.lin[1].scales), "s"(p.lin[0].tile_begin));
  } else {
    asm volatile("" ::"s"(p.x), "s"(p.ldx), "s"(p.M), "s"(p.K), "s"(rows), "s"(p.n_lin), "s"(p.lin[0].codes),
                 "s"(p.lin[0].scales), "s"(p.lin[0].tile_begin), "s"(p.lin[1].tile_begin),
                 "s"(p.lin[2].tile_begin), "s"(p.lin[3].tile_begin));
  }
  const int K = p.K;
  const int F = K >> 10;
  const int r0 = (int)blockIdx.x * WPB + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (r0 >= rows) return false;
  int li = 0;
  if (!SWI) {
#pragma unroll
    for (int j = 1; j < 4; ++j)
      if (j < p.n_lin && r0 >= p.lin[j].tile_begin) li = j;
  }
  const int n = r0 - p.lin[li].tile_begin;
  const uint8_t* xrow[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m)
    xrow[m] = static_cast<const uint8_t*>(p.x) + (int64_t)(m < p.M ? m : p.M - 1) * p.ldx * 2;
  const int rem = K - (F << 10);
  // activations: chunk c -> 32 bytes at 2 * (c * 1024 + 16 * lane) of each row, requested
  // with the chunk's weights; tail -> 2 * TB bytes per row, first
  uint32_t xc[U][MB][8];
  constexpr int XTW = TB / 2 > 0 ? TB / 2 : 1;  // tail activation words
  uint32_t xt[MB][XTW];
  const bool tl = TB != 16 || 16 * lane < rem;
  if constexpr (TB != 0) {
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      const uint8_t* a = tl ? xrow[m] + 2 * ((F << 10) + TB * lane) : xrow[m];
#pragma unroll
      for (int e = 0; e < TB / 4; ++e) {
        const u32x2 v = *reinterpret_cast<const u32x2*>(a + 8 * e);
        xt[m][2 * e] = v[0];
        xt[m][2 * e + 1] = v[1];
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  const int8_t* wrow[P];
  float sc[P];
#pragma unroll
  for (int pl = 0; pl < P; ++pl) {
    const QrowLin& L = p.lin[SWI ? pl : li];
    wrow[pl] = L.codes + (int64_t)n * K;
    sc[pl] = L.scales[n];
  }
  int tw[P][4];
  if constexpr (TB != 0) {
#pragma unroll
    for (int pl = 0; pl < P; ++pl) {
      const int8_t* t = wrow[pl] + (F << 10);
      if constexpr (TB == 16) {
        const i32x4 v = __builtin_nontemporal_load(
            reinterpret_cast<const i32x4*>(16 * lane < rem ? t + 16 * lane : wrow[pl]));
        tw[pl][0] = v[0]; tw[pl][1] = v[1]; tw[pl][2] = v[2]; tw[pl][3] = v[3];
      } else if constexpr (TB == 12) {
        const u32x3 v = __builtin_nontemporal_load(reinterpret_cast<const u32x3*>(t + 12 * lane));
        tw[pl][0] = v[0]; tw[pl][1] = v[1]; tw[pl][2] = v[2]; tw[pl][3] = 0;
      } else if constexpr (TB == 8) {
        const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(t + 8 * lane));
        tw[pl][0] = v[0]; tw[pl][1] = v[1]; tw[pl][2] = 0; tw[pl][3] = 0;
      } else {
        const unsigned v = __builtin_nontemporal_load(reinterpret_cast<const unsigned*>(t + 4 * lane));
        tw[pl][0] = v; tw[pl][1] = 0; tw[pl][2] = 0; tw[pl][3] = 0;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  int wv[P][U][4];
  auto load_chunk = [&](int c) {
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      const uint8_t* xa = c < F ? xrow[m] + 2 * (c * 1024 + 16 * lane) : xrow[m];
      const i32x4 v0 = *reinterpret_cast<const i32x4*>(xa);
      const i32x4 v1 = *reinterpret_cast<const i32x4*>(xa + 16);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xc[c][m][e] = static_cast<uint32_t>(v0[e]);
        xc[c][m][4 + e] = static_cast<uint32_t>(v1[e]);
      }
    }
#pragma unroll
    for (int pl = 0; pl < P; ++pl) {
      const int8_t* a = c < F ? wrow[pl] + c * 1024 + 16 * lane : wrow[pl];
      const i32x4 v = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(a));
      wv[pl][c][0] = v[0]; wv[pl][c][1] = v[1]; wv[pl][c][2] = v[2]; wv[pl][c][3] = v[3];
    }
    __builtin_amdgcn_sched_barrier(0);
  };
#pragma unroll
  for (int c = 0; c < W; ++c) load_chunk(c);
  n_out = n;
  li_out = li;
#pragma unroll
  for (int pl = 0; pl < P; ++pl)
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[pl][m] = 0.f;
  if constexpr (TB != 0) {
    if (tl) {
#pragma unroll
      for (int pl = 0; pl < P; ++pl)
#pragma unroll
        for (int j = 0; j < TB / 4; ++j) {
          uint32_t a, b;
          deq_word<XT>(tw[pl][j], sc[pl], a, b);
#pragma unroll
          for (int m = 0; m < MB; ++m) acc[pl][m] = dot_word<XT>(a, b, xt[m][2 * j], xt[m][2 * j + 1], acc[pl][m]);
        }
    }
  }
#pragma unroll
  for (int c = 0; c < U; ++c) {
    if (c < F) {
#pragma unroll
      for (int pl = 0; pl < P; ++pl)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          uint32_t a, b;
          deq_word<XT>(wv[pl][c][j], sc[pl], a, b);
#pragma unroll
          for (int m = 0; m < MB; ++m)
            acc[pl][m] = dot_word<XT>(a, b, xc[c][m][2 * j], xc[c][m][2 * j + 1], acc[pl][m]);
        }
    }
    if (c + W < U) load_chunk(c + W);
  }
#pragma unroll
  for (int pl = 0; pl < P; ++pl)
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[pl][m] = wave_sum_dpp(acc[pl][m]);
  return true;
}


template <int XT, int MB, int U, int TB, bool SWI>
__device__ __forceinline__ void gemv_valu_body(const QrowParams& p, int rows, uint8_t* xs);

template <int XT, int MB, int U, int TB, bool SWI>
__global__ __launch_bounds__((kGemvWaves<XT, MB, U, SWI> * 64)) void k_gemv_valu(QrowParams p, int rows) {
  extern __shared__ __attribute__((aligned(16))) uint8_t xs[];
  gemv_valu_body<XT, MB, U, TB, SWI>(p, rows, xs);
}

// The register path with scalar arguments.  The hardware preloads the first 14 argument
// dwords into SGPRs (16 user SGPRs, 2 of them the argument segment address; the build
// asks for them with -amdgpu-kernarg-preload-count=16), so the arguments the first loads
// need come first, 8-byte ones on even dwords: activations, K, the row count, the first
// linear's rows (SwiGLU: both linears), the linears' first rows.  Same-box graph timing
// of the paired SwiGLU launch at M = 1: 6.556 us with the parameter block, 6.530 with
// scalar arguments, 6.470 preloaded.
template <int XT, int MB, int U, int TB>
__global__ __launch_bounds__((kGemvWaves<XT, MB, U, true> * 64)) void k_gemv_xg_swi(
    const void* x, int64_t ldx, int K, int rows, const int8_t* gc, const float* gs, const int8_t* uc,
    const float* us, int M, void* y, int64_t ldy) {
  QrowParams p{};
  p.x = x;
  p.ldx = ldx;
  p.M = MB == 1 ? 1 : M;
  p.K = K;
  p.n_lin = 2;
  p.lin[0] = QrowLin{gc, gs, y, ldy, rows, 0};
  p.lin[1] = QrowLin{uc, us, nullptr, 0, rows, 0};
  gemv_valu_body<XT, MB, U, TB, true>(p, rows, nullptr);
}

template <int XT, int MB, int U, int TB>
__global__ __launch_bounds__((kGemvWaves<XT, MB, U, false> * 64)) void k_gemv_xg(
    const void* x, int64_t ldx, int K, int rows, int n_lin, int t1, const int8_t* c0, const float* s0, int t2,
    int t3, int M, const int8_t* c1, const float* s1, const int8_t* c2, const float* s2, const int8_t* c3,
    const float* s3, void* y0, int64_t ldy0, void* y1, int64_t ldy1, void* y2, int64_t ldy2, void* y3,
    int64_t ldy3, int n0, int n1, int n2, int n3) {
  // the wave's linear picked here with scalar selects: the body then sees one linear and
  // indexes nothing at run time (a run-time index into the local block puts it in scratch)
  constexpr int WPB = kGemvWaves<XT, MB, U, false>;
  const int r0 = (int)blockIdx.x * WPB + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool l1 = n_lin > 1 && r0 >= t1, l2 = n_lin > 2 && r0 >= t2, l3 = n_lin > 3 && r0 >= t3;
  QrowParams p{};
  p.x = x;
  p.ldx = ldx;
  p.M = MB == 1 ? 1 : M;
  p.K = K;
  p.n_lin = 1;
  p.lin[0] = QrowLin{l3 ? c3 : l2 ? c2 : l1 ? c1 : c0, l3 ? s3 : l2 ? s2 : l1 ? s1 : s0,
                     l3 ? y3 : l2 ? y2 : l1 ? y1 : y0,   l3 ? ldy3 : l2 ? ldy2 : l1 ? ldy1 : ldy0,
                     l3 ? n3 : l2 ? n2 : l1 ? n1 : n0,   l3 ? t3 : l2 ? t2 : l1 ? t1 : 0};
  gemv_valu_body<XT, MB, U, TB, false>(p, rows, nullptr);
}

template <int XT, int MB, int U, int TB, bool SWI>
__device__ __forceinline__ void gemv_valu_body(const QrowParams& p, int rows, uint8_t* xs) {
  const int lane = threadIdx.x & 63;
  const int M = p.M;
  float acc[SWI ? 2 : 1][MB];
  int n, li;
  if constexpr (kGemvXg<XT, MB, U>) {
    if (!gemv_wave_xg<XT, MB, U, TB, SWI>(p, rows, acc, n, li)) return;
  } else {
    if (!gemv_wave_rows<XT, MB, U, TB, SWI>(p, rows, xs, acc, n, li, (int)blockIdx.x, true)) return;
  }
  if (lane != 0) return;
  const QrowLin& L = p.lin[li];
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    if (m >= M) continue;
    const int64_t yi = (int64_t)m * L.ldy + n;
    if constexpr (SWI) {
      const float gt = bf16_bits_to_f32(f32_to_bf16_bits(acc[0][m]));
      const float ut = bf16_bits_to_f32(f32_to_bf16_bits(acc[1][m]));
      const float sl = bf16_bits_to_f32(f32_to_bf16_bits(silu_f32(gt)));
      static_cast<uint16_t*>(L.y)[yi] = f32_to_bf16_bits(sl * ut);
    } else if constexpr (XT == QS_F32) {
      static_cast<float*>(L.y)[yi] = acc[0][m];
    } else if constexpr (XT == QS_BF16) {
      static_cast<uint16_t*>(L.y)[yi] = f32_to_bf16_bits(acc[0][m]);
    } else {
      static_cast<uint16_t*>(L.y)[yi] = f32_to_f16_bits(acc[0][m]);
    }
  }
}

// ----------------------------------------------------------------------------------
// head top-2 (fused_qrow_top2, dense_qstore_cuda.py:578-674, 1239-1317)
// ----------------------------------------------------------------------------------
// Order of candidates: larger value first, lower index on ties; the second is the best
// candidate other than the first.  Rows past the semantic row count never compete.
__device__ __forceinline__ bool top2_better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// Value selects rather than branches: branching on which reference to update made the
// compiler keep the four values in scratch memory, whose accesses share the vector-memory
// wait counter with the weight loads.
__device__ __forceinline__ void top2_push(float v, int i, float& v1, int& i1, float& v2, int& i2) {
  const bool b1 = top2_better(v, i, v1, i1);
  const bool b2 = top2_better(v, i, v2, i2);
  const float nv2 = b1 ? v1 : (b2 ? v : v2);
  const int ni2 = b1 ? i1 : (b2 ? i : i2);
  v1 = b1 ? v : v1;
  i1 = b1 ? i : i1;
  v2 = nv2;
  i2 = ni2;
}

// Workgroup epilogue: each wave's running first/second per activation row -> this
// workgroup's first and second, written to part_v / part_i [M][gridDim.x][2].
template <int WPB, int MB>
__device__ __forceinline__ void block_top2(const float (&v1)[MB], const int (&i1)[MB], const float (&v2)[MB],
                                           const int (&i2)[MB], int M, float* part_v, int* part_i) {
  __shared__ float tv[WPB][MB][2];
  __shared__ int ti[WPB][MB][2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (lane == 0) {
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      tv[wave][m][0] = v1[m];
      ti[wave][m][0] = i1[m];
      tv[wave][m][1] = v2[m];
      ti[wave][m][1] = i2[m];
    }
  }
  __syncthreads();
  if (tid < M && tid < MB) {
    float a1 = -INFINITY, a2 = -INFINITY;
    int b1 = INT_MAX, b2 = INT_MAX;
#pragma unroll
    for (int w = 0; w < WPB; ++w) {
      top2_push(tv[w][tid][0], ti[w][tid][0], a1, b1, a2, b2);
      top2_push(tv[w][tid][1], ti[w][tid][1], a1, b1, a2, b2);
    }
    const int64_t o = ((int64_t)tid * gridDim.x + blockIdx.x) * 2;
    part_v[o] = a1;
    part_i[o] = b1;
    part_v[o + 1] = a2;
    part_i[o + 1] = b2;
  }
}

// Fused W8A16 / fp32 head GEMV + top-2: the decode GEMV's row work (one wave per row of
// the semantic prefix), no logits written.  Persistent: workgroup g takes the 8-row
// blocks g, g + G, ... (G = gridDim.x), stages the activations once and keeps each
// wave's running first/second in registers.
template <int XT, int MB, int U, int TB>
__global__ __launch_bounds__((GemvShape<false, MB>::waves * 64)) void k_gemv_top2(QrowParams p, int rows,
                                                                                   int start_row, float* part_v,
                                                                                   int* part_i) {
  extern __shared__ __attribute__((aligned(16))) uint8_t xs[];
  constexpr int WPB = GemvShape<false, MB>::waves;
  const int nblk = (rows + WPB - 1) / WPB;
  float v1[MB], v2[MB];
  int i1[MB], i2[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    v1[m] = v2[m] = -INFINITY;
    i1[m] = i2[m] = INT_MAX;
  }
  bool stage = true;
  for (int blk = blockIdx.x; blk < nblk; blk += gridDim.x) {
    float acc[1][MB];
    int n, li;
    if (gemv_wave_rows<XT, MB, U, TB, false>(p, rows, xs, acc, n, li, blk, stage)) {
#pragma unroll
      for (int m = 0; m < MB; ++m) top2_push(acc[0][m], start_row + n, v1[m], i1[m], v2[m], i2[m]);
    }
    stage = false;
  }
  block_top2<WPB, MB>(v1, i1, v2, i2, p.M, part_v, part_i);
}

// The same launch for MB = 1 or 2 bf16/f16 activation rows and K / 1024 = U (1 or 2) full
// chunks: each wave loads the activations of its own weight bytes into registers once
// (as gemv_wave_xg does per row) and walks its rows blk * 8 + wave, blk = g, g + G, ...
// with the next row's weights in flight while the current row is reduced.  Every load is
// unconditional (a row past the end re-reads the wave's current row; activation rows
// m >= M read row M - 1), so the waits stay per buffer.  Same products, order, wave sum
// and candidates as k_gemv_top2.
template <int XT, int MB, int U, int TB>
__global__ __launch_bounds__(512) void k_gemv_top2_xg(QrowParams p, int rows, int start_row, float* part_v,
                                                      int* part_i) {
  constexpr int WPB = 8;
  static_assert(U <= 2, "register activations cover at most two chunks");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int K = p.K;
  constexpr int F = U;  // full chunks (the host checks K >> 10 == U)
  const int rem = K - (F << 10);
  uint32_t xc[U][MB][8];
  constexpr int XTW = TB / 2 > 0 ? TB / 2 : 1;
  uint32_t xt[MB][XTW];
  const bool tl = TB != 16 || 16 * lane < rem;
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    const uint8_t* xg = static_cast<const uint8_t*>(p.x) + (int64_t)(m < p.M ? m : p.M - 1) * p.ldx * 2;
#pragma unroll
    for (int c = 0; c < U; ++c) {
      const uint8_t* a = xg + 2 * (c * 1024 + 16 * lane);
      const i32x4 v0 = *reinterpret_cast<const i32x4*>(a);
      const i32x4 v1 = *reinterpret_cast<const i32x4*>(a + 16);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xc[c][m][e] = static_cast<uint32_t>(v0[e]);
        xc[c][m][4 + e] = static_cast<uint32_t>(v1[e]);
      }
    }
    if constexpr (TB != 0) {
      const uint8_t* a = tl ? xg + 2 * ((F << 10) + TB * lane) : xg;
#pragma unroll
      for (int e = 0; e < TB / 4; ++e) {
        const u32x2 v = *reinterpret_cast<const u32x2*>(a + 8 * e);
        xt[m][2 * e] = v[0];
        xt[m][2 * e + 1] = v[1];
      }
    }
  }
  const int8_t* codes = p.lin[0].codes;
  const float* scales = p.lin[0].scales;
  int tw[2][4], wv[2][U][4];
  float sc[2];
  auto load = [&](int b, int row) {
    const int8_t* wrow = codes + (int64_t)row * K;
    sc[b] = scales[row];
    if constexpr (TB != 0) {
      const int8_t* t = wrow + (F << 10);
      if constexpr (TB == 16) {
        const i32x4 v = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(tl ? t + 16 * lane : wrow));
        tw[b][0] = v[0]; tw[b][1] = v[1]; tw[b][2] = v[2]; tw[b][3] = v[3];
      } else if constexpr (TB == 12) {
        const u32x3 v = __builtin_nontemporal_load(reinterpret_cast<const u32x3*>(t + 12 * lane));
        tw[b][0] = v[0]; tw[b][1] = v[1]; tw[b][2] = v[2]; tw[b][3] = 0;
      } else if constexpr (TB == 8) {
        const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(t + 8 * lane));
        tw[b][0] = v[0]; tw[b][1] = v[1]; tw[b][2] = 0; tw[b][3] = 0;
      } else {
        const unsigned v = __builtin_nontemporal_load(reinterpret_cast<const unsigned*>(t + 4 * lane));
        tw[b][0] = v; tw[b][1] = 0; tw[b][2] = 0; tw[b][3] = 0;
      }
    }
#pragma unroll
    for (int c = 0; c < U; ++c) {
      const i32x4 v = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(wrow + c * 1024 + 16 * lane));
      wv[b][c][0] = v[0]; wv[b][c][1] = v[1]; wv[b][c][2] = v[2]; wv[b][c][3] = v[3];
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  float v1[MB], v2[MB];
  int i1[MB], i2[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    v1[m] = v2[m] = -INFINITY;
    i1[m] = i2[m] = INT_MAX;
  }
  auto reduce = [&](int b, int row) {
    float acc[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[m] = 0.f;
    if constexpr (TB != 0) {
      if (tl) {
#pragma unroll
        for (int j = 0; j < TB / 4; ++j) {
          uint32_t a, c2;
          deq_word<XT>(tw[b][j], sc[b], a, c2);
#pragma unroll
          for (int m = 0; m < MB; ++m) acc[m] = dot_word<XT>(a, c2, xt[m][2 * j], xt[m][2 * j + 1], acc[m]);
        }
      }
    }
#pragma unroll
    for (int c = 0; c < U; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t a, c2;
        deq_word<XT>(wv[b][c][j], sc[b], a, c2);
#pragma unroll
        for (int m = 0; m < MB; ++m) acc[m] = dot_word<XT>(a, c2, xc[c][m][2 * j], xc[c][m][2 * j + 1], acc[m]);
      }
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      acc[m] = wave_sum_dpp(acc[m]);
      if (row < rows) top2_push(acc[m], start_row + row, v1[m], i1[m], v2[m], i2[m]);
    }
  };
  const int stride = (int)gridDim.x * WPB;
  int r = (int)blockIdx.x * WPB + wave;
  load(0, r < rows ? r : rows - 1);
  for (; r < rows; r += 2 * stride) {
    load(1, r + stride < rows ? r + stride : r);
    reduce(0, r);
    load(0, r + 2 * stride < rows ? r + 2 * stride : r);
    reduce(1, r + stride);
  }
  block_top2<WPB, MB>(v1, i1, v2, i2, p.M, part_v, part_i);
}

// Any K / alignment: one wave per row, one activation row per launch (x points at it),
// the same arithmetic contract as k_generic.
__global__ __launch_bounds__(256) void k_generic_top2(QrowParams p, int x_dtype, int rows, int start_row,
                                                      float* part_v, int* part_i) {
  const int lane = threadIdx.x & 63;
  const int n = (int)(blockIdx.x * 4 + (threadIdx.x >> 6));
  const bool has = n < rows;
  const int8_t* w = p.lin[0].codes + (int64_t)(has ? n : 0) * p.K;
  const float s = p.lin[0].scales[has ? n : 0];
  float acc = 0.f;
  for (int k = lane; k < p.K; k += 64) {
    float wf = static_cast<float>(w[k]) * s;
    float xf;
    if (x_dtype == QS_F32) {
      xf = static_cast<const float*>(p.x)[k];
    } else if (x_dtype == QS_BF16) {
      wf = bf16_bits_to_f32(f32_to_bf16_bits(wf));
      xf = bf16_bits_to_f32(static_cast<const uint16_t*>(p.x)[k]);
    } else {
      wf = f16_bits_to_f32(f32_to_f16_bits(wf));
      xf = f16_bits_to_f32(static_cast<const uint16_t*>(p.x)[k]);
    }
    acc = fmaf(xf, wf, acc);
  }
  float v1[1] = {has ? wave_sum_dpp(acc) : -INFINITY}, v2[1] = {-INFINITY};
  int i1[1] = {has ? start_row + n : INT_MAX}, i2[1] = {INT_MAX};
  block_top2<4, 1>(v1, i1, v2, i2, 1, part_v, part_i);
}

// Candidates [M][C] of the blocks -> first and second per row.
__global__ __launch_bounds__(256) void k_top2_reduce(const float* __restrict__ part_v,
                                                     const int* __restrict__ part_i, int C,
                                                     int* __restrict__ out_i, float* __restrict__ out_v) {
  // Partials come from the previous launch, so every read misses the cache: all U loads
  // of a round are issued before any is merged.  (-inf, INT_MAX) pads are no-ops.
  constexpr int U = 8;
  __shared__ float sv[4][2];
  __shared__ int si[4][2];
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* pv = part_v + (int64_t)m * C;
  const int* pi = part_i + (int64_t)m * C;
  float v1 = -INFINITY, v2 = -INFINITY;
  int i1 = INT_MAX, i2 = INT_MAX;
  for (int c0 = tid; c0 < C; c0 += 256 * U) {
    float v[U];
    int ix[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + 256 * u;
      v[u] = c < C ? pv[c] : -INFINITY;
      ix[u] = c < C ? pi[c] : INT_MAX;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) top2_push(v[u], ix[u], v1, i1, v2, i2);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float o1 = __shfl_xor(v1, off), o2 = __shfl_xor(v2, off);
    const int j1 = __shfl_xor(i1, off), j2 = __shfl_xor(i2, off);
    top2_push(o1, j1, v1, i1, v2, i2);
    top2_push(o2, j2, v1, i1, v2, i2);
  }
  if (lane == 0) {
    sv[wave][0] = v1;
    si[wave][0] = i1;
    sv[wave][1] = v2;
    si[wave][1] = i2;
  }
  __syncthreads();
  if (tid == 0) {
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      top2_push(sv[w][0], si[w][0], v1, i1, v2, i2);
      top2_push(sv[w][1], si[w][1], v1, i1, v2, i2);
    }
    out_v[2 * m] = v1;
    out_i[2 * m] = i1;
    out_v[2 * m + 1] = v2;
    out_i[2 * m + 1] = i2;
  }
}

// FP32 candidate rerank (_rerank_qrow_candidates_fp32, dense_qstore_cuda.py:1189-1236):
// score = sum_k float(x[k]) * (float(code[k]) * scale), fp32; best score wins, lower
// index on ties.  Wave c of workgroup m scores candidate c of row m.
__global__ __launch_bounds__(1024) void k_rerank_fp32(const void* __restrict__ x, int x_dtype, int64_t ldx,
                                                      const int8_t* __restrict__ codes,
                                                      const float* __restrict__ scales, int page_rows, int K,
                                                      int64_t start_row, const int64_t* __restrict__ cand, int C,
                                                      int64_t* __restrict__ out_i, float* __restrict__ out_v) {
  __shared__ float sv[16];
  __shared__ int64_t si[16];
  const int m = blockIdx.x, lane = threadIdx.x & 63, c = threadIdx.x >> 6;
  const int64_t idx = cand[(int64_t)m * C + c];
  const int64_t local = idx - start_row;
  const bool ok = local >= 0 && local < page_rows;
  const int8_t* w = codes + (ok ? local : 0) * (int64_t)K;
  const float s = scales[ok ? local : 0];
  float acc = 0.f;
  for (int k = lane; k < K; k += 64) {
    float xf;
    if (x_dtype == QS_F32) xf = static_cast<const float*>(x)[(int64_t)m * ldx + k];
    else if (x_dtype == QS_BF16) xf = bf16_bits_to_f32(static_cast<const uint16_t*>(x)[(int64_t)m * ldx + k]);
    else xf = f16_bits_to_f32(static_cast<const uint16_t*>(x)[(int64_t)m * ldx + k]);
    acc = fmaf(xf, static_cast<float>(w[k]) * s, acc);
  }
  acc = wave_sum_dpp(acc);
  if (lane == 0) {
    sv[c] = ok ? acc : -INFINITY;
    si[c] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float bv = sv[0];
    int64_t bi = si[0];
    for (int j = 1; j < C; ++j)
      if (sv[j] > bv || (sv[j] == bv && si[j] < bi)) {
        bv = sv[j];
        bi = si[j];
      }
    out_v[m] = bv;
    out_i[m] = bi;
  }
}

// ----------------------------------------------------------------------------------
// generic fallback: any K, any alignment.  One wave per (linear, row).
// ----------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_generic(QrowParams p, int x_dtype) {
  const int lane = threadIdx.x & 63;
  const int gw = (int)(blockIdx.x * 4 + (threadIdx.x >> 6));
  int li = 0;
#pragma unroll
  for (int j = 1; j < 4; ++j)
    if (j < p.n_lin && gw >= p.lin[j].tile_begin) li = j;
  const QrowLin& L = p.lin[li];
  const int n = gw - L.tile_begin;
  if (n >= L.N) return;
  const int8_t* w = L.codes + (int64_t)n * p.K;
  const float s = L.scales[n];
  for (int m = 0; m < p.M; ++m) {
    float acc = 0.f;
    for (int k = lane; k < p.K; k += 64) {
      float wf = static_cast<float>(w[k]) * s;
      float xf;
      const int64_t xi = (int64_t)m * p.ldx + k;
      if (x_dtype == QS_F32) {
        xf = static_cast<const float*>(p.x)[xi];
      } else if (x_dtype == QS_BF16) {
        wf = bf16_bits_to_f32(f32_to_bf16_bits(wf));
        xf = bf16_bits_to_f32(static_cast<const uint16_t*>(p.x)[xi]);
      } else {
        wf = f16_bits_to_f32(f32_to_f16_bits(wf));
        xf = f16_bits_to_f32(static_cast<const uint16_t*>(p.x)[xi]);
      }
      acc = fmaf(xf, wf, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) {
      const int64_t yi = (int64_t)m * L.ldy + n;
      if (x_dtype == QS_F32)
        static_cast<float*>(L.y)[yi] = acc;
      else if (x_dtype == QS_BF16)
        static_cast<uint16_t*>(L.y)[yi] = f32_to_bf16_bits(acc);
      else
        static_cast<uint16_t*>(L.y)[yi] = f32_to_f16_bits(acc);
    }
  }
}

// generic SwiGLU fallback (bf16): one wave per output column n.
__global__ __launch_bounds__(256) void k_generic_swiglu(QrowParams p) {
  const int lane = threadIdx.x & 63;
  const int n = (int)(blockIdx.x * 4 + (threadIdx.x >> 6));
  if (n >= p.lin[0].N) return;
  const int8_t* wg = p.lin[0].codes + (int64_t)n * p.K;
  const int8_t* wu = p.lin[1].codes + (int64_t)n * p.K;
  const float sg = p.lin[0].scales[n], su = p.lin[1].scales[n];
  const uint16_t* x = static_cast<const uint16_t*>(p.x);
  for (int m = 0; m < p.M; ++m) {
    float ag = 0.f, au = 0.f;
    for (int k = lane; k < p.K; k += 64) {
      const float xf = bf16_bits_to_f32(x[(int64_t)m * p.ldx + k]);
      ag = fmaf(xf, bf16_bits_to_f32(f32_to_bf16_bits(static_cast<float>(wg[k]) * sg)), ag);
      au = fmaf(xf, bf16_bits_to_f32(f32_to_bf16_bits(static_cast<float>(wu[k]) * su)), au);
    }
    ag = wave_sum(ag);
    au = wave_sum(au);
    if (lane == 0) {
      const float gt = bf16_bits_to_f32(f32_to_bf16_bits(ag));
      const float ut = bf16_bits_to_f32(f32_to_bf16_bits(au));
      const float sl = bf16_bits_to_f32(f32_to_bf16_bits(silu_f32(gt)));
      static_cast<uint16_t*>(p.lin[0].y)[(int64_t)m * p.lin[0].ldy + n] =
          f32_to_bf16_bits(sl * ut);
    }
  }
}

// ----------------------------------------------------------------------------------
// host launchers
// ----------------------------------------------------------------------------------
namespace {

// K-split (waves per plane) chosen from (N, K) only -- never from M -- so the
// accumulation order of a row does not depend on the batch.  Aim for ~16 waves per CU
// over 256 CUs and at most 8 chunks per wave per round.
int pick_kw(int64_t N, int64_t K) {
  const int64_t tiles = cdiv(N, 16);
  const int64_t chunks = K / 128;
  int w = 4;
  while (w < 16 && (tiles * w < 4096 || chunks > (int64_t)w * 4)) w *= 2;
  return w;
}

// Streaming kernel: K slices per tile from (tiles, K) only, for about 2048 waves per
// launch while every slice keeps at least four 128-k chunks (two for launches of fewer
// than 1024 waves).  Two-plane (SwiGLU) waves hold more registers, so their workgroups
// stop at 8 waves.
int pick_kw_s(int64_t tiles, int64_t K, int P) {
  const int64_t chunks = K / 128;
  const int cap = P == 2 ? 8 : 16;
  int w = 1;
  while (w < cap && tiles * w < 2048 && (int64_t)4 * w <= chunks) w *= 2;
  if (w < cap && tiles * w < 1024 && (int64_t)2 * w <= chunks) w *= 2;
  return w;
}

// The streaming kernel addresses every operand with 31-bit buffer offsets.
bool stream_fits(const QrowParams& q) {
  if ((int64_t)q.M * q.ldx * 2 >= INT_MAX) return false;
  for (int i = 0; i < q.n_lin; ++i)
    if ((int64_t)q.lin[i].N * q.K >= INT_MAX) return false;
  return true;
}

// LDS bytes for the activations of the streaming kernel, 0 when they are read from
// L2: a copy per workgroup pays off while it is small next to the workgroup's weights --
// up to 25 KB (M <= 8 rows of a 1536-wide layer), or up to 144 KB when the launch has
// at most one workgroup per CU anyway (few, long tiles such as 1536 x 8960).
size_t stream_xl_bytes(const QrowParams& q, int blocks) {
  const size_t b = (size_t)q.M * (size_t)(2 * q.K + 16);
  if (b <= 25 * 1024) return b;
  if (blocks <= 256 && b <= 144 * 1024) return b;
  return 0;
}

// Returns false (nothing launched) for a plain linear whose activations do not go to LDS.
// The window holds two chunks: a deeper one (4) measured 8-15% slower, its extra
// registers costing a wave per SIMD.
template <int P, int MT, int KW, bool F16>
bool launch_w8a16_s_kw(const QrowParams& p, int blocks, hipStream_t s) {
  const size_t xl = stream_xl_bytes(p, blocks);
  if (xl) {
    hipLaunchKernelGGL((k_w8a16_s<P, MT, KW, 2, F16, true>), dim3(blocks), dim3(KW * 64), xl, s, p);
    return true;
  }
  if constexpr (P == 2) {  // plain linears take the streaming kernel only with LDS activations
    hipLaunchKernelGGL((k_w8a16_s<P, MT, KW, 2, F16, false>), dim3(blocks), dim3(KW * 64), 0, s, p);
    return true;
  }
  return false;
}

template <int P, int MT, bool F16>
bool launch_w8a16_s(const QrowParams& p, int blocks, int kw, hipStream_t s) {
  if (kw == 1) return launch_w8a16_s_kw<P, MT, 1, F16>(p, blocks, s);
  if (kw == 2) return launch_w8a16_s_kw<P, MT, 2, F16>(p, blocks, s);
  if (kw == 4) return launch_w8a16_s_kw<P, MT, 4, F16>(p, blocks, s);
  if (kw == 8) return launch_w8a16_s_kw<P, MT, 8, F16>(p, blocks, s);
  if constexpr (P == 1) return launch_w8a16_s_kw<P, MT, 16, F16>(p, blocks, s);
  return false;
}

template <int P, int MT, int KW, bool F16>
void launch_w8a16_kw(const QrowParams& p, int blocks, hipStream_t s) {
  const int u = (int)cdiv(p.K / 128, KW);
  // two activation tiles double the live activation registers: keep U at 2
  if constexpr (MT == 2) {
    hipLaunchKernelGGL((k_w8a16<P, MT, KW, 2, F16>), dim3(blocks), dim3(P * KW * 64), 0, s, p);
  } else {
    if (u <= 2)
      hipLaunchKernelGGL((k_w8a16<P, MT, KW, 2, F16>), dim3(blocks), dim3(P * KW * 64), 0, s, p);
    else
      hipLaunchKernelGGL((k_w8a16<P, MT, KW, 4, F16>), dim3(blocks), dim3(P * KW * 64), 0, s, p);
  }
}

template <int P, int MT, bool F16>
void launch_w8a16(const QrowParams& p, int blocks, int kw, hipStream_t s) {
  if (kw == 4) {
    launch_w8a16_kw<P, MT, 4, F16>(p, blocks, s);
  } else if (kw == 8) {
    launch_w8a16_kw<P, MT, 8, F16>(p, blocks, s);
  } else {
    if constexpr (P == 1)
      launch_w8a16_kw<P, MT, 16, F16>(p, blocks, s);
    else
      launch_w8a16_kw<P, MT, 8, F16>(p, blocks, s);  // 2 planes x 8 = 1024 threads
  }
}

bool mfma_eligible(const QrowParams& p, int x_dtype) {
  if (x_dtype != QS_BF16 && x_dtype != QS_F16) return false;
  if (p.K % 128 != 0 || p.ldx % 8 != 0 || !aligned(p.x, 16)) return false;
  for (int i = 0; i < p.n_lin; ++i)
    if (!aligned(p.lin[i].codes, 16)) return false;
  return true;
}

int validate_common(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K) {
  if (!x) return fail(QS_ERR_INVALID, "activation pointer is null");
  if (x_dtype != QS_F32 && x_dtype != QS_BF16 && x_dtype != QS_F16)
    return fail(QS_ERR_INVALID, "activation dtype must be F32, BF16 or F16");
  if (M < 0 || K <= 0) return fail(QS_ERR_INVALID, "invalid M=%lld K=%lld", (long long)M, (long long)K);
  if (ldx < K) return fail(QS_ERR_INVALID, "ldx (%lld) < K (%lld)", (long long)ldx, (long long)K);
  if (K > (int64_t)1 << 30 || M > (int64_t)1 << 30)
    return fail(QS_ERR_LIMIT, "dimension exceeds 2^30");
  return QS_OK;
}

constexpr int kLdsBudget = 64 * 1024;

// Activation rows per VALU launch: the largest of 4/2/1 whose LDS copy fits.
int valu_mb(int x_dtype, int64_t K, int64_t M) {
  const int es = x_dtype == QS_F32 ? 4 : 2;
  const int cap = x_dtype == QS_F32 ? 4 : 2;
  for (int mb = cap; mb >= 1; mb /= 2)
    if ((int64_t)mb * K * es <= kLdsBudget && (mb <= M || mb == 1)) return mb;
  return 0;
}

bool valu_eligible(const QrowParams& p, int x_dtype) {
  const int es = x_dtype == QS_F32 ? 4 : 2;
  if (p.K % 16 != 0 || (p.ldx * es) % 16 != 0 || !aligned(p.x, 16)) return false;
  if ((int64_t)p.K * es > kLdsBudget || p.K > 12 * 1024) return false;
  for (int i = 0; i < p.n_lin; ++i)
    if (!aligned(p.lin[i].codes, 16)) return false;
  return true;
}

// Tail kind of a K: 0 (K % 1024 == 0), 4/8/12 bytes per lane (K % 256 == 0), else 16.
int gemv_tail(int64_t K) {
  const int64_t rem = K % 1024;
  if (rem == 0) return 0;
  if (rem % 256 == 0) return (int)(rem / 64);
  return 16;
}

template <int XT, int MB, int U, int TB, bool SWI>
void launch_valu_u(const QrowParams& q, int rows, size_t lds, hipStream_t s) {
  constexpr int WPB = kGemvWaves<XT, MB, U, SWI>;
  const dim3 grid((unsigned)cdiv(rows, WPB)), block(WPB * 64);
  if constexpr (kGemvXg<XT, MB, U>) {  // no LDS activations on the register path
    const QrowLin* L = q.lin;
    if constexpr (SWI)
      hipLaunchKernelGGL((k_gemv_xg_swi<XT, MB, U, TB>), grid, block, 0, s, q.x, q.ldx, q.K, rows, L[0].codes,
                         L[0].scales, L[1].codes, L[1].scales, q.M, L[0].y, L[0].ldy);
    else
      hipLaunchKernelGGL((k_gemv_xg<XT, MB, U, TB>), grid, block, 0, s, q.x, q.ldx, q.K, rows, q.n_lin,
                         L[1].tile_begin, L[0].codes, L[0].scales, L[2].tile_begin, L[3].tile_begin, q.M, L[1].codes,
                         L[1].scales, L[2].codes, L[2].scales, L[3].codes, L[3].scales, L[0].y, L[0].ldy, L[1].y,
                         L[1].ldy, L[2].y, L[2].ldy, L[3].y, L[3].ldy, L[0].N, L[1].N, L[2].N, L[3].N);
  } else {
    hipLaunchKernelGGL((k_gemv_valu<XT, MB, U, TB, SWI>), grid, block, lds, s, q, rows);
  }
}

template <int XT, int MB, int TB, bool SWI>
void launch_valu_tb(const QrowParams& q, int rows, size_t lds, hipStream_t s) {
  const int F = q.K >> 10;
  if (F <= 1) launch_valu_u<XT, MB, 1, TB, SWI>(q, rows, lds, s);
  else if (F <= 2) launch_valu_u<XT, MB, 2, TB, SWI>(q, rows, lds, s);
  else if (F <= 4) launch_valu_u<XT, MB, 4, TB, SWI>(q, rows, lds, s);
  else if (F <= 8) launch_valu_u<XT, MB, 8, TB, SWI>(q, rows, lds, s);
  else launch_valu_u<XT, MB, 12, TB, SWI>(q, rows, lds, s);
}

template <int XT, int MB, bool SWI>
void launch_valu_mb(const QrowParams& q, int rows, size_t lds, hipStream_t s) {
  switch (gemv_tail(q.K)) {
    case 0: launch_valu_tb<XT, MB, 0, SWI>(q, rows, lds, s); break;
    case 4: launch_valu_tb<XT, MB, 4, SWI>(q, rows, lds, s); break;
    case 8: launch_valu_tb<XT, MB, 8, SWI>(q, rows, lds, s); break;
    case 12: launch_valu_tb<XT, MB, 12, SWI>(q, rows, lds, s); break;
    default: launch_valu_tb<XT, MB, 16, SWI>(q, rows, lds, s); break;
  }
}

// Activation rows up to which bf16/f16 calls take the VALU (register-activation) kernel
// rather than the MFMA tiles: the weights are read once either way, and at M <= 4 the
// VALU dot work still hides under the weight stream.
#ifndef QS_VALU_ROWS
#define QS_VALU_ROWS 4
#endif
constexpr int64_t kValuRows = QS_VALU_ROWS;

// VALU path: rows of x in batches of MB (each batch one launch).  Every row is reduced
// in the same order whatever M is.
int run_valu(QrowParams p, int x_dtype, int64_t M, hipStream_t s, bool swiglu) {
  const int es = x_dtype == QS_F32 ? 4 : 2;
  // bf16/f16 rows take the register-activation kernel in batches of up to 4
  const int mb = x_dtype == QS_F32 ? valu_mb(x_dtype, p.K, M) : (M <= 1 ? 1 : M <= 2 ? 2 : 4);
  int rows = 0;
  if (swiglu) {
    rows = p.lin[0].N;
  } else {
    for (int i = 0; i < p.n_lin; ++i) {
      p.lin[i].tile_begin = rows;
      rows += p.lin[i].N;
    }
  }
  for (int64_t m0 = 0; m0 < M; m0 += mb) {
    QrowParams q = p;
    q.M = (int)((M - m0) < mb ? (M - m0) : mb);
    q.x = static_cast<const char*>(p.x) + m0 * p.ldx * es;
    for (int i = 0; i < q.n_lin; ++i)
      if (p.lin[i].y) q.lin[i].y = static_cast<char*>(p.lin[i].y) + m0 * p.lin[i].ldy * es;
    const size_t lds = (size_t)q.M * q.K * es;
    if (swiglu) {
      if (mb == 4) launch_valu_mb<QS_BF16, 4, true>(q, rows, lds, s);
      else if (mb == 2) launch_valu_mb<QS_BF16, 2, true>(q, rows, lds, s);
      else launch_valu_mb<QS_BF16, 1, true>(q, rows, lds, s);
    } else if (x_dtype == QS_F32) {
      if (mb == 4) launch_valu_mb<QS_F32, 4, false>(q, rows, lds, s);
      else if (mb == 2) launch_valu_mb<QS_F32, 2, false>(q, rows, lds, s);
      else launch_valu_mb<QS_F32, 1, false>(q, rows, lds, s);
    } else if (x_dtype == QS_BF16) {
      if (mb == 4) launch_valu_mb<QS_BF16, 4, false>(q, rows, lds, s);
      else if (mb == 2) launch_valu_mb<QS_BF16, 2, false>(q, rows, lds, s);
      else launch_valu_mb<QS_BF16, 1, false>(q, rows, lds, s);
    } else {
      if (mb == 4) launch_valu_mb<QS_F16, 4, false>(q, rows, lds, s);
      else if (mb == 2) launch_valu_mb<QS_F16, 2, false>(q, rows, lds, s);
      else launch_valu_mb<QS_F16, 1, false>(q, rows, lds, s);
    }
  }
  return hip_check(hipGetLastError(), "k_gemv_valu launch");
}

// Workgroups of the persistent top-2 launch: 4 resident 8-wave workgroups per CU.
constexpr int kTop2Grid = 1024;
int top2_grid(int rows) {
  const int nblk = (int)cdiv(rows, GemvShape<false, 1>::waves);
  return nblk < kTop2Grid ? nblk : kTop2Grid;
}

template <int XT, int MB, int TB>
void launch_top2_tb(const QrowParams& q, int rows, int start_row, float* pv, int* pi, size_t lds,
                    hipStream_t s) {
  constexpr int WPB = GemvShape<false, MB>::waves;
  static_assert(GemvShape<false, 1>::waves == 8, "k_gemv_top2_xg takes the 8-row blocks of top2_grid");
  const dim3 grid((unsigned)top2_grid(rows)), block(WPB * 64);
  const int F = q.K >> 10;
  if constexpr (MB <= 2 && XT != QS_F32) {  // one or two bf16/f16 rows: register activations
    if (F == 1) {
      hipLaunchKernelGGL((k_gemv_top2_xg<XT, MB, 1, TB>), grid, block, 0, s, q, rows, start_row, pv, pi);
      return;
    }
    if (F == 2) {
      hipLaunchKernelGGL((k_gemv_top2_xg<XT, MB, 2, TB>), grid, block, 0, s, q, rows, start_row, pv, pi);
      return;
    }
  }
  if (F <= 1)
    hipLaunchKernelGGL((k_gemv_top2<XT, MB, 1, TB>), grid, block, lds, s, q, rows, start_row, pv, pi);
  else if (F <= 2)
    hipLaunchKernelGGL((k_gemv_top2<XT, MB, 2, TB>), grid, block, lds, s, q, rows, start_row, pv, pi);
  else if (F <= 4)
    hipLaunchKernelGGL((k_gemv_top2<XT, MB, 4, TB>), grid, block, lds, s, q, rows, start_row, pv, pi);
  else if (F <= 8)
    hipLaunchKernelGGL((k_gemv_top2<XT, MB, 8, TB>), grid, block, lds, s, q, rows, start_row, pv, pi);
  else
    hipLaunchKernelGGL((k_gemv_top2<XT, MB, 12, TB>), grid, block, lds, s, q, rows, start_row, pv, pi);
}

template <int XT, int MB>
void launch_top2_mb(const QrowParams& q, int rows, int start_row, float* pv, int* pi, size_t lds,
                    hipStream_t s) {
  switch (gemv_tail(q.K)) {
    case 0: launch_top2_tb<XT, MB, 0>(q, rows, start_row, pv, pi, lds, s); break;
    case 4: launch_top2_tb<XT, MB, 4>(q, rows, start_row, pv, pi, lds, s); break;
    case 8: launch_top2_tb<XT, MB, 8>(q, rows, start_row, pv, pi, lds, s); break;
    case 12: launch_top2_tb<XT, MB, 12>(q, rows, start_row, pv, pi, lds, s); break;
    default: launch_top2_tb<XT, MB, 16>(q, rows, start_row, pv, pi, lds, s); break;
  }
}

// Candidate blocks of the head top-2 for `rows` semantic rows (the generic path's 4-row
// blocks; the fused path uses 8-row blocks, so this bounds both).
int64_t top2_blocks(int64_t rows) { return cdiv(rows, 4); }

// Runs one set of linears sharing x, M <= 32 rows at a time for the MFMA path.
int run_linears(QrowParams p, int x_dtype, int64_t M, hipStream_t s, bool row_stable) {
  if (M == 0) return QS_OK;
  const int esz = x_dtype == QS_F32 ? 4 : 2;
  // decode-sized batches (and the row-stable contract) take the VALU path
  if ((row_stable || M <= kValuRows || x_dtype == QS_F32) && valu_eligible(p, x_dtype))
    return run_valu(p, x_dtype, M, s, false);
  if (!row_stable && mfma_eligible(p, x_dtype)) {
    for (int64_t m0 = 0; m0 < M; m0 += 32) {
      QrowParams q = p;
      const int mm = (int)((M - m0) < 32 ? (M - m0) : 32);
      q.M = mm;
      q.x = static_cast<const char*>(p.x) + m0 * p.ldx * esz;
      int blocks = 0;
      int64_t nmax = 0;
      for (int i = 0; i < q.n_lin; ++i) {
        q.lin[i].y = static_cast<char*>(p.lin[i].y) + m0 * p.lin[i].ldy * 2;
        q.lin[i].tile_begin = blocks;
        blocks += (int)cdiv(q.lin[i].N, 16);
        nmax = q.lin[i].N > nmax ? q.lin[i].N : nmax;
      }
      const bool f16 = x_dtype == QS_F16;
      // long rows with LDS-resident activations stream (few tiles, deep K); the rest
      // keep the round-based kernel, which measured faster for 1536-wide layers
      if (q.K >= 4096 && stream_fits(q) && stream_xl_bytes(q, blocks)) {
        const int kw = pick_kw_s(blocks, q.K, 1);
        bool done;
        if (mm <= 16)
          done = f16 ? launch_w8a16_s<1, 1, true>(q, blocks, kw, s) : launch_w8a16_s<1, 1, false>(q, blocks, kw, s);
        else
          done = f16 ? launch_w8a16_s<1, 2, true>(q, blocks, kw, s) : launch_w8a16_s<1, 2, false>(q, blocks, kw, s);
        if (done) continue;
      }
      const int kw = pick_kw(nmax, q.K);
      if (mm <= 16)
        f16 ? launch_w8a16<1, 1, true>(q, blocks, kw, s) : launch_w8a16<1, 1, false>(q, blocks, kw, s);
      else
        f16 ? launch_w8a16<1, 2, true>(q, blocks, kw, s) : launch_w8a16<1, 2, false>(q, blocks, kw, s);
    }
    return hip_check(hipGetLastError(), "k_w8a16 launch");
  }
  if (valu_eligible(p, x_dtype)) return run_valu(p, x_dtype, M, s, false);
  int waves = 0;
  for (int i = 0; i < p.n_lin; ++i) {
    p.lin[i].tile_begin = waves;
    waves += p.lin[i].N;
  }
  p.M = (int)M;
  hipLaunchKernelGGL(k_generic, dim3((unsigned)cdiv(waves, 4)), dim3(256), 0, s, p, x_dtype);
  return hip_check(hipGetLastError(), "k_generic launch");
}

}  // namespace
}  // namespace qs

using namespace qs;

extern "C" int qs_qrow_dequant(const int8_t* codes, const float* scales, void* out, int out_dtype,
                               int64_t N, int64_t K, int64_t ld_out, void* stream) {
  if (!codes || !scales || !out) return fail(QS_ERR_INVALID, "dequant: null pointer");
  if (N < 0 || K <= 0 || ld_out < K) return fail(QS_ERR_INVALID, "dequant: bad shape");
  if (out_dtype != QS_F32 && out_dtype != QS_BF16 && out_dtype != QS_F16)
    return fail(QS_ERR_INVALID, "dequant: out dtype must be F32, BF16 or F16");
  if (N == 0) return QS_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int osz = out_dtype == QS_F32 ? 4 : 2;
  // per-row pieces must fit the 32-bit column arithmetic of k_dequant_v
  const bool fast = K % 16 == 0 && aligned(codes, 16) && aligned(out, 16) && (ld_out * osz) % 16 == 0 &&
                    K <= (int64_t(1) << 33);
  if (fast) {
    constexpr int U = kDequantPieces;
    const int64_t work = N * (K / (out_dtype == QS_F32 ? 4 : 8));
    const int64_t chunks = cdiv(work, 256 * U);
    const unsigned blocks = (unsigned)(chunks < 65536 ? chunks : 65536);
    if (out_dtype == QS_F32)
      hipLaunchKernelGGL((k_dequant_v<QS_F32, U>), dim3(blocks), dim3(256), 0, s, codes, scales, out, N, K, ld_out);
    else if (out_dtype == QS_BF16)
      hipLaunchKernelGGL((k_dequant_v<QS_BF16, U>), dim3(blocks), dim3(256), 0, s, codes, scales, out, N, K, ld_out);
    else
      hipLaunchKernelGGL((k_dequant_v<QS_F16, U>), dim3(blocks), dim3(256), 0, s, codes, scales, out, N, K, ld_out);
  } else {
    const int64_t work = N * K;
    const unsigned blocks = (unsigned)(cdiv(work, 256) < 65536 ? cdiv(work, 256) : 65536);
    hipLaunchKernelGGL(k_dequant_any, dim3(blocks), dim3(256), 0, s, codes, scales, out, out_dtype, N, K, ld_out);
  }
  return hip_check(hipGetLastError(), "dequant launch");
}

extern "C" int qs_qrow_matmul(const void* x, int x_dtype, int64_t ldx, const int8_t* codes,
                              const float* scales, void* y, int64_t ldy, int64_t M, int64_t N,
                              int64_t K, void* stream) {
  int st = validate_common(x, x_dtype, ldx, M, K);
  if (st) return st;
  if (!codes || !scales || !y) return fail(QS_ERR_INVALID, "matmul: null pointer");
  if (N <= 0 || N > (int64_t)1 << 30) return fail(QS_ERR_INVALID, "matmul: bad N=%lld", (long long)N);
  if (ldy < N) return fail(QS_ERR_INVALID, "matmul: ldy < N");
  QrowParams p{};
  p.x = x;
  p.ldx = ldx;
  p.M = (int)M;
  p.K = (int)K;
  p.n_lin = 1;
  p.lin[0] = QrowLin{codes, scales, y, ldy, (int)N, 0};
  return run_linears(p, x_dtype, M, static_cast<hipStream_t>(stream), false);
}

extern "C" int qs_qrow_matmul_row_stable(const void* x, int x_dtype, int64_t ldx,
                                         const int8_t* codes, const float* scales, void* y,
                                         int64_t ldy, int64_t M, int64_t N, int64_t K,
                                         void* stream) {
  int st = validate_common(x, x_dtype, ldx, M, K);
  if (st) return st;
  if (!codes || !scales || !y) return fail(QS_ERR_INVALID, "matmul_row_stable: null pointer");
  if (N <= 0 || N > (int64_t)1 << 30) return fail(QS_ERR_INVALID, "matmul_row_stable: bad N");
  if (ldy < N) return fail(QS_ERR_INVALID, "matmul_row_stable: ldy < N");
  QrowParams p{};
  p.x = x;
  p.ldx = ldx;
  p.M = (int)M;
  p.K = (int)K;
  p.n_lin = 1;
  p.lin[0] = QrowLin{codes, scales, y, ldy, (int)N, 0};
  return run_linears(p, x_dtype, M, static_cast<hipStream_t>(stream), true);
}

extern "C" int qs_qrow_matmul_multi(const void* x, int x_dtype, int64_t ldx, int n_linear,
                                    const int8_t* const* codes, const float* const* scales,
                                    void* const* y, const int64_t* ldy, const int64_t* N,
                                    int64_t M, int64_t K, void* stream) {
  int st = validate_common(x, x_dtype, ldx, M, K);
  if (st) return st;
  if (n_linear < 1 || n_linear > 4) return fail(QS_ERR_LIMIT, "matmul_multi: 1..4 linears");
  if (!codes || !scales || !y || !ldy || !N) return fail(QS_ERR_INVALID, "matmul_multi: null array");
  QrowParams p{};
  p.x = x;
  p.ldx = ldx;
  p.M = (int)M;
  p.K = (int)K;
  p.n_lin = n_linear;
  for (int i = 0; i < n_linear; ++i) {
    if (!codes[i] || !scales[i] || !y[i]) return fail(QS_ERR_INVALID, "matmul_multi: null pointer in linear %d", i);
    if (N[i] <= 0 || N[i] > (int64_t)1 << 30 || ldy[i] < N[i])
      return fail(QS_ERR_INVALID, "matmul_multi: bad N/ldy for linear %d", i);
    p.lin[i] = QrowLin{codes[i], scales[i], y[i], ldy[i], (int)N[i], 0};
  }
  return run_linears(p, x_dtype, M, static_cast<hipStream_t>(stream), false);
}

extern "C" int qs_qrow_swiglu(const void* x, int64_t ldx, const int8_t* gate_codes,
                              const float* gate_scales, const int8_t* up_codes,
                              const float* up_scales, void* y, int64_t ldy, int64_t M, int64_t N,
                              int64_t K, void* stream) {
  int st = validate_common(x, QS_BF16, ldx, M, K);
  if (st) return st;
  if (!gate_codes || !gate_scales || !up_codes || !up_scales || !y)
    return fail(QS_ERR_INVALID, "swiglu: null pointer");
  if (N <= 0 || N > (int64_t)1 << 30 || ldy < N) return fail(QS_ERR_INVALID, "swiglu: bad N/ldy");
  if (M == 0) return QS_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  QrowParams p{};
  p.x = x;
  p.ldx = ldx;
  p.K = (int)K;
  p.n_lin = 2;
  p.lin[0] = QrowLin{gate_codes, gate_scales, y, ldy, (int)N, 0};
  p.lin[1] = QrowLin{up_codes, up_scales, nullptr, 0, (int)N, 0};
  if (M <= kValuRows && valu_eligible(p, QS_BF16)) return run_valu(p, QS_BF16, M, s, true);
  if (mfma_eligible(p, QS_BF16)) {
    for (int64_t m0 = 0; m0 < M; m0 += 32) {
      QrowParams q = p;
      const int mm = (int)((M - m0) < 32 ? (M - m0) : 32);
      q.M = mm;
      q.x = static_cast<const uint16_t*>(x) + m0 * ldx;
      q.lin[0].y = static_cast<uint16_t*>(y) + m0 * ldy;
      const int blocks = (int)cdiv(N, 16);
      if (stream_fits(q)) {
        const int kw = pick_kw_s(blocks, K, 2);
        if (mm <= 16)
          launch_w8a16_s<2, 1, false>(q, blocks, kw, s);
        else
          launch_w8a16_s<2, 2, false>(q, blocks, kw, s);
        continue;
      }
      const int kw = pick_kw(N, K);
      if (mm <= 16)
        launch_w8a16<2, 1, false>(q, blocks, kw, s);
      else
        launch_w8a16<2, 2, false>(q, blocks, kw, s);
    }
    return hip_check(hipGetLastError(), "k_w8a16 swiglu launch");
  }
  p.M = (int)M;
  hipLaunchKernelGGL(k_generic_swiglu, dim3((unsigned)cdiv(N, 4)), dim3(256), 0, s, p);
  return hip_check(hipGetLastError(), "k_generic_swiglu launch");
}

extern "C" size_t qs_qrow_top2_workspace_bytes(int64_t M, int64_t row_count) {
  if (M <= 0 || row_count <= 0) return 0;
  return (size_t)(M * top2_blocks(row_count) * 2) * (sizeof(float) + sizeof(int));
}

namespace qs {
namespace {

// Argument checks shared by the two top-2 entry points (everything but the workspace).
int top2_validate(const void* x, int x_dtype, int64_t ldx, const int8_t* codes, const float* scales,
                  int64_t M, int64_t row_count, int64_t K, int64_t start_row,
                  const int32_t* out_indices, const float* out_values) {
  if (!codes || !scales || !out_indices || !out_values) return fail(QS_ERR_INVALID, "qrow_top2: null pointer");
  int st = validate_common(x, x_dtype, ldx, M, K);
  if (st) return st;
  if (row_count < 2 || row_count > INT_MAX - 1) return fail(QS_ERR_INVALID, "qrow_top2: row_count must be >= 2");
  if (start_row < 0 || start_row + row_count > INT_MAX) return fail(QS_ERR_LIMIT, "qrow_top2: indices exceed int32");
  if (M > 65535) return fail(QS_ERR_LIMIT, "qrow_top2: at most 65535 activation rows");
  return QS_OK;
}

// Launches of the top-2 search for validated arguments, M >= 1, with the per-block
// candidates in `workspace` (at least qs_qrow_top2_workspace_bytes(M, row_count) bytes).
// Every candidate slot the reduce reads is written by the search first, so the workspace
// needs no clearing between calls.
int top2_launch(const void* x, int x_dtype, int64_t ldx, const int8_t* codes, const float* scales,
                int64_t M, int64_t row_count, int64_t K, int64_t start_row, void* workspace,
                int32_t* out_indices, float* out_values, hipStream_t s) {
  int st;
  const int es = x_dtype == QS_F32 ? 4 : 2;
  const int64_t nblk_max = top2_blocks(row_count);
  float* pv = static_cast<float*>(workspace);
  int* pi = reinterpret_cast<int*>(pv + M * nblk_max * 2);
  QrowParams p{};
  p.x = x;
  p.ldx = ldx;
  p.K = (int)K;
  p.n_lin = 1;
  p.lin[0] = QrowLin{codes, scales, nullptr, 0, (int)row_count, 0};
  const int rows = (int)row_count;
  int C;
  if (valu_eligible(p, x_dtype)) {
    const int mb = valu_mb(x_dtype, K, M);
    C = 2 * top2_grid(rows);
    for (int64_t m0 = 0; m0 < M; m0 += mb) {
      QrowParams q = p;
      q.M = (int)((M - m0) < mb ? (M - m0) : mb);
      q.x = static_cast<const char*>(x) + m0 * ldx * es;
      float* qv = pv + m0 * C;
      int* qi = pi + m0 * C;
      const size_t lds = (size_t)q.M * K * es;
      if (x_dtype == QS_F32) {
        if (mb == 4) launch_top2_mb<QS_F32, 4>(q, rows, (int)start_row, qv, qi, lds, s);
        else if (mb == 2) launch_top2_mb<QS_F32, 2>(q, rows, (int)start_row, qv, qi, lds, s);
        else launch_top2_mb<QS_F32, 1>(q, rows, (int)start_row, qv, qi, lds, s);
      } else if (x_dtype == QS_BF16) {
        if (mb == 2) launch_top2_mb<QS_BF16, 2>(q, rows, (int)start_row, qv, qi, lds, s);
        else launch_top2_mb<QS_BF16, 1>(q, rows, (int)start_row, qv, qi, lds, s);
      } else {
        if (mb == 2) launch_top2_mb<QS_F16, 2>(q, rows, (int)start_row, qv, qi, lds, s);
        else launch_top2_mb<QS_F16, 1>(q, rows, (int)start_row, qv, qi, lds, s);
      }
    }
  } else {
    const int nblk = (int)nblk_max;
    C = 2 * nblk;
    for (int64_t m = 0; m < M; ++m) {
      QrowParams q = p;
      q.M = 1;
      q.x = static_cast<const char*>(x) + m * ldx * es;
      hipLaunchKernelGGL(k_generic_top2, dim3((unsigned)nblk), dim3(256), 0, s, q, x_dtype, rows,
                         (int)start_row, pv + m * C, pi + m * C);
    }
  }
  st = hip_check(hipGetLastError(), "qrow top-2 launch");
  if (st) return st;
  hipLaunchKernelGGL(k_top2_reduce, dim3((unsigned)M), dim3(256), 0, s, pv, pi, C, out_indices, out_values);
  return hip_check(hipGetLastError(), "k_top2_reduce launch");
}

}  // namespace
}  // namespace qs

extern "C" int qs_qrow_top2(const void* x, int x_dtype, int64_t ldx, const int8_t* codes,
                            const float* scales, int64_t M, int64_t row_count, int64_t K,
                            int64_t start_row, void* workspace, size_t workspace_bytes,
                            int32_t* out_indices, float* out_values, void* stream) {
  int st = top2_validate(x, x_dtype, ldx, codes, scales, M, row_count, K, start_row, out_indices,
                         out_values);
  if (st) return st;
  if (M == 0) return QS_OK;
  if (!workspace || workspace_bytes < qs_qrow_top2_workspace_bytes(M, row_count))
    return fail(QS_ERR_INVALID, "qrow_top2: workspace smaller than qs_qrow_top2_workspace_bytes()");
  return top2_launch(x, x_dtype, ldx, codes, scales, M, row_count, K, start_row, workspace,
                     out_indices, out_values, static_cast<hipStream_t>(stream));
}

// ---- allocation-free top-2 -------------------------------------------------------------
// The candidates live in a file-scope device array, one copy per GPU.  Host code never
// passes `scratch` itself to a kernel: its host-side name is a stand-in, not a device
// address.  The device address comes from hipGetSymbolAddress, taken once per device
// with that device current, and kept in g_scratch_ptr.
static __device__ __align__(256) unsigned char scratch[QS_TOP2_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on `dev`, resolved on first use.
int scratch_ptr(int dev, void** out) {
  if (dev < 0 || dev >= kMaxDevices) return fail(QS_ERR_UNSUPPORTED, "qrow_top2_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int prev = 0;
    hipError_t e = hipGetDevice(&prev);
    if (e != hipSuccess) return hip_check(e, "qrow_top2_noalloc: hipGetDevice");
    if (prev != dev && (e = hipSetDevice(dev)) != hipSuccess)
      return hip_check(e, "qrow_top2_noalloc: hipSetDevice");
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (prev != dev) {
      hipError_t r = hipSetDevice(prev);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess) return hip_check(e, "qrow_top2_noalloc: hipGetSymbolAddress(scratch)");
    if (!p) return fail(QS_ERR_HIP, "qrow_top2_noalloc: scratch has no device address");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return QS_OK;
}
}  // namespace

extern "C" int qs_qrow_top2_noalloc(const void* x, int x_dtype, int64_t ldx, const int8_t* codes,
                                    const float* scales, int64_t M, int64_t row_count, int64_t K,
                                    int64_t start_row, int32_t* out_indices, float* out_values,
                                    void* stream) {
  int st = top2_validate(x, x_dtype, ldx, codes, scales, M, row_count, K, start_row, out_indices,
                         out_values);
  if (st) return st;
  if (M == 0) return QS_OK;
  if (qs_qrow_top2_workspace_bytes(M, row_count) > (size_t)QS_TOP2_SCRATCH_BYTES)
    return fail(QS_ERR_LIMIT,
                "qrow_top2_noalloc: M=%lld x %lld rows needs %zu scratch bytes, more than the %d "
                "bytes of the per-device scratch array",
                (long long)M, (long long)row_count, qs_qrow_top2_workspace_bytes(M, row_count),
                QS_TOP2_SCRATCH_BYTES);
  hipStream_t s = static_cast<hipStream_t>(stream);
  int dev = -1;
  hipError_t e = s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return hip_check(e, "qrow_top2_noalloc: stream device");
  void* ws = nullptr;
  st = scratch_ptr(dev, &ws);
  if (st) return st;
  return top2_launch(x, x_dtype, ldx, codes, scales, M, row_count, K, start_row, ws, out_indices,
                     out_values, s);
}

extern "C" int qs_qrow_rerank_fp32(const void* x, int x_dtype, int64_t ldx, const int8_t* codes,
                                   const float* scales, int64_t page_rows, int64_t K, int64_t start_row,
                                   const int64_t* candidates, int C, int64_t M, int64_t* out_indices,
                                   float* out_values, void* stream) {
  if (!codes || !scales || !candidates || !out_indices || !out_values)
    return fail(QS_ERR_INVALID, "qrow_rerank: null pointer");
  int st = validate_common(x, x_dtype, ldx, M, K);
  if (st) return st;
  if (C < 1 || C > 16) return fail(QS_ERR_LIMIT, "qrow_rerank: 1..16 candidates per row");
  if (page_rows < 1 || page_rows > INT_MAX) return fail(QS_ERR_INVALID, "qrow_rerank: bad page_rows");
  if (M == 0) return QS_OK;
  if (M > 65535) return fail(QS_ERR_LIMIT, "qrow_rerank: at most 65535 activation rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_rerank_fp32, dim3((unsigned)M), dim3(64 * C), 0, s, x, x_dtype, ldx, codes, scales,
                     (int)page_rows, (int)K, start_row, candidates, C, out_indices, out_values);
  return hip_check(hipGetLastError(), "k_rerank_fp32 launch");
}
