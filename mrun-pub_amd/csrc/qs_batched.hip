// Batched-decode W8A16 qrow linears on gfx950 (1 <= M <= 32 bf16/f16 activation rows).
//
// Kernels
//   k_bd2<P, MT, WR, WK, F16, MS2> : one workgroup = (16 * WR weight rows of P planes, K slice;
//                               MS2: one 16-row half of 17..32 activation rows);
//                               P = 2 pairs the gate and up rows of a SwiGLU tile.  The
//                               slice's activations reach LDS by DMA and serve all of the
//                               workgroup's rows; the weights stream from HBM into VGPRs,
//                               are dequantized in registers to the W8A16 contract
//                               bf16(float(code) * scale) and fed to
//                               v_mfma_f32_16x16x32_{bf16,f16}.
//   k_bd2_reduce<P, F16>      : the K slices' fp32 partial sums added in slice order, and the
//                               epilogue (bf16/f16, or the paired SwiGLU).
// MFMA operand mapping (16x16x32, wave64): lane l supplies row (l & 15) of A and column
// (l & 15) of B, 8 consecutive k of k-block (l >> 4); the accumulator of lane l holds
// D[4(l >> 4) + q][l & 15], q = 0..3.
#include "qs_common.h"

#include <algorithm>

namespace qs {
namespace {

struct BdecLin {
  const int8_t* codes;
  const float* scales;
  void* y;
  int64_t ldy;
  int N;
  int tile_begin;  // first workgroup row tile of this linear
  int n_begin;     // first output column of this linear in the partial rows
};

// The checked call arguments shared by the entry points.
struct BdecParams {
  const uint16_t* x;
  int64_t ldx;
  int M, K;
  int n_lin;
  BdecLin lin[4];
  bool f16;
};

template <bool F16>
struct Half;
template <>
struct Half<false> {
  typedef bf16x8 vec;
  static __device__ __forceinline__ void deq(i32x4 w, float s, vec& lo, vec& hi) { deq16_bf16(w, s, lo, hi); }
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t out(float v) { return f32_to_bf16_bits(v); }
};
template <>
struct Half<true> {
  typedef f16x8 vec;
  static __device__ __forceinline__ void deq(i32x4 w, float s, vec& lo, vec& hi) { deq16_f16(w, s, lo, hi); }
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t out(float v) { return f32_to_f16_bits(v); }
};

__device__ __forceinline__ float silu(float g) { return g * (1.0f / (1.0f + expf(-g))); }

// Epilogue of one output: plane sums -> bf16/f16 (P = 1) or the paired SwiGLU (P = 2).
template <int P, bool F16>
__device__ __forceinline__ uint16_t bdec_out(const float (&v)[P]) {
  if constexpr (P == 2) {
    const float gt = bf16_bits_to_f32(f32_to_bf16_bits(v[0]));
    const float ut = bf16_bits_to_f32(f32_to_bf16_bits(v[1]));
    const float sl = bf16_bits_to_f32(f32_to_bf16_bits(silu(gt)));
    return f32_to_bf16_bits(sl * ut);
  } else {
    return Half<F16>::out(v[0]);
  }
}

int bdec_prepare(BdecParams& p, const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K) {
  if (!x) return fail(QS_ERR_INVALID, "qrow batched: null activations");
  if (x_dtype != QS_BF16 && x_dtype != QS_F16) return fail(QS_ERR_INVALID, "qrow batched: activations BF16 or F16");
  if (M < 1 || M > 32) return fail(QS_ERR_LIMIT, "qrow batched: 1 <= M <= 32");
  if (K < 128 || K % 128 || K > ((int64_t)1 << 30))
    return fail(QS_ERR_UNSUPPORTED, "qrow batched: K must be a positive multiple of 128");
  if (ldx < K || (ldx * 2) % 16 || !aligned(x, 16))
    return fail(QS_ERR_UNSUPPORTED, "qrow batched: activation rows must be 16-byte aligned");
  p = BdecParams{};
  p.x = static_cast<const uint16_t*>(x);
  p.ldx = ldx;
  p.M = (int)M;
  p.K = (int)K;
  p.f16 = x_dtype == QS_F16;
  return QS_OK;
}

// ---------------------------------------------------------------------------------
// k_bd2: one workgroup = (RS <= 16 * WR weight rows, K slice); its WR * WK waves own 16 rows
// (masked past the workgroup's RS) x a contiguous part of the slice each.  The slice's activations [M, slice] reach LDS by
// DMA (buffer_load ... lds, 1 KiB per wave instruction, 16-byte chunk j of row m at slot
// j ^ (m & 15), so the 16 rows of a fragment read fall in distinct banks); the wave's
// weight chunks (64 k of 16 rows, 16 bytes per lane) are all requested right behind the
// copies and land in VGPRs while the copies are waited for.  Dequantized weights are the
// MFMA A operand, the activations B, so lane l ends up with 4 consecutive output columns
// of one activation row.  The WK parts are summed in fixed order through LDS; with S > 1
// slices the fp32 partial sums go to the workspace and k_bd2_reduce sums them in slice
// order and stores the epilogue.  WK, S and the slice length -- the K order of every sum --
// depend on (N, K) only (WR and RS, the rows per workgroup, and the activation-row split
// may follow M: they change no sum), and
// an MFMA sums each output over its k in a fixed order whatever the other rows hold, so a
// row's result does not depend on the rest of the batch.
// ---------------------------------------------------------------------------------
constexpr int kBd2MaxPS = 8;   // 64-k chunks per wave part (all requested at once)
constexpr int kBd2MaxCS = 20;  // 64-k chunks per slice: <= 80 KiB of activations at M = 32,
                               // so two workgroups fit a CU's LDS
constexpr int kBd2MaxS = 16;   // slices (k_bd2_reduce requests all of them at once)

struct Bd2Params {
  const uint16_t* x;
  int64_t ldx;
  int M, K, C;   // C = K / 64
  int S, CS;     // slices and 64-k chunks per slice (even: 16-chunk LDS row groups)
  int RS;        // weight rows per workgroup (a multiple of 4, at most 16 * WR)
  int n_lin, n_total;
  int vec;       // outputs and partial rows allow 4-wide stores
  BdecLin lin[4];
  float* part;   // [S][P][M][n_total] when S > 1
};

// One wave's 1 KiB global -> LDS copy (lane l's 16 bytes at buffer offset voff land at
// dst + 16 l).  Not a template: in template-dependent code the host compilation pass drops
// the kernel's launch stub over this builtin.
__device__ __forceinline__ void bd2_copy16(__amdgpu_buffer_rsrc_t r, uint8_t* dst, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, 0, 0, 0);
}

// Sections 6-7 of k_bd2: the WK parts of the wave's 16 rows summed in order through
// LDS (bsm, WK * WR * P * MT * 64 f32x4), then the epilogue (S == 1) or the slice's partial
// sums (S > 1).  n0: the wave's first row; N: the row bound (the workgroup's share).
template <int P, int MT, int WR, int WK, bool F16>
__device__ __forceinline__ void bd2_finish(const Bd2Params& p, const BdecLin& L0, const f32x4 (&acc)[P][MT],
                                           uint8_t* bsm, int wr, int wk, int lane, int col, int grp, int n0,
                                           int N, int s, int m0, bool sync_first) {
  // 6. the WK parts summed in order wk = 0, 1, ... through LDS
  f32x4 out[P][MT];
  if constexpr (WK > 1) {
    if (sync_first) __syncthreads();  // every wave is done with the LDS activation slice
    f32x4* red = reinterpret_cast<f32x4*>(bsm);  // [WK][WR][P][MT][64]
#pragma unroll
    for (int pl = 0; pl < P; ++pl)
#pragma unroll
      for (int t = 0; t < MT; ++t) red[(((wk * WR + wr) * P + pl) * MT + t) * 64 + lane] = acc[pl][t];
    __syncthreads();
    if (wk != 0) return;
#pragma unroll
    for (int pl = 0; pl < P; ++pl)
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        f32x4 a = red[((wr * P + pl) * MT + t) * 64 + lane];
#pragma unroll
        for (int k2 = 1; k2 < WK; ++k2) a += red[(((k2 * WR + wr) * P + pl) * MT + t) * 64 + lane];
        out[pl][t] = a;
      }
  } else {
#pragma unroll
    for (int pl = 0; pl < P; ++pl)
#pragma unroll
      for (int t = 0; t < MT; ++t) out[pl][t] = acc[pl][t];
  }

  // 7. lane holds D[n = nb + q][m = m0 + 16 t + col]
  const int nb = n0 + 4 * grp;
  if (nb >= N) return;
  const bool full = p.vec && nb + 3 < N;
  if (p.S == 1) {
    uint16_t* y = static_cast<uint16_t*>(L0.y);
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = m0 + 16 * t + col;
      if (m >= p.M) continue;
      uint16_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v[P];
#pragma unroll
        for (int pl = 0; pl < P; ++pl) v[pl] = out[pl][t][q];
        o[q] = bdec_out<P, F16>(v);
      }
      uint16_t* yr = y + (int64_t)m * L0.ldy + nb;
      if (full) {
        *reinterpret_cast<uint2*>(yr) = make_uint2(o[0] | (uint32_t)o[1] << 16, o[2] | (uint32_t)o[3] << 16);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (nb + q < N) yr[q] = o[q];
      }
    }
    return;
  }
#pragma unroll
  for (int pl = 0; pl < P; ++pl)
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = m0 + 16 * t + col;
      if (m >= p.M) continue;
      float* pr = p.part + (((int64_t)s * P + pl) * p.M + m) * p.n_total + L0.n_begin + nb;
      if (full) {
        *reinterpret_cast<f32x4*>(pr) = out[pl][t];
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (nb + q < N) pr[q] = out[pl][t][q];
      }
    }
}

template <int P, int MT, int WR, int WK, bool F16, bool MS2>
__global__ __launch_bounds__(WR * WK * 64) void k_bd2(Bd2Params p) {
  typedef Half<F16> H;
  typedef typename H::vec hvec;
  constexpr int NW = WR * WK;
  extern __shared__ __attribute__((aligned(1024))) uint8_t bsm[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave % WR, wk = wave / WR;
  const int col = lane & 15, grp = lane >> 4;
  // unit u = (row tile, slice).  MS2: activation rows 0-15 and 16-31 of a unit in two
  // workgroups, blocks 16q + j and 16q + 8 + j (j < 8; the host launches MS2 only when the
  // unit count is a multiple of 8), so both halves run on one XCD (blocks are dealt to the
  // 8 XCDs round robin) and the second reads the unit's weights from that XCD's L2
  int u = (int)blockIdx.x, m0 = 0;
  if constexpr (MS2) {
    u = (((int)blockIdx.x >> 4) << 3) + ((int)blockIdx.x & 7);
    m0 = ((int)blockIdx.x & 8) << 1;
  }
  // One argument from each 64-byte argument line the prologue reads, requested in one
  // batch at entry.  Left to itself the compiler asks for the arguments in dependent
  // rounds (the slice count, then the linears' first tiles, then the selected linear's
  // fields at a computed offset), a scalar-cache miss each, before the first row scale is
  // requested; with every line fetched at entry the later rounds hit the scalar cache.
  static_assert(offsetof(Bd2Params, lin) + 3 * sizeof(BdecLin) < 256, "argument lines");
  if constexpr (P == 1)
    asm volatile("" ::"s"(p.S), "s"(p.lin[0].N), "s"(p.lin[1].tile_begin), "s"(p.lin[3].tile_begin));
  else
    asm volatile("" ::"s"(p.S), "s"(p.lin[0].N));
  const int tile = u / p.S;
  const int s = u - tile * p.S;
  int li = 0;
  if (P == 1) {
#pragma unroll
    for (int j = 1; j < 4; ++j)
      if (j < p.n_lin && tile >= p.lin[j].tile_begin) li = j;
  }
  const BdecLin& L0 = p.lin[li];
  const int tb = (tile - L0.tile_begin) * p.RS;  // the workgroup's first row
  const int N = min(L0.N, tb + p.RS);             // rows past this bound are another workgroup's
  const int n0 = tb + 16 * wr;                    // this wave's 16 rows (masked at N)
  const int c0 = s * p.CS;
  const int cs = min(p.CS, p.C - c0);  // chunks of this slice, >= 1
  const int kbeg = c0 * 64;
  const int NCH = p.CS * 8;  // 16-byte chunks per staged activation row

  // 1. row scales: the oldest requests, so the wait below covers them
  const int nr = n0 + col;
  float sc[P];
#pragma unroll
  for (int pl = 0; pl < P; ++pl) sc[pl] = p.lin[P == 2 ? pl : li].scales[nr < N ? nr : tb];

  // Early dequant: the weights are requested first and each chunk is dequantized into bf16
  // registers as it lands, while the activation copies are still in flight; the MFMAs
  // follow the barrier.  It holds P * 8 VGPRs per chunk, so the 16-wave paired forms keep
  // the late order (copies first, dequant after the barrier) to stay out of scratch.
  constexpr bool EARLY = !(P == 2 && WR * WK > 12);
  const int PS = (cs + WK - 1) / WK;
  const int cb = wk * PS;
  const int ce = min(cs, cb + PS);
  const int wlim = L0.N * p.K;
  const int wlane = nr < N ? nr * p.K + kbeg + 16 * grp : wlim;  // rows past N: no access
  i32x4 wv[kBd2MaxPS][P];
  // this wave's part of the slice's weights: every chunk requested at once (zero past the
  // part and for rows >= N, whose lane offsets lie past the buffer)
  auto load_weights = [&]() {
#pragma unroll
    for (int pl = 0; pl < P; ++pl) {
      const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<int8_t*>(p.lin[P == 2 ? pl : li].codes), (short)0, wlim, 0x00020000);
#pragma unroll
      for (int c = 0; c < kBd2MaxPS; ++c)
        wv[c][pl] = __builtin_bit_cast(
            i32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, cb + c < ce && nr < N ? wlane + 64 * (cb + c) : wlim, 0, 0));
    }
  };
  // the activation slice [16 MT rows][NCH chunks] -> LDS; rows >= M and chunks past the
  // slice read out of the buffer's range (zero, no memory access)
  const int xlim = p.M * (int)p.ldx * 2;
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.x), (short)0, xlim, 0x00020000);
  auto copy_slice = [&]() {
    const int total = 16 * MT * NCH;
    for (int u0 = wave * 64; u0 < total; u0 += NW * 64) {
      const int e = u0 + lane;
      const int m = e / NCH, jj = e - m * NCH, j = jj ^ (m & 15);
      const bool ok = m0 + m < p.M && j < 8 * cs;
      bd2_copy16(xr, bsm + 16 * u0, ok ? ((m0 + m) * (int)p.ldx + kbeg + 8 * j) * 2 : xlim);
    }
  };
  hvec wb[EARLY ? kBd2MaxPS : 1][P][2];
  if constexpr (EARLY) {
    // 2. weights, 3. copies, 4. each weight chunk dequantized as it lands (loads return in
    //    issue order, so the weights need no copy to land), 5. every copy of this wave has
    //    landed, and the barrier makes every wave's visible
    load_weights();
    __builtin_amdgcn_sched_barrier(0);
    copy_slice();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < kBd2MaxPS; ++c)
      if (cb + c < ce) {
#pragma unroll
        for (int pl = 0; pl < P; ++pl) H::deq(wv[c][pl], sc[pl], wb[c][pl][0], wb[c][pl][1]);
      }
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  } else {
    // 2. copies, 3. weights, 4. this wave's copies have landed once at most its
    //    kBd2MaxPS * P weight loads are outstanding; the barrier then makes every wave's
    //    copies visible
    copy_slice();
    __builtin_amdgcn_sched_barrier(0);
    load_weights();
    __builtin_amdgcn_sched_barrier(0);
    static_assert(kBd2MaxPS * P == 8 || kBd2MaxPS * P == 16, "wait counts below");
    if constexpr (kBd2MaxPS * P == 16)
      asm volatile("s_waitcnt vmcnt(16)\n\ts_barrier" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
  }

  // 6. MFMA over the part
  f32x4 acc[P][MT];
#pragma unroll
  for (int pl = 0; pl < P; ++pl)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[pl][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < kBd2MaxPS; ++c) {
    if (cb + c < ce) {
      const int j = 8 * (cb + c) + 2 * grp;  // chunk of k = 64 (cb + c) + 16 grp in the slice
      hvec xa[MT][2];
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const int m = 16 * t + col;
#pragma unroll
        for (int h = 0; h < 2; ++h)
          xa[t][h] = *reinterpret_cast<const hvec*>(bsm + 16 * (m * NCH + ((j + h) ^ (m & 15))));
      }
#pragma unroll
      for (int pl = 0; pl < P; ++pl) {
        hvec b0, b1;
        if constexpr (EARLY) {
          b0 = wb[c][pl][0];
          b1 = wb[c][pl][1];
        } else {
          H::deq(wv[c][pl], sc[pl], b0, b1);
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          acc[pl][t] = H::mma(b0, xa[t][0], acc[pl][t]);
          acc[pl][t] = H::mma(b1, xa[t][1], acc[pl][t]);
        }
      }
    }
  }

  bd2_finish<P, MT, WR, WK, F16>(p, L0, acc, bsm, wr, wk, lane, col, grp, n0, N, s, m0, true);
}

// Slice sums of k_bd2 in slice order and the epilogue: one thread per (row m, 4 columns
// of the partial row); every linear's N is a multiple of 4 (the host checks).
template <int P, bool F16>
__global__ __launch_bounds__(128) void k_bd2_reduce(Bd2Params p) {
  const int q4 = p.n_total / 4;
  const int i = (int)blockIdx.x * 128 + (int)threadIdx.x;
  const int m = i / q4;
  if (m >= p.M) return;
  const int ncol = 4 * (i - m * q4);
  int li = 0;
  if (P == 1) {
#pragma unroll
    for (int j = 1; j < 4; ++j)
      if (j < p.n_lin && ncol >= p.lin[j].n_begin) li = j;
  }
  f32x4 v[kBd2MaxS][P];  // every slice requested before the first is added
#pragma unroll
  for (int s = 0; s < kBd2MaxS; ++s)
#pragma unroll
    for (int pl = 0; pl < P; ++pl)
      if (s < p.S) v[s][pl] = *reinterpret_cast<const f32x4*>(p.part + (((int64_t)s * P + pl) * p.M + m) * p.n_total + ncol);
  f32x4 a[P];
#pragma unroll
  for (int pl = 0; pl < P; ++pl) {
    a[pl] = v[0][pl];
#pragma unroll
    for (int s = 1; s < kBd2MaxS; ++s)
      if (s < p.S) a[pl] += v[s][pl];
  }
  const BdecLin& L = p.lin[li];
  uint16_t o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float v[P];
#pragma unroll
    for (int pl = 0; pl < P; ++pl) v[pl] = a[pl][q];
    o[q] = bdec_out<P, F16>(v);
  }
  uint16_t* yr = static_cast<uint16_t*>(L.y) + (int64_t)m * L.ldy + (ncol - L.n_begin);
  if (p.vec) {
    *reinterpret_cast<uint2*>(yr) = make_uint2(o[0] | (uint32_t)o[1] << 16, o[2] | (uint32_t)o[3] << 16);
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) yr[q] = o[q];
  }
}

struct Bd2Shape {
  int WR, WK, S, CS;
  int RS;      // rows per workgroup: a multiple of 4, at most 16 * WR
  int MS = 1;  // activation-row splits (2: one 16-row half of M = 17..32 per workgroup)
};

// Split.  The K order of every sum -- WK waves per slice and S slices -- depends on (N, K)
// only; WR (rows per workgroup, which does not change any sum) may follow M.  From
// same-box timings of the config-2 shapes at M = 16 / 32:
//  * rows up to 2048 k: one slice, 16-row workgroups of 8 waves along K (q/k/v 4.9 / 6.0 us,
//    o 4.8 / 6.0 us; a K split with its reduce launch costs 2-3 us more).  For M > 16 the
//    activation rows split in two (MS = 2): two workgroups per 16-row unit, 16 activation
//    rows each, so q/k/v takes 256 workgroups with half the staged slice each; the chained
//    M = 32 pass went 1.022 -> 0.980 ms (the same split for the SwiGLU and the long rows
//    made it slower: their dequant is repeated per half);
//  * the paired SwiGLU (1536 k): one slice, 4 waves along K, about one workgroup per CU
//    (a CU streams its weights at a limited rate, so the CU with the most rows sets the
//    time): rows per workgroup ceil(N / 256) rounded up to 4, as 16-row MFMA tiles with
//    the rows past the workgroup's share masked (no loads, no stores).  8960 rows: 249
//    workgroups of 36 rows (48-row ones: 10.4 / 11.9 us; 16-row ones 10.7 / 23.0; 64-row
//    ones 11.8 / 14.3; the 96 KiB activation slice of M = 32 allows one workgroup per CU);
//  * longer rows: 64-row workgroups, slices of at most kBd2MaxCS chunks to about 256
//    workgroups, 2 or 4 waves along K (1536 x 8960: 10 slices, 9.1 / 11.5 us).
Bd2Shape bd2_shape(const int64_t* N, int n_lin, int P, int64_t K, int64_t M) {
  const int C = (int)(K / 64);
  if (C <= 32) {
    if (P == 2) {
      // about one workgroup per CU: rows per workgroup a multiple of 4 in [16, 48]
      const int rs = (int)std::min<int64_t>(48, std::max<int64_t>(16, (cdiv(N[0], 256) + 3) / 4 * 4));
      return Bd2Shape{(rs + 15) / 16, 4, 1, C, rs};
    }
    return Bd2Shape{1, 8, 1, C, 16, 2};
  }
  Bd2Shape sh{4, 1, 1, C, 64};
  int64_t tiles = 0;
  for (int i = 0; i < (P == 2 ? 1 : n_lin); ++i) tiles += cdiv(N[i], 16 * sh.WR);
  // slices: enough for about 256 workgroups and for the LDS cap, at most kBd2MaxS; then
  // equal even lengths
  int S = (int)std::max<int64_t>(1, 256 / tiles);
  S = std::max(S, (C + kBd2MaxCS - 1) / kBd2MaxCS);
  S = std::min(S, kBd2MaxS);
  int CS = (C + S - 1) / S;
  CS += CS & 1;
  sh.S = (C + CS - 1) / CS;
  sh.CS = CS;
  const int need = (CS + kBd2MaxPS - 1) / kBd2MaxPS;
  sh.WK = need <= 1 ? 1 : need <= 2 ? 2 : 4;
  return sh;
}

template <int P, int MT, bool F16>
void bd2_launch_mt(const Bd2Params& p, const Bd2Shape& sh, int64_t tiles, hipStream_t s) {
  const dim3 grid((unsigned)(tiles * sh.S));
  const size_t xbytes = (size_t)16 * MT * sh.CS * 8 * 16;
  const size_t rbytes = (size_t)sh.WK * sh.WR * P * MT * 64 * 16;
  const size_t lds = std::max(xbytes, rbytes);
#define QS_BD2(WR_, WK_)                                                                              \
  if (sh.WR == WR_ && sh.WK == WK_) {                                                                 \
    hipLaunchKernelGGL((k_bd2<P, MT, WR_, WK_, F16, false>), grid, dim3(WR_ * WK_ * 64), lds, s, p);  \
    return;                                                                                           \
  }
  QS_BD2(4, 1) QS_BD2(4, 2) QS_BD2(4, 4) QS_BD2(3, 4) QS_BD2(2, 4) QS_BD2(1, 4) QS_BD2(1, 8)
#undef QS_BD2
}

template <int P>
int bd2_launch(Bd2Params& p, const Bd2Shape& sh, void* workspace, size_t workspace_bytes, bool f16, hipStream_t s) {
  int64_t tiles = 0;
  int nb = 0;
  for (int i = 0; i < (P == 2 ? 1 : p.n_lin); ++i) {
    p.lin[i].tile_begin = (int)tiles;
    p.lin[i].n_begin = nb;
    tiles += cdiv(p.lin[i].N, sh.RS);
    nb += p.lin[i].N;
  }
  p.n_total = nb;
  p.S = sh.S;
  p.CS = sh.CS;
  p.RS = sh.RS;
  if (p.S > 1) {
    const size_t need = (size_t)p.S * P * p.M * p.n_total * sizeof(float);
    if (!workspace || workspace_bytes < need)
      return fail(QS_ERR_INVALID, "qrow batched: workspace smaller than qs_qrow_batched_workspace_bytes()");
    if (!aligned(workspace, 16)) return fail(QS_ERR_INVALID, "qrow batched: workspace must be 16-byte aligned");
  }
  p.part = static_cast<float*>(workspace);
  bool split = false;
  if constexpr (P == 1) {
    split = p.M > 16 && sh.MS == 2 && (tiles * sh.S) % 8 == 0 && sh.WR == 1 && sh.WK == 8;
    if (split) {  // one 16-row half of the activations per workgroup, two workgroups per unit
      const dim3 grid((unsigned)(2 * tiles * sh.S));
      const size_t lds = std::max((size_t)16 * sh.CS * 8 * 16, (size_t)8 * 64 * 16);
      if (f16) hipLaunchKernelGGL((k_bd2<1, 1, 1, 8, true, true>), grid, dim3(512), lds, s, p);
      else hipLaunchKernelGGL((k_bd2<1, 1, 1, 8, false, true>), grid, dim3(512), lds, s, p);
    }
  }
  if (split) {
  } else if (p.M > 16) {
    if (f16) bd2_launch_mt<P, 2, true>(p, sh, tiles, s);
    else bd2_launch_mt<P, 2, false>(p, sh, tiles, s);
  } else {
    if (f16) bd2_launch_mt<P, 1, true>(p, sh, tiles, s);
    else bd2_launch_mt<P, 1, false>(p, sh, tiles, s);
  }
  int st = hip_check(hipGetLastError(), "k_bd2 launch");
  if (st || p.S == 1) return st;
  const int64_t threads = (int64_t)p.M * (p.n_total / 4);
  const dim3 rg((unsigned)cdiv(threads, 128));
  if (f16) hipLaunchKernelGGL((k_bd2_reduce<P, true>), rg, dim3(128), 0, s, p);
  else hipLaunchKernelGGL((k_bd2_reduce<P, false>), rg, dim3(128), 0, s, p);
  return hip_check(hipGetLastError(), "k_bd2_reduce launch");
}

// The batched entry points on k_bd2: limits, the (N, K) split and the store layout.
template <int P>
int bd2_run(const BdecParams& b, const int64_t* N, int n_lin, void* workspace, size_t workspace_bytes,
            hipStream_t s, const Bd2Shape* forced = nullptr) {
  Bd2Params p{};
  p.x = b.x;
  p.ldx = b.ldx;
  p.M = b.M;
  p.K = b.K;
  p.C = b.K / 64;
  p.n_lin = b.n_lin;
  for (int i = 0; i < 4; ++i) p.lin[i] = b.lin[i];
  if ((int64_t)b.M * b.ldx * 2 >= INT_MAX) return fail(QS_ERR_LIMIT, "qrow batched: activations exceed 2^31 bytes");
  bool vec = true;
  for (int i = 0; i < (P == 2 ? 1 : n_lin); ++i) {
    if ((N[i] + 64) * b.K >= INT_MAX) return fail(QS_ERR_LIMIT, "qrow batched: weights exceed 2^31 bytes");
    vec = vec && N[i] % 4 == 0 && p.lin[i].ldy % 4 == 0 && aligned(p.lin[i].y, 8);
  }
  p.vec = vec;
  const Bd2Shape sh = forced ? *forced : bd2_shape(N, n_lin, P, b.K, b.M);
  if ((sh.CS + sh.WK - 1) / sh.WK > kBd2MaxPS || sh.S > kBd2MaxS)
    return fail(QS_ERR_UNSUPPORTED, "qrow batched: K = %d needs more than %d slices of %d chunks", b.K, kBd2MaxS,
                4 * kBd2MaxPS);
  if (sh.S > 1) {
    for (int i = 0; i < (P == 2 ? 1 : n_lin); ++i)
      if (N[i] % 4) return fail(QS_ERR_UNSUPPORTED, "qrow batched: a K split needs N %% 4 == 0");
  }
  return bd2_launch<P>(p, sh, workspace, workspace_bytes, b.f16, s);
}

}  // namespace
}  // namespace qs

using namespace qs;

extern "C" size_t qs_qrow_batched_workspace_bytes(int64_t M, int n_linear, const int64_t* N, int64_t K,
                                                  int swiglu) {
  if (!N || n_linear < 1 || n_linear > 4 || M < 1 || K < 128) return 0;
  const int P = swiglu ? 2 : 1;
  int64_t cols = 0;
  for (int i = 0; i < (P == 2 ? 1 : n_linear); ++i) cols += N[i];
  const Bd2Shape sh = bd2_shape(N, n_linear, P, K, std::min<int64_t>(M, 32));
  return sh.S > 1 ? (size_t)sh.S * P * std::min<int64_t>(M, 32) * cols * sizeof(float) : 0;
}

extern "C" int qs_qrow_matmul_batched(const void* x, int x_dtype, int64_t ldx, int n_linear,
                                      const int8_t* const* codes, const float* const* scales, void* const* y,
                                      const int64_t* ldy, const int64_t* N, int64_t M, int64_t K,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  if (n_linear < 1 || n_linear > 4) return fail(QS_ERR_LIMIT, "qrow batched: 1..4 linears");
  if (!codes || !scales || !y || !ldy || !N) return fail(QS_ERR_INVALID, "qrow batched: null array");
  BdecParams p;
  int st = bdec_prepare(p, x, x_dtype, ldx, M, K);
  if (st) return st;
  p.n_lin = n_linear;
  for (int i = 0; i < n_linear; ++i) {
    if (!codes[i] || !scales[i] || !y[i]) return fail(QS_ERR_INVALID, "qrow batched: null pointer in linear %d", i);
    if (N[i] <= 0 || N[i] > ((int64_t)1 << 30) || ldy[i] < N[i])
      return fail(QS_ERR_INVALID, "qrow batched: bad N/ldy for linear %d", i);
    if (!aligned(codes[i], 16)) return fail(QS_ERR_UNSUPPORTED, "qrow batched: weight rows must be 16-byte aligned");
    p.lin[i] = BdecLin{codes[i], scales[i], y[i], ldy[i], (int)N[i], 0, 0};
  }
  return bd2_run<1>(p, N, n_linear, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int qs_qrow_swiglu_batched(const void* x, int64_t ldx, const int8_t* gate_codes,
                                      const float* gate_scales, const int8_t* up_codes, const float* up_scales,
                                      void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  if (!gate_codes || !gate_scales || !up_codes || !up_scales || !y)
    return fail(QS_ERR_INVALID, "swiglu batched: null pointer");
  if (N <= 0 || N > ((int64_t)1 << 30) || ldy < N) return fail(QS_ERR_INVALID, "swiglu batched: bad N/ldy");
  if (!aligned(gate_codes, 16) || !aligned(up_codes, 16))
    return fail(QS_ERR_UNSUPPORTED, "swiglu batched: weight rows must be 16-byte aligned");
  BdecParams p;
  int st = bdec_prepare(p, x, QS_BF16, ldx, M, K);
  if (st) return st;
  p.n_lin = 2;
  p.lin[0] = BdecLin{gate_codes, gate_scales, y, ldy, (int)N, 0, 0};
  p.lin[1] = BdecLin{up_codes, up_scales, nullptr, 0, (int)N, 0, 0};
  const int64_t Ns[1] = {N};
  return bd2_run<2>(p, Ns, 1, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}
