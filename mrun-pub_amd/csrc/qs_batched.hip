// Batched-decode W8A16 qrow linears on gfx950 (1 <= M <= 32 bf16/f16 activation rows).
//
// Kernel
//   k_bdec<P, MT, F16> : one workgroup = (64-row weight tile, K slice).  Its 4 waves own 16
//                        weight rows each (P = 2: the same 16 rows of gate and of up) and
//                        share ONE LDS copy of the activation slice [M, slice], so the
//                        activations cross the memory system 2M/64 bytes per weight byte
//                        (<= 1 at M = 32) instead of once per 16-row tile.  The activation
//                        slice is requested first, the weights second (HBM straight to
//                        VGPRs, nontemporal 128-bit loads), so the LDS staging waits only for
//                        the activations while the weights stay in flight.  Weights are
//                        dequantized in registers to the W8A16 contract bf16(float(code) *
//                        scale) and fed to v_mfma_f32_16x16x32_{bf16,f16} with the
//                        activations as operand A.
//                        With one slice the epilogue is stored straight from the
//                        accumulators.  Otherwise each slice's fp32 partial sums go to the
//                        workspace through coherent stores, the workgroup bumps its tile's
//                        counter, and the workgroup that brings it to S sums the S partials
//                        of every output of the tile in slice order s = 0..S-1 (coherent
//                        loads), stores the epilogue (bf16/f16, or the paired SwiGLU) and
//                        resets the counter to zero for the next call.  No workgroup ever
//                        waits for another, and there is no second launch.
// The split S and the slice length depend on (N, K) only, never on M, and a 16x16x32 MFMA
// sums every output element over its k in a fixed order whatever the other rows hold, so
// a row's result does not depend on the rest of the batch.
//
// MFMA operand mapping (16x16x32, wave64): lane l supplies row (l & 15) of A and column
// (l & 15) of B, 8 consecutive k of k-block (l >> 4).  Per 128-k chunk a lane reads the
// 32 contiguous weight bytes at k = 128c + 32(l >> 4) of its row and the matching 32
// activations; each 8 of them feed one MFMA.  The accumulator of lane l holds
// D[4(l >> 4) + q][l & 15], q = 0..3.
#include "qs_common.h"

namespace qs {
namespace {

constexpr int kBdecRows = 64;   // weight rows per workgroup tile
constexpr int kBdecWaves = 4;   // 16 rows per wave

// 128-k chunks per slice at most: K <= 2048 takes one slice, so no workgroup hands partial
// sums to another; the slice's activations sit in LDS
template <int P>
constexpr int kBdecMaxCS = 16;
// slices at most (the fixup holds every partial of its outputs in VGPRs at once)
template <int P>
constexpr int kBdecMaxS = P == 2 ? 1 : 8;
// weight chunks in flight per wave: the whole slice (a 64-row tile runs one workgroup per
// CU, 1 wave per SIMD, so the registers are there; every byte is requested at once)
template <int P>
constexpr int kBdecWin = 16;

struct BdecLin {
  const int8_t* codes;
  const float* scales;
  void* y;
  int64_t ldy;
  int N;
  int tile_begin;  // first 64-row tile of this linear
  int n_begin;     // first output column of this linear in the partial rows
};

struct BdecParams {
  const uint16_t* x;
  int64_t ldx;
  int M, K, C;     // C = K / 128
  int S, CS;       // slices and chunks per slice (the last slice may be shorter)
  int n_lin;
  int n_total;     // columns of a partial row (sum of N over the linears)
  BdecLin lin[4];
  float* part;     // [S][P][M][n_total]
  int* counters;   // [tiles], zero on entry and on exit
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

// LDS row stride of the staged activation slice, in bytes: 16 bytes of padding put
// consecutive rows 4 banks apart, so the 16 rows a fragment read touches do not collide.
template <int P>
constexpr int kXStride = kBdecMaxCS<P> * 256 + 16;

__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

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

template <int P, int MT, bool F16>
__global__ __launch_bounds__(kBdecWaves * 64, 1) void k_bdec(BdecParams p) {
  typedef Half<F16> H;
  typedef typename H::vec hvec;
  constexpr int CSM = kBdecMaxCS<P>;
  constexpr int XS = kXStride<P>;
  constexpr int XPT = 16 * MT * CSM * 16 / (kBdecWaves * 64);  // staged vectors per thread
  __shared__ __attribute__((aligned(16))) uint8_t xs[16 * MT * XS];
  __shared__ int last;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int tile = (int)blockIdx.x / p.S;
  const int s = (int)blockIdx.x - tile * p.S;
  int li = 0;
  if (P == 1) {
#pragma unroll
    for (int j = 1; j < 4; ++j)
      if (j < p.n_lin && tile >= p.lin[j].tile_begin) li = j;
  }
  const BdecLin& L0 = p.lin[li];
  const int N = L0.N;
  const int t0 = (tile - L0.tile_begin) * kBdecRows;  // first row of the tile
  const int n0 = t0 + 16 * wave;
  const int n = n0 + col < N ? n0 + col : N - 1;  // clamped rows are loaded, never stored
  const int c0 = s * p.CS;
  const int cs = min(p.CS, p.C - c0);  // >= 1

  // 1. activation slice [16*MT rows, cs*128 k] -> registers, rows >= M as zeros
  const int vec_per_row = cs * 16;
  const int total = 16 * MT * vec_per_row;
  i32x4 xv[XPT];
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int v = tid + i * kBdecWaves * 64;
    const int m = v / vec_per_row;
    const int e = v - m * vec_per_row;
    xv[i] = (v < total && m < p.M)
                ? *reinterpret_cast<const i32x4*>(p.x + (int64_t)m * p.ldx + (int64_t)c0 * 128 + 8 * e)
                : i32x4{0, 0, 0, 0};
  }
  __builtin_amdgcn_sched_barrier(0);
  // 2. the first window of this wave's weight chunks (16 rows) -> VGPRs
  constexpr int WW = kBdecWin<P>;
  const int8_t* wrow[P];
#pragma unroll
  for (int pl = 0; pl < P; ++pl)
    wrow[pl] = p.lin[P == 2 ? pl : li].codes + (int64_t)n * p.K + (int64_t)c0 * 128 + 32 * grp;
  i32x4 wv[CSM][P][2];
  auto load_chunk = [&](int c) {
#pragma unroll
    for (int pl = 0; pl < P; ++pl)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        wv[c][pl][h] = c < cs ? __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(wrow[pl] + c * 128 + 16 * h))
                              : i32x4{0, 0, 0, 0};
  };
#pragma unroll
  for (int c = 0; c < WW; ++c) load_chunk(c);
  float sc[P];
#pragma unroll
  for (int pl = 0; pl < P; ++pl) sc[pl] = p.lin[P == 2 ? pl : li].scales[n];
  __builtin_amdgcn_sched_barrier(0);
  // 3. stage the activations (waits for them only)
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int v = tid + i * kBdecWaves * 64;
    if (v < total) {
      const int m = v / vec_per_row;
      const int e = v - m * vec_per_row;
      *reinterpret_cast<i32x4*>(xs + m * XS + 16 * e) = xv[i];
    }
  }
  __syncthreads();

  // 4. MFMA over the slice; chunk c + WW is requested once chunk c is consumed
  f32x4 acc[P][MT];
#pragma unroll
  for (int pl = 0; pl < P; ++pl)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[pl][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < CSM; ++c) {
    if (c < cs) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        hvec a[MT][2];
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            a[t][j] = *reinterpret_cast<const hvec*>(xs + (16 * t + col) * XS + 2 * (c * 128 + 32 * grp + 16 * h + 8 * j));
#pragma unroll
        for (int pl = 0; pl < P; ++pl) {
          hvec b0, b1;
          H::deq(wv[c][pl][h], sc[pl], b0, b1);
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            acc[pl][t] = H::mma(a[t][0], b0, acc[pl][t]);
            acc[pl][t] = H::mma(a[t][1], b1, acc[pl][t]);
          }
        }
      }
    }
    if (c + WW < CSM) load_chunk(c + WW);
  }

  // lane holds D[m = 16t + 4grp + q][n0 + col]
  const int no = n0 + col;
  if (p.S == 1) {  // the whole K in one slice: store the epilogue directly
    if (no >= N) return;
    uint16_t* y = static_cast<uint16_t*>(L0.y);
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = 16 * t + 4 * grp + q;
        float v[P];
#pragma unroll
        for (int pl = 0; pl < P; ++pl) v[pl] = acc[pl][t][q];
        if (m < p.M) y[(int64_t)m * L0.ldy + no] = bdec_out<P, F16>(v);
      }
    return;
  }

  // 5. partial sums of this slice (coherent stores), then the tile's arrival counter
  if (no < N) {
    const int ncol = L0.n_begin + no;
#pragma unroll
    for (int pl = 0; pl < P; ++pl)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int m = 16 * t + 4 * grp + q;
          if (m < p.M) store_coherent(&p.part[(((int64_t)s * P + pl) * p.M + m) * p.n_total + ncol], acc[pl][t][q]);
        }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
  __syncthreads();
  if (tid == 0)
    last = __hip_atomic_fetch_add(&p.counters[tile], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == p.S - 1;
  __syncthreads();
  if (!last) return;

  // 6. the tile's last workgroup: fixed-order sum over the slices, epilogue, counter reset.
  //    Thread tid owns column r = tid % 64 of rows m = tid / 64 + 4i; all of its partials
  //    are requested before the first is summed, so the fixup costs one memory latency.
  constexpr int SM = kBdecMaxS<P>;
  constexpr int OPT = 16 * MT / kBdecWaves;  // outputs per thread
  const int r = tid & 63;
  const int mg = tid >> 6;
  const bool rok = t0 + r < N;
  const int64_t ncol = L0.n_begin + t0 + (rok ? r : 0);
  float pv[OPT][P][SM];
#pragma unroll
  for (int o = 0; o < OPT; ++o) {
    const int m = mg + kBdecWaves * o;
#pragma unroll
    for (int pl = 0; pl < P; ++pl)
#pragma unroll
      for (int k2 = 0; k2 < SM; ++k2)
        pv[o][pl][k2] = (k2 < p.S && m < p.M && rok)
                            ? load_coherent(&p.part[(((int64_t)k2 * P + pl) * p.M + m) * p.n_total + ncol])
                            : 0.f;
  }
  uint16_t* y = static_cast<uint16_t*>(L0.y);
#pragma unroll
  for (int o = 0; o < OPT; ++o) {
    const int m = mg + kBdecWaves * o;
    float v[P];
#pragma unroll
    for (int pl = 0; pl < P; ++pl) {
      float a = pv[o][pl][0];
#pragma unroll
      for (int k2 = 1; k2 < SM; ++k2)
        if (k2 < p.S) a = add_rn(a, pv[o][pl][k2]);
      v[pl] = a;
    }
    if (m < p.M && rok) y[(int64_t)m * L0.ldy + t0 + r] = bdec_out<P, F16>(v);
  }
  if (tid == 0) __hip_atomic_store(&p.counters[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Slices from K only: as few as hold at most kBdecMaxCS<P> chunks each, of equal length.
void bdec_split(int64_t n_tiles, int C, int P, int& S, int& CS) {
  (void)n_tiles;
  const int csm = P == 2 ? kBdecMaxCS<2> : kBdecMaxCS<1>;
  S = (C + csm - 1) / csm;  // may exceed kBdecMaxS<P>: rejected by the caller
  CS = (C + S - 1) / S;
  S = (C + CS - 1) / CS;
}

void bdec_shape(const int64_t* N, int n_lin, int P, int64_t& tiles, int64_t& cols) {
  tiles = cols = 0;
  for (int i = 0; i < n_lin; ++i) {
    tiles += cdiv(N[i], kBdecRows);
    cols += N[i];
    if (P == 2) break;  // gate and up share the tiles and the columns
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
  p.C = (int)(K / 128);
  p.f16 = x_dtype == QS_F16;
  return QS_OK;
}

template <int P>
int bdec_launch(BdecParams& p, void* workspace, size_t workspace_bytes, int* counters, int64_t n_counters,
                hipStream_t s) {
  int64_t N[4], tiles, cols;
  for (int i = 0; i < p.n_lin; ++i) N[i] = p.lin[i].N;
  bdec_shape(N, p.n_lin, P, tiles, cols);
  int tb = 0, nb = 0;
  for (int i = 0; i < (P == 2 ? 1 : p.n_lin); ++i) {
    p.lin[i].tile_begin = tb;
    p.lin[i].n_begin = nb;
    tb += (int)cdiv(p.lin[i].N, kBdecRows);
    nb += p.lin[i].N;
  }
  p.n_total = (int)cols;
  bdec_split(tiles, p.C, P, p.S, p.CS);
  if (p.S > kBdecMaxS<P>)
    return fail(QS_ERR_UNSUPPORTED, "qrow batched: K = %d is longer than %d x %d x 128", p.K, kBdecMaxS<P>,
                kBdecMaxCS<P>);
  if (p.S > 1) {
    const size_t need = (size_t)p.S * P * p.M * p.n_total * sizeof(float);
    if (!workspace || workspace_bytes < need)
      return fail(QS_ERR_INVALID, "qrow batched: workspace smaller than qs_qrow_batched_workspace_bytes()");
    if (!counters || n_counters < tiles)
      return fail(QS_ERR_INVALID, "qrow batched: fewer tile counters than qs_qrow_batched_counters()");
  }
  p.part = static_cast<float*>(workspace);
  p.counters = counters;
  const dim3 grid((unsigned)(tiles * p.S)), block(kBdecWaves * 64);
  const bool mt2 = p.M > 16;
  if (p.f16) {
    if (mt2) hipLaunchKernelGGL((k_bdec<P, 2, true>), grid, block, 0, s, p);
    else hipLaunchKernelGGL((k_bdec<P, 1, true>), grid, block, 0, s, p);
  } else {
    if (mt2) hipLaunchKernelGGL((k_bdec<P, 2, false>), grid, block, 0, s, p);
    else hipLaunchKernelGGL((k_bdec<P, 1, false>), grid, block, 0, s, p);
  }
  return hip_check(hipGetLastError(), "k_bdec launch");
}

}  // namespace
}  // namespace qs

using namespace qs;

extern "C" size_t qs_qrow_batched_workspace_bytes(int64_t M, int n_linear, const int64_t* N, int64_t K,
                                                  int swiglu) {
  if (!N || n_linear < 1 || n_linear > 4 || M < 1 || K < 128) return 0;
  const int P = swiglu ? 2 : 1;
  int64_t tiles, cols;
  bdec_shape(N, n_linear, P, tiles, cols);
  int S, CS;
  bdec_split(tiles, (int)(K / 128), P, S, CS);
  return S > 1 ? (size_t)S * P * M * cols * sizeof(float) : 0;
}

extern "C" int64_t qs_qrow_batched_counters(int n_linear, const int64_t* N, int swiglu) {
  if (!N || n_linear < 1 || n_linear > 4) return 0;
  int64_t tiles, cols;
  bdec_shape(N, n_linear, swiglu ? 2 : 1, tiles, cols);
  return tiles;
}

extern "C" int qs_qrow_matmul_batched(const void* x, int x_dtype, int64_t ldx, int n_linear,
                                      const int8_t* const* codes, const float* const* scales, void* const* y,
                                      const int64_t* ldy, const int64_t* N, int64_t M, int64_t K,
                                      void* workspace, size_t workspace_bytes, int32_t* counters,
                                      int64_t n_counters, void* stream) {
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
  return bdec_launch<1>(p, workspace, workspace_bytes, counters, n_counters, static_cast<hipStream_t>(stream));
}

extern "C" int qs_qrow_swiglu_batched(const void* x, int64_t ldx, const int8_t* gate_codes,
                                      const float* gate_scales, const int8_t* up_codes, const float* up_scales,
                                      void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* workspace,
                                      size_t workspace_bytes, int32_t* counters, int64_t n_counters, void* stream) {
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
  return bdec_launch<2>(p, workspace, workspace_bytes, counters, n_counters, static_cast<hipStream_t>(stream));
}
