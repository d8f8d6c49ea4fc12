// Routed-MoE hot path on gfx950: router, route compiler, routed-row quantization, ragged
// grouped int8 GEMM (W8A8, optional fused SwiGLU epilogue, slot indirection) and the
// fixed-rank-order reducer.
//
// Kernels
//   k_moe_router      : one wave per token: fp32 softmax over E logits, top-k (ties ->
//                       lower expert id), optional renormalisation, weights as fp32/bf16.
//   k_moe_route_par   : one workgroup per expert (moderate A * E): ballot counts of the
//                       lower experts give its start, then its assignments in index order.
//   k_moe_route       : one workgroup; expert histogram, exclusive prefix and a STABLE
//                       expert-major scatter (wave ballots give each assignment its rank
//                       among earlier same-expert assignments), so the queue order equals
//                       the reference's stable argsort and is identical on every call.
//   k_moe_gather_quant: per routed row, int8 per-token quantization of source[token_ids[a]]
//                       (the W8A8 recipe: s = max|x|/127, 0 -> 1; rint; clamp +-127);
//                       k_moe_gather_quant8 is the same with a wave per row and 16-byte
//                       loads (H % 8 == 0, aligned rows).
//   k_moe_stream<...> : one workgroup per (group, 4 or 8 waves of output rows), the row
//                       blocks of a group kept on one XCD.  The group's
//                       routed rows (up to 16*MT at a time) are staged once in LDS; each
//                       wave streams its weight rows (16 rows of gate and up for SwiGLU,
//                       16-64 rows otherwise) over the full K through a window of 128-byte
//                       chunks in flight and multiplies them with v_mfma_i32_16x16x64_i8
//                       against every 16-row tile of the staged rows; epilogue (float(acc) * a_scale[row]) * w_scale[n] ->
//                       bf16/fp32, or the paired SwiGLU of gate row n and up row n + N.
//   k_moe_gemm<...>   : K beyond what the LDS tile holds: one workgroup per (group, 16-row
//                       tile); its waves split K, hold their weight slice in VGPRs and
//                       walk the group's rows 16 at a time, LDS reduction over the split.
//   k_moe_reduce      : out[t, :] = sum over rank r of float(y[inv[t*k + r], :]) *
//                       coef[inv[t*k + r]], each product rounded, summed in rank order;
//                       fp32 out, or bf16 (the fp32 sum rounded once).  k_moe_reduce8 is
//                       the same with 8 consecutive h per thread.
#include "qs_common.h"

#include <type_traits>

namespace qs {

// ----------------------------------------------------------------------------------
// router
// ----------------------------------------------------------------------------------
template <int XT>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
  if constexpr (XT == QS_F32) return static_cast<const float*>(p)[i];
  else return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}

// E <= 64 * J logits per wave (J per lane), k <= 16.  Rank r is kept by lane r (no
// dynamically indexed arrays, which would live in scratch memory).
template <int XT, int J>
__global__ __launch_bounds__(256) void k_moe_router(const void* __restrict__ logits, int T, int E,
                                                    int k, int norm, int64_t* __restrict__ idx,
                                                    void* __restrict__ w, int w_dtype) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  float v[J];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = lane + 64 * j;
    v[j] = e < E ? ld<XT>(logits, (int64_t)t * E + e) : -INFINITY;
    mx = fmaxf(mx, v[j]);
  }
  mx = wave_max(mx);
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = lane + 64 * j;
    v[j] = e < E ? expf(v[j] - mx) : 0.f;
    sum += v[j];
  }
  sum = wave_sum(sum);
#pragma unroll
  for (int j = 0; j < J; ++j) v[j] = v[j] / sum;
  float mine = 0.f;  // lane r: the weight of rank r
  int mine_idx = 0;
  float tot = 0.f;   // fp32 sum of the kept weights in rank order
  for (int r = 0; r < k; ++r) {
    float best = -1.f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int e = lane + 64 * j;
      if (e < E && (v[j] > best || (v[j] == best && e < bi))) {
        best = v[j];
        bi = e;
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ob = __shfl_xor(best, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      if (ob > best || (ob == best && oi < bi)) {
        best = ob;
        bi = oi;
      }
    }
    if (lane == r) {
      mine = best;
      mine_idx = bi;
    }
    tot += best;
#pragma unroll
    for (int j = 0; j < J; ++j)
      if (lane + 64 * j == bi) v[j] = -2.f;  // exclude
  }
  // renormalisation divides by the fp32 sum of the kept weights, summed in rank order
  if (lane < k) {
    const float wr = norm ? mine / tot : mine;
    idx[(int64_t)t * k + lane] = mine_idx;
    if (w_dtype == QS_F32)
      static_cast<float*>(w)[(int64_t)t * k + lane] = wr;
    else
      static_cast<uint16_t*>(w)[(int64_t)t * k + lane] = f32_to_bf16_bits(wr);
  }
}

// ----------------------------------------------------------------------------------
// route compiler (single workgroup, 1024 threads = 16 waves)
// ----------------------------------------------------------------------------------
constexpr int kRouteWaves = 16;
constexpr int kRouteMaxE = 512;
constexpr int kRouteBatch = 8;  // 64-assignment segments a wave loads before using them

__device__ __forceinline__ uint64_t ballot64(bool p) { return __ballot(p); }

template <int IT, int WT>
__global__ __launch_bounds__(1024) void k_moe_route(const void* __restrict__ top_idx,
                                                    const void* __restrict__ top_w, int A, int k,
                                                    int E, int64_t* __restrict__ token_ids,
                                                    float* __restrict__ coef,
                                                    int32_t* __restrict__ starts,
                                                    int32_t* __restrict__ counts,
                                                    int64_t* __restrict__ inverse) {
  __shared__ int cnt[kRouteWaves][kRouteMaxE];
  __shared__ int base[kRouteMaxE];
  __shared__ int wave_tot[kRouteMaxE / 64];
  __shared__ int total;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  auto expert_of = [&](int i) -> int {
    // int64 ids are range-checked before narrowing (2^32 + 3 is not expert 3)
    if constexpr (IT == QS_I64) {
      const int64_t x = static_cast<const int64_t*>(top_idx)[i];
      return x >= 0 && x < E ? (int)x : -1;
    } else {
      return static_cast<const int32_t*>(top_idx)[i];
    }
  };
  for (int i = tid; i < kRouteWaves * kRouteMaxE; i += 1024) (&cnt[0][0])[i] = 0;
  __syncthreads();
  // wave w owns the contiguous assignment range [lo, hi)
  const int segs = (A + 63) / 64;
  const int per = (segs + kRouteWaves - 1) / kRouteWaves;
  const int lo = wave * per * 64;
  const int hi = min(A, (wave + 1) * per * 64);
  // the wave's expert ids, 8 loads in flight per lane (one memory round trip per 512)
  for (int b0 = lo; b0 < hi; b0 += 64 * kRouteBatch) {
    int eb[kRouteBatch];
#pragma unroll
    for (int j = 0; j < kRouteBatch; ++j) {
      const int i = b0 + 64 * j + lane;
      eb[j] = i < hi ? expert_of(i) : -1;
    }
    for (int j = 0; j < kRouteBatch; ++j)
      if (eb[j] >= 0 && eb[j] < E) atomicAdd(&cnt[wave][eb[j]], 1);
  }
  __syncthreads();
  // per expert: total count, then the exclusive prefix over experts as a wave scan
  // (threads 0 .. E-1, at most 8 waves) plus the totals of the lower waves
  int c_e = 0;
  if (tid < E)
    for (int w = 0; w < kRouteWaves; ++w) c_e += cnt[w][tid];
  int incl = c_e;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  if (lane == 63 && wave < kRouteMaxE / 64) wave_tot[wave] = incl;
  __syncthreads();
  if (tid < E) {
    int excl = incl - c_e;
    for (int w = 0; w < wave; ++w) excl += wave_tot[w];
    counts[tid] = c_e;
    starts[tid] = excl;
    base[tid] = excl;
  }
  if (tid == 0) {
    int run = 0;
    for (int w = 0; w < (E + 63) / 64; ++w) run += wave_tot[w];
    total = run;
  }
  __syncthreads();
  if (tid < E) {
    int run = base[tid];
    for (int w = 0; w < kRouteWaves; ++w) {
      const int c = cnt[w][tid];
      cnt[w][tid] = run;  // becomes wave w's cursor for expert tid
      run += c;
    }
  }
  __syncthreads();
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  for (int b0 = lo; b0 < hi; b0 += 64 * kRouteBatch) {
    int eb[kRouteBatch];
    float wb[kRouteBatch];
#pragma unroll
    for (int j = 0; j < kRouteBatch; ++j) {
      const int i = b0 + 64 * j + lane;
      eb[j] = i < hi ? expert_of(i) : -1;
      if constexpr (WT == QS_F32) wb[j] = i < hi ? static_cast<const float*>(top_w)[i] : 0.f;
      else wb[j] = i < hi ? bf16_bits_to_f32(static_cast<const uint16_t*>(top_w)[i]) : 0.f;
    }
    for (int j = 0; j < kRouteBatch; ++j) {
      if (b0 + 64 * j >= hi) break;  // wave-uniform: no segment left
      const int i = b0 + 64 * j + lane;
      const bool valid = i < hi;
      const int e = eb[j];
      const bool ok = valid && e >= 0 && e < E;
      uint64_t match = ballot64(ok);
      for (int b = 0; b < nbits; ++b) {
        const uint64_t bb = ballot64(ok && ((e >> b) & 1));
        match &= ((e >> b) & 1) ? bb : ~bb;
      }
      // match: lanes with the same expert (valid ones); my rank among lower lanes
      const uint64_t lower = lane ? (~0ull >> (64 - lane)) : 0ull;
      const int rank = __popcll(match & lower);
      const int n_same = __popcll(match);
      int dest = 0;
      if (ok) dest = cnt[wave][e] + rank;
      // the highest lane of each expert group advances the cursor (after everyone read it)
      __builtin_amdgcn_wave_barrier();
      if (ok && rank == n_same - 1) cnt[wave][e] += n_same;
      __builtin_amdgcn_wave_barrier();
      if (ok) {
        token_ids[dest] = i / k;
        coef[dest] = wb[j];
        if (inverse) inverse[i] = dest;
      } else if (valid && inverse) {
        inverse[i] = -1;  // expert outside [0, E): no queue row
      }
    }
  }
  // Assignments with an expert outside [0, E) are left out of the queue.  The rows they
  // leave free at its end get token 0 and coefficient 0, so a consumer that walks all A
  // rows never reads an unwritten index.
  for (int q = total + tid; q < A; q += 1024) {
    token_ids[q] = 0;
    coef[q] = 0.f;
  }
}

// Route compiler for moderate A * E: one workgroup per expert e, 8 waves, each wave owning
// a contiguous range of 64-assignment segments.  Pass 1 counts, with ballots, the valid
// assignments of a lower expert (their sum over the waves is starts[e]) and those of e;
// pass 2 writes e's assignments in index order at starts[e] + (rank among them), which is
// the stable expert-major order of k_moe_route.  No workgroup waits for another.  Ranges
// of at most kParSegs segments per wave stay in registers between the passes.
constexpr int kParWaves = 8;
constexpr int kParSegs = 8;

template <int IT, int WT>
__device__ __forceinline__ void route_par_body(int e, const void* __restrict__ top_idx,
                                               const void* __restrict__ top_w, int A, int k, int E,
                                               int64_t* __restrict__ token_ids, float* __restrict__ coef,
                                               int32_t* __restrict__ starts, int32_t* __restrict__ counts,
                                               int64_t* __restrict__ inverse) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  auto expert_of = [&](int i) -> int {
    // int64 ids are range-checked before narrowing (2^32 + 3 is not expert 3)
    if constexpr (IT == QS_I64) {
      const int64_t x = static_cast<const int64_t*>(top_idx)[i];
      return x >= 0 && x < E ? (int)x : -1;
    } else {
      return static_cast<const int32_t*>(top_idx)[i];
    }
  };
  const int nseg = (A + 63) / 64;
  const int per = (nseg + kParWaves - 1) / kParWaves;
  const int s_lo = wave * per, s_hi = min(nseg, s_lo + per);
  const bool resident = per <= kParSegs;
  int ev[kParSegs];  // expert of assignment (seg * 64 + lane); -1: none or out of range
  auto load = [&](int s0) {
#pragma unroll
    for (int j = 0; j < kParSegs; ++j) {
      const int i = (s0 + j) * 64 + lane;
      const int x = (s0 + j < s_hi && i < A) ? expert_of(i) : -1;
      ev[j] = x >= 0 && x < E ? x : -1;
    }
  };
  int lt = 0, eq = 0;
  for (int s0 = s_lo; s0 < s_hi; s0 += kParSegs) {
    load(s0);
#pragma unroll
    for (int j = 0; j < kParSegs; ++j) {
      lt += __popcll(ballot64(ev[j] >= 0 && ev[j] < e));
      eq += __popcll(ballot64(ev[j] == e));
    }
  }
  __shared__ int s_lt[kParWaves], s_eq[kParWaves];
  if (lane == 0) {
    s_lt[wave] = lt;
    s_eq[wave] = eq;
  }
  __syncthreads();
  int start = 0, cnt = 0, run = 0;
#pragma unroll
  for (int w = 0; w < kParWaves; ++w) {
    start += s_lt[w];
    cnt += s_eq[w];
    run += w < wave ? s_eq[w] : 0;
  }
  run += start;
  if (threadIdx.x == 0) {
    starts[e] = start;
    counts[e] = cnt;
  }
  const uint64_t lower = lane ? (~0ull >> (64 - lane)) : 0ull;
  for (int s0 = s_lo; s0 < s_hi; s0 += kParSegs) {
    if (!resident) load(s0);
#pragma unroll
    for (int j = 0; j < kParSegs; ++j) {
      if (s0 + j >= s_hi) break;  // wave-uniform
      const int i = (s0 + j) * 64 + lane;
      const uint64_t m = ballot64(ev[j] == e);
      if (ev[j] == e) {
        const int dest = run + __popcll(m & lower);
        token_ids[dest] = i / k;
        if constexpr (WT == QS_F32) coef[dest] = static_cast<const float*>(top_w)[i];
        else coef[dest] = bf16_bits_to_f32(static_cast<const uint16_t*>(top_w)[i]);
        if (inverse) inverse[i] = dest;
      } else if (e == 0 && inverse && i < A && ev[j] < 0) {
        inverse[i] = -1;  // expert outside [0, E): no queue row
      }
      run += __popcll(m);
    }
  }
  // rows past the valid assignments: token 0, coefficient 0 (the last expert's workgroup
  // knows their number, start + cnt)
  if (e == E - 1)
    for (int q = start + cnt + (int)threadIdx.x; q < A; q += kParWaves * 64) {
      token_ids[q] = 0;
      coef[q] = 0.f;
    }
}

template <int IT, int WT>
__global__ __launch_bounds__(kParWaves * 64) void k_moe_route_par(
    const void* __restrict__ top_idx, const void* __restrict__ top_w, int A, int k, int E,
    int64_t* __restrict__ token_ids, float* __restrict__ coef, int32_t* __restrict__ starts,
    int32_t* __restrict__ counts, int64_t* __restrict__ inverse) {
  route_par_body<IT, WT>((int)blockIdx.x, top_idx, top_w, A, k, E, token_ids, coef, starts, counts, inverse);
}

// ----------------------------------------------------------------------------------
// routed-row quantization
// ----------------------------------------------------------------------------------
template <int XT>
__global__ __launch_bounds__(256) void k_moe_gather_quant(const void* __restrict__ src, int64_t lds_,
                                                          const int64_t* __restrict__ rows, int H,
                                                          int8_t* __restrict__ q,
                                                          float* __restrict__ scale) {
  const int64_t a = blockIdx.x;
  const int64_t r = rows ? rows[a] : a;
  const void* xr = static_cast<const char*>(src) + r * lds_ * (XT == QS_F32 ? 4 : 2);
  float amax = 0.f;
  for (int h = threadIdx.x; h < H; h += 256) amax = fmaxf(amax, fabsf(ld<XT>(xr, h)));
  amax = wave_max(amax);
  __shared__ float red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float s = amax / 127.0f;
  if (s == 0.f) s = 1.f;
  if (threadIdx.x == 0) scale[a] = s;
  for (int h = threadIdx.x; h < H; h += 256) {
    float v = rintf(ld<XT>(xr, h) / s);
    v = fminf(fmaxf(v, -127.f), 127.f);
    q[a * H + h] = static_cast<int8_t>(v);
  }
}

// One wave per routed row, 8 elements (one 16- or 32-byte piece) per lane and piece; the
// row stays in registers between the absmax and the quantization when it has at most
// 512 pieces (H <= 4096), otherwise it is read twice.  Same recipe and results as
// k_moe_gather_quant (max is order-free; x / s is the correctly rounded quotient).
template <int XT>
struct Piece8 {
  static constexpr int kBytes = XT == QS_F32 ? 32 : 16;
  i32x4 v[XT == QS_F32 ? 2 : 1];
  __device__ __forceinline__ void load(const char* p) {
    v[0] = *reinterpret_cast<const i32x4*>(p);
    if constexpr (XT == QS_F32) v[1] = *reinterpret_cast<const i32x4*>(p + 16);
  }
  __device__ __forceinline__ float at(int e) const {
    if constexpr (XT == QS_F32) return __int_as_float(v[e >> 2][e & 3]);
    else return bf16_bits_to_f32((static_cast<uint32_t>(v[0][e >> 1]) >> (16 * (e & 1))) & 0xffffu);
  }
};

constexpr int kQuantPieces = 8;  // pieces per lane kept in registers

// one wave quantizes row a (source row rows[a], or a)
template <int XT>
__device__ __forceinline__ void gather_quant8_row(int64_t a, const void* __restrict__ src, int64_t ld_src,
                                                  const int64_t* __restrict__ rows, int64_t A, int H,
                                                  int8_t* __restrict__ q, float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  if (a >= A) return;
  const int64_t r = rows ? rows[a] : a;
  const char* xr = static_cast<const char*>(src) + r * ld_src * (XT == QS_F32 ? 4 : 2);
  const int np = H >> 3;
  Piece8<XT> pc[kQuantPieces];
  float amax = 0.f;
  for (int p0 = 0; p0 < np; p0 += 64 * kQuantPieces) {
#pragma unroll
    for (int j = 0; j < kQuantPieces; ++j) {
      const int pi = p0 + 64 * j + lane;
      if (pi < np) {
        pc[j].load(xr + (int64_t)pi * Piece8<XT>::kBytes);
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(pc[j].at(e)));
      }
    }
  }
  amax = wave_max(amax);
  float s = amax / 127.0f;
  if (s == 0.f) s = 1.f;
  if (lane == 0) scale[a] = s;
  const bool resident = np <= 64 * kQuantPieces;
  int8_t* qr = q + a * H;
  const float rs = 1.0f / s;  // correctly rounded
  // wave-uniform: bf16 rows with s >= 2^-120 take the corrected product, others divide
  const bool fast = XT == QS_BF16 && s >= 0x1p-120f;
  auto quantize = [&](auto fast_tag) {
    for (int p0 = 0; p0 < np; p0 += 64 * kQuantPieces) {
#pragma unroll
      for (int j = 0; j < kQuantPieces; ++j) {
        const int pi = p0 + 64 * j + lane;
        if (pi < np) {
          if (!resident) pc[j].load(xr + (int64_t)pi * Piece8<XT>::kBytes);
          uint32_t w[2] = {0u, 0u};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float x = pc[j].at(e);
            float v = rintf(decltype(fast_tag)::value ? quot_markstein(x, s, rs) : x / s);
            v = fminf(fmaxf(v, -127.f), 127.f);
            w[e >> 2] |= (static_cast<uint32_t>(static_cast<int>(v)) & 0xffu) << (8 * (e & 3));
          }
          *reinterpret_cast<uint2*>(qr + (int64_t)pi * 8) = make_uint2(w[0], w[1]);
        }
      }
    }
  };
  if (fast) quantize(std::true_type{});
  else quantize(std::false_type{});
}

template <int XT>
__global__ __launch_bounds__(256) void k_moe_gather_quant8(const void* __restrict__ src, int64_t ld_src,
                                                           const int64_t* __restrict__ rows, int64_t A,
                                                           int H, int8_t* __restrict__ q,
                                                           float* __restrict__ scale) {
  gather_quant8_row<XT>((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6), src, ld_src, rows, A, H, q, scale);
}

// The route compiler (k_moe_route_par) and the per-token quantization of the T source
// rows in one launch: workgroups 0 .. E - 1 compile the route, the rest quantize 8 source
// rows each (a wave per row).  The two parts are independent; the grouped GEMM then reads
// the quantized rows through token_ids (a row's codes and scale do not depend on which
// expert it is routed to, so they equal the quantization of the gathered rows).
template <int IT, int WT, int XT>
__global__ __launch_bounds__(kParWaves * 64) void k_moe_route_quant(
    const void* __restrict__ top_idx, const void* __restrict__ top_w, int A, int k, int E,
    int64_t* __restrict__ token_ids, float* __restrict__ coef, int32_t* __restrict__ starts,
    int32_t* __restrict__ counts, int64_t* __restrict__ inverse, const void* __restrict__ src,
    int64_t ld_src, int64_t T, int H, int8_t* __restrict__ q, float* __restrict__ scale) {
  const int b = (int)blockIdx.x;
  if (b < E) route_par_body<IT, WT>(b, top_idx, top_w, A, k, E, token_ids, coef, starts, counts, inverse);
  else gather_quant8_row<XT>((int64_t)(b - E) * kParWaves + (threadIdx.x >> 6), src, ld_src, nullptr, T, H, q, scale);
}

// ----------------------------------------------------------------------------------
// ragged grouped int8 GEMM
// ----------------------------------------------------------------------------------
// A group's routed-row count, first queue row and weight slot, requested together: without
// a slot table the slot word is read from the starts array (a valid address either way) and
// a select drops it, so no load waits behind the null test or the empty-group exit (the
// three dependent global loads had delayed every workgroup's first weight request).
struct GroupMeta {
  int count, start, slot;
};
__device__ __forceinline__ GroupMeta group_meta(const int32_t* counts, const int32_t* starts, const int32_t* slots,
                                                int g) {
  const int32_t* sp = slots ? slots : starts;
  const int c = counts[g], st = starts[g], sv = sp[g];
  asm volatile("" ::"s"(c), "s"(st), "s"(sv));
  return GroupMeta{c, st, slots ? sv : g};
}

struct MoeGemmParams {
  const int8_t* a;       // [A, K] routed rows, expert-major
  const float* as;       // [A]
  const int8_t* w;       // group g weights at w + slot(g) * w_stride, [N_w, K] row-major
  int64_t w_stride;      // bytes
  const float* ws;       // group g scales at ws + slot(g) * ws_stride
  int64_t ws_stride;     // floats
  const int32_t* starts;
  const int32_t* counts;
  const int32_t* slots;  // nullable
  int N;                 // output features (SwiGLU: half of the weight rows)
  int K;
  void* out;             // [A, N]
  int out_dtype;
  const int64_t* row_ids;  // k_moe_stream, nullable: queue row r reads a / as at row_ids[r]
  int64_t src_rows;        // rows of a and as when row_ids is given
};

__device__ __forceinline__ float silu_f(float g) { return g * (1.0f / (1.0f + expf(-g))); }

// P = 1: plain; P = 2: paired SwiGLU (plane 0 = gate row n, plane 1 = up row n + N).
// KW waves per plane split K; each wave holds CH 64-k chunks of its 16 weight rows.
template <int P, int KW, int CH, int NT>
__global__ __launch_bounds__(P * KW * 64) void k_moe_gemm(MoeGemmParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int plane = wave % P;
  const int ks = wave / P;
  const int col = lane & 15, grp = lane >> 4;
  const int g = blockIdx.y;
  const GroupMeta gm = group_meta(p.counts, p.starts, p.slots, g);
  const int count = gm.count;
  if (count == 0) return;
  const int start = gm.start;
  const int slot = gm.slot;
  const int C = p.K / 64;
  const int ntiles = (p.N + 15) / 16;
  const int tile0 = blockIdx.x * NT;
  const int8_t* wexp = p.w + (int64_t)slot * p.w_stride + 16 * grp;

  // the wave's weight slice of one 16-row tile: chunks ks, ks + KW, ... (at most CH);
  // two slices in registers so that tile t + 1 streams in while tile t is reduced
  i32x4 wv[2][CH];
  auto wload = [&](int b, int t) {
    const int n = min(t * 16 + col, p.N - 1);
    const int8_t* wrow = wexp + (int64_t)(n + plane * p.N) * p.K;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int cc = ks + c * KW;
      wv[b][c] = cc < C ? __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(wrow + (int64_t)cc * 64))
                        : i32x4{0, 0, 0, 0};
    }
  };

  __shared__ i32x4 red[P * KW][64];
  if (tile0 < ntiles) wload(0, tile0);
  // epilogue operands of the first tile / row block, requested with the weights so that
  // the reduction does not wait for a second memory round trip
  float sc0[P], as0[4];
  {
    const int no = min(tile0 * 16 + col, p.N - 1);
#pragma unroll
    for (int pl = 0; pl < P; ++pl) sc0[pl] = p.ws[(int64_t)slot * p.ws_stride + no + pl * p.N];
#pragma unroll
    for (int q = 0; q < 4; ++q) as0[q] = p.as[start + min(4 * grp + q, count - 1)];
  }
#pragma unroll
  for (int ti = 0; ti < NT; ++ti) {
    const int t = tile0 + ti;
    if (t >= ntiles) break;
    const int b = ti & 1;
    if (ti + 1 < NT && t + 1 < ntiles) wload(b ^ 1, t + 1);
    const int n0 = t * 16;
    for (int m0 = 0; m0 < count; m0 += 16) {
      const int m = m0 + col;
      const bool mval = m < count;
      const int8_t* arow = p.a + (int64_t)(start + (mval ? m : 0)) * p.K + 16 * grp;
      i32x4 acc = {0, 0, 0, 0};
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int cc = ks + c * KW;
        if (cc < C) {
          const i32x4 av = mval ? *reinterpret_cast<const i32x4*>(arow + (int64_t)cc * 64) : i32x4{0, 0, 0, 0};
          acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, wv[b][c], acc, 0, 0, 0);
        }
      }
      red[wave][lane] = acc;
      __syncthreads();
      // the K-split partial sums of 16 rows x 16 tokens, reduced and finished by the
      // first wave of each plane group
      if (wave == 0) {
        i32x4 tot[P];
#pragma unroll
        for (int pl = 0; pl < P; ++pl) {
          i32x4 s = red[pl][lane];
#pragma unroll
          for (int k2 = 1; k2 < KW; ++k2) s += red[k2 * P + pl][lane];
          tot[pl] = s;
        }
        const int no = n0 + col;
        if (no < p.N) {
          float sc[P];
#pragma unroll
          for (int pl = 0; pl < P; ++pl)
            sc[pl] = ti == 0 ? sc0[pl] : p.ws[(int64_t)slot * p.ws_stride + no + pl * p.N];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int mr = m0 + 4 * grp + q;
            if (mr < count) {
              const int64_t row = start + mr;
              const float a_s = m0 == 0 ? as0[q] : p.as[row];
              if constexpr (P == 2) {
                const float gv = mul_rn(mul_rn(static_cast<float>(tot[0][q]), a_s), sc[0]);
                const float uv = mul_rn(mul_rn(static_cast<float>(tot[1][q]), a_s), sc[1]);
                const float gt = bf16_bits_to_f32(f32_to_bf16_bits(gv));
                const float ut = bf16_bits_to_f32(f32_to_bf16_bits(uv));
                const float sl = bf16_bits_to_f32(f32_to_bf16_bits(silu_f(gt)));
                static_cast<uint16_t*>(p.out)[row * p.N + no] = f32_to_bf16_bits(mul_rn(sl, ut));
              } else {
                const float v = mul_rn(mul_rn(static_cast<float>(tot[0][q]), a_s), sc[0]);
                if (p.out_dtype == QS_F32)
                  static_cast<float*>(p.out)[row * p.N + no] = v;
                else
                  static_cast<uint16_t*>(p.out)[row * p.N + no] = f32_to_bf16_bits(v);
              }
            }
          }
        }
      }
      __syncthreads();
    }
  }
}

// Streaming grouped GEMM.  Each wave owns RW output rows over the full K: SwiGLU
// (P = 2): 16 rows n0 .. n0 + 15 of gate and the same rows + N of up; plain (P = 1):
// NB consecutive 16-row tiles.  Its NB weight tiles are the B operands of
// v_mfma_i32_16x16x64_i8.  K is walked in chunks of CB bytes: with PAIR (K % 128 == 0)
// a chunk is 128 bytes and lane l loads the 32 contiguous bytes 32(l >> 4) .. +32 of
// tile row l & 15 as two 16-byte pieces, so each 128-byte line of a weight row is asked
// for whole by two back-to-back loads (without PAIR, 64-byte chunks, 16 bytes per lane).
// Piece j of a chunk is the k-block l >> 4 of one MFMA; the A operand is the same bytes
// of staged row (l & 15) of a 16-row tile of the group, read from LDS per piece and
// shared by the NB tiles (rows padded by 16 bytes, so the 16 rows of a read fall in
// distinct banks).  Any assignment of bytes to k-blocks that A and B share gives the
// same exact int32 sum.  The chunk loads run W chunks ahead of the MFMAs, issued in k
// order; slots past the last chunk reload it (static wait counts).  Staged rows past the
// group's count hold stale LDS data: their MFMA columns are never stored.  Weights are
// read with ordinary cached loads: nontemporal loads measured 20-30% slower here.
template <int P, int NB>
struct MoeStreamCfg {
  static constexpr int RW = P == 2 ? 16 : 16 * NB;  // output rows per wave
};

template <int P, int NB, int MT, int W, int WAVES, int PAIR>
__global__ __launch_bounds__(WAVES * 64) void k_moe_stream(MoeGemmParams p) {
  static_assert(P == 1 || NB == 2, "SwiGLU streams the gate and up tiles of one row block");
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int MC = 16 * MT;
  constexpr int NT = WAVES * 64;
  constexpr int RW = MoeStreamCfg<P, NB>::RW;
  constexpr int CB = PAIR ? 128 : 64;  // bytes of a weight row per chunk
  constexpr int PL = PAIR ? 2 : 1;     // 16-byte pieces per lane per chunk
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, q = lane >> 4;
  // Workgroup i runs on XCD i % 8.  The row blocks of one group share its staged routed
  // rows, so consecutive logical indices (group-major) go to one XCD and its L2 serves
  // the repeats: the first 8 * floor(total / 8) workgroups are dealt out XCD-major, the
  // remainder keeps its index (a bijection on [0, total)).
  const int total = gridDim.x * gridDim.y, lin = blockIdx.y * gridDim.x + blockIdx.x;
  const int per_xcd = total / 8;
  const int logical = lin < 8 * per_xcd ? (lin % 8) * per_xcd + lin / 8 : lin;
  const int g = logical / gridDim.x, bx = logical - g * gridDim.x;
  const GroupMeta gm = group_meta(p.counts, p.starts, p.slots, g);
  const int count = gm.count;
  if (count == 0) return;
  const int start = gm.start;
  const int slot = gm.slot;
  const int K = p.K, C = K / CB;
  const int xstride = K + 16;
  int8_t* xs = reinterpret_cast<int8_t*>(lds);                 // [MC][K + 16]
  float* asl = reinterpret_cast<float*>(lds + MC * xstride);   // [MC]
  int64_t* rid = reinterpret_cast<int64_t*>(asl + MC);          // [MC] with row_ids: source rows, -1 = zeros
  const int n0 = (bx * WAVES + wave) * RW;
  const bool live = n0 < p.N;
  const int lo = PAIR ? 32 * q : 16 * q;  // the lane's byte offset within a chunk
  const int8_t* wexp = p.w + (int64_t)slot * p.w_stride;
  const int8_t* wr[NB];
  float wsc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    // weight row of tile b for this lane's column
    const int nb = P == 2 ? min(n0 + col, p.N - 1) + b * p.N : min(n0 + 16 * b + col, p.N - 1);
    wr[b] = wexp + (int64_t)nb * K + lo;
    wsc[b] = p.ws[(int64_t)slot * p.ws_stride + nb];
  }
  const int ppr = K >> 4;  // 16-byte pieces per row

  for (int m0 = 0; m0 < count; m0 += MC) {
    const int mc = min(MC, count - m0);
    // the pass's source row ids, requested before the weight window
    int64_t id = -1;
    if (p.row_ids && tid < mc) id = p.row_ids[start + m0 + tid];
    __builtin_amdgcn_sched_barrier(0);
    i32x4 wv[W][NB][PL];
#pragma unroll
    for (int u = 0; u < W; ++u) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int j = 0; j < PL; ++j)
          wv[u][b][j] = *reinterpret_cast<const i32x4*>(wr[b] + (int64_t)min(u, C - 1) * CB + 16 * j);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (p.row_ids) {
      if (tid < mc) rid[tid] = id >= 0 && id < p.src_rows ? id : -1;
      __syncthreads();
    }
    // routed rows m0 .. m0 + mc of the group and their scales -> LDS, 8 loads in flight
    const int tot = mc * ppr;
    const int8_t* arows = p.a + (int64_t)(start + m0) * K;
    for (int i0 = 0; i0 < tot; i0 += 8 * NT) {
      i32x4 v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        int i = i0 + j * NT + tid;
        i = i < tot ? i : 0;
        const int t = i / ppr, pc = i - t * ppr;
        if (p.row_ids) {
          const int64_t r = rid[t];
          v[j] = r >= 0 ? *reinterpret_cast<const i32x4*>(p.a + r * K + pc * 16) : i32x4{0, 0, 0, 0};
        } else {
          v[j] = *reinterpret_cast<const i32x4*>(arows + (int64_t)t * K + pc * 16);
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = i0 + j * NT + tid;
        if (i < tot) {
          const int t = i / ppr, pc = i - t * ppr;
          *reinterpret_cast<i32x4*>(xs + t * xstride + pc * 16) = v[j];
        }
      }
    }
    if (tid < mc) asl[tid] = p.row_ids ? (rid[tid] >= 0 ? p.as[rid[tid]] : 0.f) : p.as[start + m0 + tid];
    __syncthreads();

    i32x4 acc[MT][NB];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[mt][b] = i32x4{0, 0, 0, 0};
    for (int c0 = 0; c0 < C; c0 += W) {
#pragma unroll
      for (int u = 0; u < W; ++u) {
        const int c = c0 + u;
        if (c < C) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            if (mt * 16 < mc) {
#pragma unroll
              for (int j = 0; j < PL; ++j) {
                const i32x4 av = *reinterpret_cast<const i32x4*>(xs + (mt * 16 + col) * xstride + c * CB + lo + 16 * j);
#pragma unroll
                for (int b = 0; b < NB; ++b)
                  acc[mt][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, wv[u][b][j], acc[mt][b], 0, 0, 0);
              }
            }
          }
        }
        const int cn = min(c + W, C - 1);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
#pragma unroll
          for (int j = 0; j < PL; ++j) wv[u][b][j] = *reinterpret_cast<const i32x4*>(wr[b] + (int64_t)cn * CB + 16 * j);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    // lane l holds D[row 4(l >> 4) + r of the tile][column l & 15]
    if (live) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int ml = mt * 16 + 4 * q + r;
          if (ml >= mc) continue;
          const int64_t row = start + m0 + ml;
          const float a_s = asl[ml];
          if constexpr (P == 2) {
            const int no = n0 + col;
            if (no < p.N) {
              const float gv = mul_rn(mul_rn(static_cast<float>(acc[mt][0][r]), a_s), wsc[0]);
              const float uv = mul_rn(mul_rn(static_cast<float>(acc[mt][1][r]), a_s), wsc[1]);
              const float gt = bf16_bits_to_f32(f32_to_bf16_bits(gv));
              const float ut = bf16_bits_to_f32(f32_to_bf16_bits(uv));
              const float sl = bf16_bits_to_f32(f32_to_bf16_bits(silu_f(gt)));
              static_cast<uint16_t*>(p.out)[row * p.N + no] = f32_to_bf16_bits(mul_rn(sl, ut));
            }
          } else {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
              const int no = n0 + 16 * b + col;
              if (no < p.N) {
                const float v = mul_rn(mul_rn(static_cast<float>(acc[mt][b][r]), a_s), wsc[b]);
                if (p.out_dtype == QS_F32)
                  static_cast<float*>(p.out)[row * p.N + no] = v;
                else
                  static_cast<uint16_t*>(p.out)[row * p.N + no] = f32_to_bf16_bits(v);
              }
            }
          }
        }
      }
    }
    __syncthreads();  // the next pass overwrites the staged rows
  }
}

// W8A16 streaming grouped GEMM: k_moe_stream's walk (XCD-grouped row blocks, each wave
// streaming its weight rows over the full K through a window of W chunks in registers)
// with bf16 routed rows and no activation quantization.  Each weight piece is dequantized
// in registers to bf16(float(code) * w_scale[n]) (the W8A16 weight contract of the qrow
// path) and multiplied by v_mfma_f32_16x16x32_bf16 with fp32 accumulation: lane l's 16
// codes at k offset o of its weight row (l & 15) are the B operands of two MFMAs (codes
// o .. o + 7 and o + 8 .. o + 15), whose A operands are the same k elements of staged row
// (l & 15) of a 16-row tile.  The rows are staged in K phases of KPH elements (MC rows of
// KPH bf16 plus 16 bytes of pad in LDS), so every K fits: a phase boundary is a workgroup
// barrier and a restage while the weight window stays in flight.  KPH is a multiple of
// W chunks, so the window's register slot of chunk c stays c % W.  With row_ids, staged
// row r of the group is source row row_ids[start + r] (the reference's
// source.index_select(token_ids) folded into the staging); an id outside [0, src_rows)
// stages zeros.  A pass's ids are requested before its weight window and kept in LDS
// (after the staged rows), so no staging load waits on an id load.
struct MoeW16Params {
  const uint16_t* a;      // bf16 [src_rows or A, K]
  const int64_t* row_ids; // nullable gather of the routed rows
  int64_t src_rows;
  const int8_t* w;
  int64_t w_stride;       // bytes
  const float* ws;
  int64_t ws_stride;      // floats
  const int32_t* starts;
  const int32_t* counts;
  const int32_t* slots;   // nullable
  int N, K, KPH;
  void* out;
  int out_dtype;
};

template <int P, int NB, int MT, int W, int WAVES, int PAIR>
__global__ __launch_bounds__(WAVES * 64) void k_moe_stream_w16(MoeW16Params p) {
  static_assert(P == 1 || NB == 2, "SwiGLU streams the gate and up tiles of one row block");
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int MC = 16 * MT;
  constexpr int NT = WAVES * 64;
  constexpr int RW = MoeStreamCfg<P, NB>::RW;
  constexpr int CB = PAIR ? 128 : 64;  // codes of a weight row per chunk
  constexpr int PL = PAIR ? 2 : 1;     // 16-code pieces per lane per chunk
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, q = lane >> 4;
  const int total = gridDim.x * gridDim.y, lin = blockIdx.y * gridDim.x + blockIdx.x;
  const int per_xcd = total / 8;
  const int logical = lin < 8 * per_xcd ? (lin % 8) * per_xcd + lin / 8 : lin;
  const int g = logical / gridDim.x, bx = logical - g * gridDim.x;
  const GroupMeta gm = group_meta(p.counts, p.starts, p.slots, g);
  const int count = gm.count;
  if (count == 0) return;
  const int start = gm.start;
  const int slot = gm.slot;
  const int K = p.K, C = K / CB, KPH = p.KPH, CPH = KPH / CB;
  const int xstride = 2 * KPH + 16;  // bytes per staged row
  const int n0 = (bx * WAVES + wave) * RW;
  const bool live = n0 < p.N;
  const int lo = PAIR ? 32 * q : 16 * q;  // the lane's code offset within a chunk
  const int8_t* wexp = p.w + (int64_t)slot * p.w_stride;
  const int8_t* wr[NB];
  float wsc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int nb = P == 2 ? min(n0 + col, p.N - 1) + b * p.N : min(n0 + 16 * b + col, p.N - 1);
    wr[b] = wexp + (int64_t)nb * K + lo;
    wsc[b] = p.ws[(int64_t)slot * p.ws_stride + nb];
  }

  int64_t* rid = reinterpret_cast<int64_t*>(lds + MC * xstride);  // [MC] source rows, -1 = zeros
  // rows m0 .. m0 + mc of the group, elements k0 .. k0 + KPH (or K), 8 loads in flight
  auto stage = [&](int m0, int mc, int k0) {
    const int ppr = min(KPH, K - k0) >> 3;  // 16-byte pieces per staged row
    const int tot = mc * ppr;
    for (int i0 = 0; i0 < tot; i0 += 8 * NT) {
      i32x4 v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        int i = i0 + j * NT + tid;
        i = i < tot ? i : 0;
        const int t = i / ppr, pc = i - t * ppr;
        const int64_t r = p.row_ids ? rid[t] : start + m0 + t;
        v[j] = r >= 0 ? *reinterpret_cast<const i32x4*>(p.a + r * K + k0 + pc * 8) : i32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = i0 + j * NT + tid;
        if (i < tot) {
          const int t = i / ppr, pc = i - t * ppr;
          *reinterpret_cast<i32x4*>(lds + t * xstride + pc * 16) = v[j];
        }
      }
    }
  };

  for (int m0 = 0; m0 < count; m0 += MC) {
    const int mc = min(MC, count - m0);
    int64_t id = -1;
    if (p.row_ids && tid < mc) id = p.row_ids[start + m0 + tid];
    __builtin_amdgcn_sched_barrier(0);
    i32x4 wv[W][NB][PL];
#pragma unroll
    for (int u = 0; u < W; ++u) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int j = 0; j < PL; ++j)
          wv[u][b][j] = *reinterpret_cast<const i32x4*>(wr[b] + (int64_t)min(u, C - 1) * CB + 16 * j);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (p.row_ids) {
      if (tid < mc) rid[tid] = id >= 0 && id < p.src_rows ? id : -1;
      __syncthreads();
    }
    stage(m0, mc, 0);
    __syncthreads();

    f32x4 acc[MT][NB];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[mt][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    int cb = 0;  // first chunk of the staged phase
    for (int c0 = 0; c0 < C; c0 += W) {
      if (c0 - cb == CPH) {
        cb = c0;
        __syncthreads();  // every wave is done with the previous phase
        stage(m0, mc, cb * CB);
        __syncthreads();
      }
#pragma unroll
      for (int u = 0; u < W; ++u) {
        const int c = c0 + u;
        if (c < C) {
          const uint8_t* xa = lds + col * xstride + 2 * ((c - cb) * CB + lo);
#pragma unroll
          for (int j = 0; j < PL; ++j) {
            bf16x8 wb[NB][2];
#pragma unroll
            for (int b = 0; b < NB; ++b) deq16_bf16(wv[u][b][j], wsc[b], wb[b][0], wb[b][1]);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              if (mt * 16 < mc) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                  const bf16x8 av = *reinterpret_cast<const bf16x8*>(xa + mt * 16 * xstride + 32 * j + 16 * h);
#pragma unroll
                  for (int b = 0; b < NB; ++b)
                    acc[mt][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, wb[b][h], acc[mt][b], 0, 0, 0);
                }
              }
            }
          }
        }
        const int cn = min(c + W, C - 1);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
#pragma unroll
          for (int j = 0; j < PL; ++j) wv[u][b][j] = *reinterpret_cast<const i32x4*>(wr[b] + (int64_t)cn * CB + 16 * j);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    // lane l holds D[row 4(l >> 4) + r of the tile][column l & 15]
    if (live) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int ml = mt * 16 + 4 * q + r;
          if (ml >= mc) continue;
          const int64_t row = start + m0 + ml;
          if constexpr (P == 2) {
            const int no = n0 + col;
            if (no < p.N) {
              const float gt = bf16_bits_to_f32(f32_to_bf16_bits(acc[mt][0][r]));
              const float ut = bf16_bits_to_f32(f32_to_bf16_bits(acc[mt][1][r]));
              const float sl = bf16_bits_to_f32(f32_to_bf16_bits(silu_f(gt)));
              static_cast<uint16_t*>(p.out)[row * p.N + no] = f32_to_bf16_bits(mul_rn(sl, ut));
            }
          } else {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
              const int no = n0 + 16 * b + col;
              if (no < p.N) {
                if (p.out_dtype == QS_F32)
                  static_cast<float*>(p.out)[row * p.N + no] = acc[mt][b][r];
                else
                  static_cast<uint16_t*>(p.out)[row * p.N + no] = f32_to_bf16_bits(acc[mt][b][r]);
              }
            }
          }
        }
      }
    }
    __syncthreads();  // the next pass overwrites the staged rows
  }
}

// ----------------------------------------------------------------------------------
// stable rank-order reduce
// ----------------------------------------------------------------------------------
template <int YT, int OT>
__global__ __launch_bounds__(256) void k_moe_reduce(const void* __restrict__ y,
                                                    const float* __restrict__ coef,
                                                    const int64_t* __restrict__ inv, int k,
                                                    int H, void* __restrict__ out) {
  const int64_t t = blockIdx.x;
  const int h = blockIdx.y * 256 + threadIdx.x;
  if (h >= H) return;
  float acc = 0.f;
  for (int r = 0; r < k; ++r) {
    const int64_t a = inv[t * k + r];
    // a < 0: the route compiler dropped this rank (expert out of range); it adds nothing
    const float c = a < 0 ? 0.f : mul_rn(ld<YT>(y, a * H + h), coef[a]);
    acc = r == 0 ? c : add_rn(acc, c);
  }
  if constexpr (OT == QS_F32) static_cast<float*>(out)[t * H + h] = acc;
  else static_cast<uint16_t*>(out)[t * H + h] = f32_to_bf16_bits(acc);
}

// Eight consecutive h per thread (16- or 32-byte loads of y), one token per blockIdx.x;
// the same products, sums and order as k_moe_reduce.  OT = BF16 rounds the fp32 sum once
// (RNE), which is the fp32 reduce followed by a cast to bf16.
template <int YT, int OT>
__global__ __launch_bounds__(256) void k_moe_reduce8(const void* __restrict__ y,
                                                     const float* __restrict__ coef,
                                                     const int64_t* __restrict__ inv, int k,
                                                     int H, void* __restrict__ out) {
  const int64_t t = blockIdx.x;
  const int h0 = (blockIdx.y * 256 + threadIdx.x) * 8;
  if (h0 >= H) return;
  float acc[8];
  // ranks in batches of 8: every row of a batch is requested before the first is used
  constexpr int RB = 8;
  for (int r0 = 0; r0 < k; r0 += RB) {
    int64_t a[RB];
    float cf[RB];
    Piece8<YT> pc[RB];
#pragma unroll
    for (int j = 0; j < RB; ++j) a[j] = r0 + j < k ? inv[t * k + r0 + j] : -1;
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      if (a[j] >= 0) {
        cf[j] = coef[a[j]];
        pc[j].load(static_cast<const char*>(y) + (a[j] * H + h0) * (YT == QS_F32 ? 4 : 2));
      }
    }
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      if (r0 + j >= k) break;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // a negative inverse entry: the route compiler dropped this rank, it adds 0
        const float c = a[j] < 0 ? 0.f : mul_rn(pc[j].at(e), cf[j]);
        acc[e] = r0 + j == 0 ? c : add_rn(acc[e], c);
      }
    }
  }
  if constexpr (OT == QS_F32) {
    float* o = static_cast<float*>(out) + t * H + h0;
    *reinterpret_cast<f32x4*>(o) = f32x4{acc[0], acc[1], acc[2], acc[3]};
    *reinterpret_cast<f32x4*>(o + 4) = f32x4{acc[4], acc[5], acc[6], acc[7]};
  } else {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = static_cast<uint32_t>(f32_to_bf16_bits(acc[2 * e])) | (static_cast<uint32_t>(f32_to_bf16_bits(acc[2 * e + 1])) << 16);
    *reinterpret_cast<i32x4*>(static_cast<uint16_t*>(out) + t * H + h0) =
        i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
  }
}

}  // namespace qs

using namespace qs;

extern "C" int qs_moe_router(const void* logits, int logit_dtype, int64_t T, int E, int k,
                             int norm_topk, int64_t* top_idx, void* top_w, int w_dtype,
                             void* stream) {
  if (!logits || !top_idx || !top_w) return fail(QS_ERR_INVALID, "moe_router: null pointer");
  if (T < 0 || E < 1 || E > 1024 || k < 1 || k > 16 || k > E)
    return fail(QS_ERR_LIMIT, "moe_router: need 1 <= E <= 1024, 1 <= k <= min(16, E)");
  if (w_dtype != QS_F32 && w_dtype != QS_BF16) return fail(QS_ERR_INVALID, "moe_router: weight dtype F32 or BF16");
  if (T == 0) return QS_OK;
  if (logit_dtype != QS_F32 && logit_dtype != QS_BF16) return fail(QS_ERR_INVALID, "moe_router: logits F32 or BF16");
  if (T > (int64_t)INT32_MAX) return fail(QS_ERR_LIMIT, "moe_router: too many tokens");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned blocks = (unsigned)cdiv(T, 4);
#define QS_ROUTER(J)                                                                                        \
  do {                                                                                                      \
    if (logit_dtype == QS_F32)                                                                              \
      hipLaunchKernelGGL((k_moe_router<QS_F32, J>), dim3(blocks), dim3(256), 0, s, logits, (int)T, E, k,    \
                         norm_topk, top_idx, top_w, w_dtype);                                               \
    else                                                                                                    \
      hipLaunchKernelGGL((k_moe_router<QS_BF16, J>), dim3(blocks), dim3(256), 0, s, logits, (int)T, E, k,   \
                         norm_topk, top_idx, top_w, w_dtype);                                               \
  } while (0)
  if (E <= 64) QS_ROUTER(1);
  else if (E <= 128) QS_ROUTER(2);
  else if (E <= 256) QS_ROUTER(4);
  else if (E <= 512) QS_ROUTER(8);
  else QS_ROUTER(16);
#undef QS_ROUTER
  return hip_check(hipGetLastError(), "k_moe_router launch");
}

extern "C" int qs_moe_route(const void* top_idx, int idx_dtype, const void* top_w, int w_dtype,
                            int64_t T, int k, int E, int64_t* token_ids, float* coef,
                            int32_t* starts, int32_t* counts, int64_t* inverse, void* stream) {
  if (!top_idx || !top_w || !token_ids || !coef || !starts || !counts)
    return fail(QS_ERR_INVALID, "moe_route: null pointer");
  if (T < 0 || k < 1 || E < 1) return fail(QS_ERR_INVALID, "moe_route: bad shape");
  if (E > kRouteMaxE) return fail(QS_ERR_LIMIT, "moe_route: at most %d experts", kRouteMaxE);
  if (T * k > (int64_t)1 << 28) return fail(QS_ERR_LIMIT, "moe_route: too many assignments");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int A = (int)(T * k);
  // one workgroup per expert while the E re-reads of the A expert ids stay small (they
  // come from L2); a single workgroup otherwise
  const bool par = (int64_t)A * E <= ((int64_t)1 << 22);
#define QS_ROUTE(IT, WT)                                                                              \
  do {                                                                                                \
    if (par)                                                                                          \
      hipLaunchKernelGGL((k_moe_route_par<IT, WT>), dim3(E), dim3(kParWaves * 64), 0, s, top_idx, top_w, \
                         A, k, E, token_ids, coef, starts, counts, inverse);                          \
    else                                                                                              \
      hipLaunchKernelGGL((k_moe_route<IT, WT>), dim3(1), dim3(1024), 0, s, top_idx, top_w, A, k, E,   \
                         token_ids, coef, starts, counts, inverse);                                   \
  } while (0)
  if (idx_dtype == QS_I64 && w_dtype == QS_F32) QS_ROUTE(QS_I64, QS_F32);
  else if (idx_dtype == QS_I64 && w_dtype == QS_BF16) QS_ROUTE(QS_I64, QS_BF16);
  else if (idx_dtype == QS_I32 && w_dtype == QS_F32) QS_ROUTE(QS_I32, QS_F32);
  else if (idx_dtype == QS_I32 && w_dtype == QS_BF16) QS_ROUTE(QS_I32, QS_BF16);
  else return fail(QS_ERR_INVALID, "moe_route: indices I32/I64, weights F32/BF16");
#undef QS_ROUTE
  return hip_check(hipGetLastError(), "k_moe_route launch");
}

extern "C" int qs_moe_route_quant(const void* top_idx, int idx_dtype, const void* top_w, int w_dtype,
                                  int64_t T, int k, int E, int64_t* token_ids, float* coef, int32_t* starts,
                                  int32_t* counts, int64_t* inverse, const void* source, int src_dtype,
                                  int64_t ld_src, int64_t H, int8_t* q, float* scale, void* stream) {
  if (!top_idx || !top_w || !token_ids || !coef || !starts || !counts || !source || !q || !scale)
    return fail(QS_ERR_INVALID, "moe_route_quant: null pointer");
  if (T < 0 || k < 1 || E < 1 || H <= 0 || ld_src < H) return fail(QS_ERR_INVALID, "moe_route_quant: bad shape");
  if (E > kRouteMaxE) return fail(QS_ERR_LIMIT, "moe_route_quant: at most %d experts", kRouteMaxE);
  if (T * k > (int64_t)1 << 28 || H > INT32_MAX) return fail(QS_ERR_LIMIT, "moe_route_quant: too many assignments");
  if (src_dtype != QS_BF16 && src_dtype != QS_F32) return fail(QS_ERR_INVALID, "moe_route_quant: source F32 or BF16");
  const int A = (int)(T * k);
  const int64_t esize = src_dtype == QS_F32 ? 4 : 2;
  const bool fused = (int64_t)A * E <= ((int64_t)1 << 22) && H % 8 == 0 && aligned(source, 16) &&
                     (ld_src * esize) % 16 == 0 && aligned(q, 8) && T > 0;
  if (!fused) {
    const int st = qs_moe_route(top_idx, idx_dtype, top_w, w_dtype, T, k, E, token_ids, coef, starts, counts,
                                inverse, stream);
    if (st) return st;
    return qs_moe_gather_quant(source, src_dtype, ld_src, nullptr, T, H, q, scale, stream);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(E + cdiv(T, kParWaves)));
#define QS_RQ(IT, WT)                                                                                    \
  do {                                                                                                   \
    if (src_dtype == QS_BF16)                                                                            \
      hipLaunchKernelGGL((k_moe_route_quant<IT, WT, QS_BF16>), grid, dim3(kParWaves * 64), 0, s, top_idx,  \
                         top_w, A, k, E, token_ids, coef, starts, counts, inverse, source, ld_src, T,      \
                         (int)H, q, scale);                                                              \
    else                                                                                                 \
      hipLaunchKernelGGL((k_moe_route_quant<IT, WT, QS_F32>), grid, dim3(kParWaves * 64), 0, s, top_idx,   \
                         top_w, A, k, E, token_ids, coef, starts, counts, inverse, source, ld_src, T,      \
                         (int)H, q, scale);                                                              \
  } while (0)
  if (idx_dtype == QS_I64 && w_dtype == QS_F32) QS_RQ(QS_I64, QS_F32);
  else if (idx_dtype == QS_I64 && w_dtype == QS_BF16) QS_RQ(QS_I64, QS_BF16);
  else if (idx_dtype == QS_I32 && w_dtype == QS_F32) QS_RQ(QS_I32, QS_F32);
  else if (idx_dtype == QS_I32 && w_dtype == QS_BF16) QS_RQ(QS_I32, QS_BF16);
  else return fail(QS_ERR_INVALID, "moe_route_quant: indices I32/I64, weights F32/BF16");
#undef QS_RQ
  return hip_check(hipGetLastError(), "k_moe_route_quant launch");
}

extern "C" int qs_moe_gather_quant(const void* source, int src_dtype, int64_t ld_src,
                                   const int64_t* rows, int64_t A, int64_t H, int8_t* q,
                                   float* scale, void* stream) {
  if (!source || !q || !scale) return fail(QS_ERR_INVALID, "moe_gather_quant: null pointer");
  if (A < 0 || H <= 0 || ld_src < H) return fail(QS_ERR_INVALID, "moe_gather_quant: bad shape");
  if (A == 0) return QS_OK;
  if (src_dtype != QS_BF16 && src_dtype != QS_F32) return fail(QS_ERR_INVALID, "moe_gather_quant: source F32 or BF16");
  if (H > INT32_MAX) return fail(QS_ERR_LIMIT, "moe_gather_quant: H too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t esize = src_dtype == QS_F32 ? 4 : 2;
  if (H % 8 == 0 && aligned(source, 16) && (ld_src * esize) % 16 == 0 && aligned(q, 8)) {
    const dim3 grid((unsigned)cdiv(A, 4));
    if (src_dtype == QS_BF16)
      hipLaunchKernelGGL(k_moe_gather_quant8<QS_BF16>, grid, dim3(256), 0, s, source, ld_src, rows, A, (int)H, q, scale);
    else
      hipLaunchKernelGGL(k_moe_gather_quant8<QS_F32>, grid, dim3(256), 0, s, source, ld_src, rows, A, (int)H, q, scale);
    return hip_check(hipGetLastError(), "k_moe_gather_quant8 launch");
  }
  if (A > INT32_MAX) return fail(QS_ERR_LIMIT, "moe_gather_quant: too many rows for the unaligned path");
  if (src_dtype == QS_BF16)
    hipLaunchKernelGGL(k_moe_gather_quant<QS_BF16>, dim3((unsigned)A), dim3(256), 0, s, source, ld_src, rows, (int)H, q, scale);
  else
    hipLaunchKernelGGL(k_moe_gather_quant<QS_F32>, dim3((unsigned)A), dim3(256), 0, s, source, ld_src, rows, (int)H, q, scale);
  return hip_check(hipGetLastError(), "k_moe_gather_quant launch");
}

namespace {
constexpr int kMoeTilesPerBlock = 1;  // 16-row tiles per workgroup, streamed back to back
constexpr size_t kMoeStreamLds = 144 * 1024;  // staged routed rows of k_moe_stream

template <int P, int KW>
void launch_moe_gemm(const MoeGemmParams& p, int G, hipStream_t s) {
  const int C = p.K / 64;
  const int ch = (C + KW - 1) / KW;
  constexpr int NT = kMoeTilesPerBlock;
  dim3 grid((unsigned)cdiv(cdiv(p.N, 16), NT), (unsigned)G);
  if (ch <= 2) hipLaunchKernelGGL((k_moe_gemm<P, KW, 2, NT>), grid, dim3(P * KW * 64), 0, s, p);
  else if (ch <= 4) hipLaunchKernelGGL((k_moe_gemm<P, KW, 4, NT>), grid, dim3(P * KW * 64), 0, s, p);
  else if (ch <= 8) hipLaunchKernelGGL((k_moe_gemm<P, KW, 8, NT>), grid, dim3(P * KW * 64), 0, s, p);
  else hipLaunchKernelGGL((k_moe_gemm<P, KW, 16, NT>), grid, dim3(P * KW * 64), 0, s, p);
}

// LDS bytes of k_moe_stream for MT row tiles; 0 when it does not fit.
size_t moe_stream_lds(int MT, int64_t K) {
  const size_t b = (size_t)16 * MT * (size_t)(K + 16) + (size_t)16 * MT * (4 + 8);
  return b <= kMoeStreamLds ? b : 0;
}

// Launch shapes measured on config-4 shapes (E 128, H 2048, I 768, T 64 / 512):
// SwiGLU streams with 4 waves when one row tile is staged (T = 64: 70 us vs 76 us with 8),
// 8 waves for two and 12 for four; two 128-byte chunks in flight.  Plain products keep 128 bytes
// of each weight row in flight for NB >= 2 tiles per wave, 256 for one.
template <int P, int NB, int MT, int PAIR, int WAVES_SET = 0>
void launch_moe_stream_mt(const MoeGemmParams& p, int G, hipStream_t s) {
  // SwiGLU with 64-row passes: 12 waves (N = 768: four workgroups per expert, two full
  // rounds of the CUs at 128 experts; T = 512 gate/up 85.3 -> 82.6 us against 8 waves)
  constexpr int WAVES = WAVES_SET ? WAVES_SET : (P == 2 ? (MT == 1 ? 4 : (MT == 4 ? 12 : 8)) : 4);
  constexpr int WP = P == 2 ? 2 : (NB >= 2 ? 1 : 2);  // 128-byte chunks in flight
  constexpr int W = PAIR ? WP : 2 * WP;
  constexpr int RW = MoeStreamCfg<P, NB>::RW;
  const dim3 grid((unsigned)cdiv(p.N, RW * WAVES), (unsigned)G), block(WAVES * 64);
  hipLaunchKernelGGL((k_moe_stream<P, NB, MT, W, WAVES, PAIR>), grid, block, moe_stream_lds(MT, p.K), s, p);
}

template <int P, int NB>
void launch_moe_stream(const MoeGemmParams& p, int G, int MT, hipStream_t s) {
  if (p.K % 128 == 0) {
    if (MT == 4) launch_moe_stream_mt<P, NB, 4, 1>(p, G, s);
    else if (MT == 2) launch_moe_stream_mt<P, NB, 2, 1>(p, G, s);
    else launch_moe_stream_mt<P, NB, 1, 1>(p, G, s);
  } else {
    if (MT == 4) launch_moe_stream_mt<P, NB, 4, 0>(p, G, s);
    else if (MT == 2) launch_moe_stream_mt<P, NB, 2, 0>(p, G, s);
    else launch_moe_stream_mt<P, NB, 1, 0>(p, G, s);
  }
}
// K phase of k_moe_stream_w16: the whole K when MC staged rows fit kMoeStreamLds, else
// the fewest phases of a multiple of W chunks each that fit.
int moe_w16_phase(int MT, int64_t K, int CB, int W, size_t cap) {
  const int64_t C = K / CB;
  for (int64_t kp = 1; kp <= C; ++kp) {
    const int64_t cph = kp == 1 ? C : cdiv(cdiv(C, kp), W) * W;
    if ((size_t)16 * MT * (size_t)(2 * cph * CB + 16 + 8) <= cap) return (int)(cph * CB);
  }
  return 0;
}

// Launch shapes of k_moe_stream_w16, measured on config-4 shapes (E 128, H 2048, I 768):
// SwiGLU with 8 waves for one or two row tiles and 12 for four (two 128-byte chunks in
// flight).  Plain products with 64-row passes (MT = 4) use 4 waves of NB tiles and cap the
// staged slice at 72 KB so that two or three workgroups share a CU (T = 512 down
// 74 -> 51 us); shorter passes use 8 waves of at most 2 tiles (T = 64 down 41 -> 36 us).
// The dequantization costs 2.5 VALU operations per code, so the stream needs more waves
// per SIMD than the int8 one to keep its loads in flight.
template <int P, int NB, int MT, int PAIR, int WAVES>
void launch_moe_w16_mt(MoeW16Params p, int G, size_t cap, hipStream_t s) {
  constexpr int WP = P == 2 ? 2 : (NB >= 2 ? 1 : 2);  // w16 chunks in flight
  constexpr int W = PAIR ? WP : 2 * WP;
  constexpr int RW = MoeStreamCfg<P, NB>::RW;
  p.KPH = moe_w16_phase(MT, p.K, PAIR ? 128 : 64, W, cap);
  const size_t lds = (size_t)16 * MT * (size_t)(2 * p.KPH + 16 + 8);  // staged rows + their ids
  const dim3 grid((unsigned)cdiv(p.N, RW * WAVES), (unsigned)G), block(WAVES * 64);
  hipLaunchKernelGGL((k_moe_stream_w16<P, NB, MT, W, WAVES, PAIR>), grid, block, lds, s, p);
}

template <int P, int NB, int MT, int WAVES>
void launch_moe_w16_pair(const MoeW16Params& p, int G, size_t cap, hipStream_t s) {
  if (p.K % 128 == 0) launch_moe_w16_mt<P, NB, MT, 1, WAVES>(p, G, cap, s);
  else launch_moe_w16_mt<P, NB, MT, 0, WAVES>(p, G, cap, s);
}

void launch_moe_w16(const MoeW16Params& p, int G, int MT, bool swiglu, hipStream_t s) {
  const int64_t K = p.K;
  if (swiglu) {
    if (MT == 4) launch_moe_w16_pair<2, 2, 4, 12>(p, G, kMoeStreamLds, s);  // 102.1 -> 91.2 us at T = 512 (8 waves)
    else if (MT == 2) launch_moe_w16_pair<2, 2, 2, 8>(p, G, kMoeStreamLds, s);
    else launch_moe_w16_pair<2, 2, 1, 8>(p, G, kMoeStreamLds, s);  // T = 64 layer 128.8 -> 125.3 us (4 waves)
  } else if (MT == 4) {
    constexpr size_t cap = 72 * 1024;
    if (K <= 1024) launch_moe_w16_pair<1, 4, 4, 4>(p, G, cap, s);
    else if (K <= 2048) launch_moe_w16_pair<1, 2, 4, 4>(p, G, cap, s);
    else launch_moe_w16_pair<1, 1, 4, 4>(p, G, cap, s);
  } else if (MT == 2) {
    if (K <= 2048) launch_moe_w16_pair<1, 2, 2, 8>(p, G, kMoeStreamLds, s);
    else launch_moe_w16_pair<1, 1, 2, 8>(p, G, kMoeStreamLds, s);
  } else {
    if (K <= 2048) launch_moe_w16_pair<1, 2, 1, 8>(p, G, kMoeStreamLds, s);
    else launch_moe_w16_pair<1, 1, 1, 8>(p, G, kMoeStreamLds, s);
  }
}
}  // namespace

extern "C" int qs_moe_grouped_gemm_w8a16(const void* a, const int64_t* row_ids, int64_t src_rows,
                                         const int8_t* w, int64_t w_stride, const float* w_scale,
                                         int64_t ws_stride, const int32_t* starts, const int32_t* counts,
                                         const int32_t* slots, int G, int64_t N, int64_t K,
                                         int64_t max_rows, int swiglu, void* out, int out_dtype,
                                         void* stream) {
  if (!a || !w || !w_scale || !starts || !counts || !out)
    return fail(QS_ERR_INVALID, "moe_grouped_gemm_w8a16: null pointer");
  if (G < 1 || G > 65535 || N <= 0 || K <= 0 || src_rows < 0)
    return fail(QS_ERR_INVALID, "moe_grouped_gemm_w8a16: bad shape");
  if (N > (1 << 30) || K > (1 << 20)) return fail(QS_ERR_LIMIT, "moe_grouped_gemm_w8a16: N or K too large");
  if (K % 64 != 0) return fail(QS_ERR_UNSUPPORTED, "moe_grouped_gemm_w8a16: K must be a multiple of 64");
  if (!aligned(a, 16) || !aligned(w, 16) || w_stride % 16 != 0)
    return fail(QS_ERR_UNSUPPORTED, "moe_grouped_gemm_w8a16: operands must be 16-byte aligned");
  if (swiglu && out_dtype != QS_BF16) return fail(QS_ERR_INVALID, "moe_grouped_gemm_w8a16: SwiGLU output is BF16");
  if (out_dtype != QS_BF16 && out_dtype != QS_F32)
    return fail(QS_ERR_INVALID, "moe_grouped_gemm_w8a16: out F32 or BF16");
  if (max_rows < 0) return fail(QS_ERR_INVALID, "moe_grouped_gemm_w8a16: max_rows must be >= 0");
  if (src_rows > (int64_t)1 << 40) return fail(QS_ERR_LIMIT, "moe_grouped_gemm_w8a16: src_rows too large");
  MoeW16Params p{static_cast<const uint16_t*>(a), row_ids, src_rows, w, w_stride, w_scale, ws_stride,
                 starts, counts, slots, (int)N, (int)K, 0, out, out_dtype};
  hipStream_t s = static_cast<hipStream_t>(stream);
  // row tiles sized for twice the mean rows per group, as the int8 stream
  const int64_t mean = max_rows > 0 ? cdiv(max_rows, G) : 16;
  const int MT = 2 * mean <= 16 ? 1 : (2 * mean <= 32 ? 2 : 4);
  launch_moe_w16(p, G, MT, swiglu != 0, s);
  return hip_check(hipGetLastError(), "k_moe_stream_w16 launch");
}

namespace {
int grouped_gemm_i8(const int8_t* a, const float* a_scale, const int64_t* row_ids, int64_t src_rows,
                    const int8_t* w, int64_t w_stride, const float* w_scale, int64_t ws_stride,
                    const int32_t* starts, const int32_t* counts, const int32_t* slots, int G, int64_t N,
                    int64_t K, int64_t max_rows, int swiglu, void* out, int out_dtype, void* stream) {
  if (!a || !a_scale || !w || !w_scale || !starts || !counts || !out)
    return fail(QS_ERR_INVALID, "moe_grouped_gemm: null pointer");
  if (G < 1 || G > 65535 || N <= 0 || K <= 0) return fail(QS_ERR_INVALID, "moe_grouped_gemm: bad shape");
  if (K % 64 != 0 || K > (swiglu ? 8192 : 16384))
    return fail(QS_ERR_UNSUPPORTED, "moe_grouped_gemm: K must be a multiple of 64, <= 8192 (SwiGLU) / 16384");
  if (!aligned(a, 16) || !aligned(w, 16) || w_stride % 16 != 0)
    return fail(QS_ERR_UNSUPPORTED, "moe_grouped_gemm: operands must be 16-byte aligned");
  if (swiglu && out_dtype != QS_BF16) return fail(QS_ERR_INVALID, "moe_grouped_gemm: SwiGLU output is BF16");
  if (out_dtype != QS_BF16 && out_dtype != QS_F32) return fail(QS_ERR_INVALID, "moe_grouped_gemm: out F32 or BF16");
  if (max_rows < 0) return fail(QS_ERR_INVALID, "moe_grouped_gemm: max_rows must be >= 0");
  if (src_rows < 0) return fail(QS_ERR_INVALID, "moe_grouped_gemm: src_rows must be >= 0");
  MoeGemmParams p{a, a_scale, w, w_stride, w_scale, ws_stride, starts, counts, slots, (int)N, (int)K, out, out_dtype,
                  row_ids, src_rows};
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Streaming kernel: row tiles sized for twice the mean rows per group (max_rows / G),
  // so that most groups take one pass over their weights; 0 = unknown -> 2 tiles.
  const int64_t mean = max_rows > 0 ? cdiv(max_rows, G) : 16;
  int MT = 2 * mean <= 16 ? 1 : (2 * mean <= 32 ? 2 : 4);
  while (MT > 1 && !moe_stream_lds(MT, K)) MT /= 2;
  // The K-split kernel only takes K beyond what the staged row tile fits in LDS (with
  // 128-byte chunk loads the stream also beats it on short groups: T = 64 down 50 -> 42 us).
  if (moe_stream_lds(MT, K)) {
    // plain: row tiles per wave so that a wave streams about 48 KB or more
    if (swiglu) launch_moe_stream<2, 2>(p, G, MT, s);
    else if (K <= 1024 && MT == 4) {
      // 64-row passes of short rows (T = 512 down): 8 waves of two tiles (43.0 -> 40.0 us;
      // shorter passes keep 4 waves of four tiles: T = 64 down 34.2 against 35.4)
      if (K % 128 == 0) launch_moe_stream_mt<1, 2, 4, 1, 8>(p, G, s);
      else launch_moe_stream_mt<1, 2, 4, 0, 8>(p, G, s);
    } else if (K <= 1024) launch_moe_stream<1, 4>(p, G, MT, s);
    else if (K <= 2048) launch_moe_stream<1, 2>(p, G, MT, s);
    else launch_moe_stream<1, 1>(p, G, MT, s);
    return hip_check(hipGetLastError(), "k_moe_stream launch");
  }
  if (row_ids)
    return fail(QS_ERR_UNSUPPORTED, "moe_grouped_gemm: row_ids need the streaming kernel (16 staged rows of K + 28 "
                "bytes within %d bytes of LDS)", (int)kMoeStreamLds);
  const int C = (int)(K / 64);
  // K split so that each wave holds at most 16 chunks of 64 k of its tile (<= 1024 threads)
  if (swiglu) {
    if (C <= 32) launch_moe_gemm<2, 4>(p, G, s);
    else launch_moe_gemm<2, 8>(p, G, s);
  } else {
    if (C <= 32) launch_moe_gemm<1, 4>(p, G, s);
    else if (C <= 128) launch_moe_gemm<1, 8>(p, G, s);
    else launch_moe_gemm<1, 16>(p, G, s);
  }
  return hip_check(hipGetLastError(), "k_moe_gemm launch");
}
}  // namespace

extern "C" int qs_moe_grouped_gemm_i8(const int8_t* a, const float* a_scale, const int8_t* w,
                                      int64_t w_stride, const float* w_scale, int64_t ws_stride,
                                      const int32_t* starts, const int32_t* counts,
                                      const int32_t* slots, int G, int64_t N, int64_t K,
                                      int64_t max_rows, int swiglu, void* out, int out_dtype,
                                      void* stream) {
  return grouped_gemm_i8(a, a_scale, nullptr, 0, w, w_stride, w_scale, ws_stride, starts, counts, slots, G, N, K,
                         max_rows, swiglu, out, out_dtype, stream);
}

extern "C" int qs_moe_grouped_gemm_i8_rows(const int8_t* a, const float* a_scale, const int64_t* row_ids,
                                           int64_t src_rows, const int8_t* w, int64_t w_stride,
                                           const float* w_scale, int64_t ws_stride, const int32_t* starts,
                                           const int32_t* counts, const int32_t* slots, int G, int64_t N,
                                           int64_t K, int64_t max_rows, int swiglu, void* out, int out_dtype,
                                           void* stream) {
  if (!row_ids) return fail(QS_ERR_INVALID, "moe_grouped_gemm_rows: null row_ids");
  return grouped_gemm_i8(a, a_scale, row_ids, src_rows, w, w_stride, w_scale, ws_stride, starts, counts, slots, G,
                         N, K, max_rows, swiglu, out, out_dtype, stream);
}

extern "C" int qs_moe_route_reduce_to(const void* expert_out, int y_dtype, const float* coef,
                                      const int64_t* inverse, int64_t T, int k, int64_t H,
                                      void* out, int out_dtype, void* stream) {
  if (!expert_out || !coef || !inverse || !out) return fail(QS_ERR_INVALID, "moe_route_reduce: null pointer");
  if (T < 0 || k < 1 || H <= 0) return fail(QS_ERR_INVALID, "moe_route_reduce: bad shape");
  if (T > INT32_MAX || H > 65535 * 256) return fail(QS_ERR_LIMIT, "moe_route_reduce: T or H too large");
  if (y_dtype != QS_BF16 && y_dtype != QS_F32) return fail(QS_ERR_INVALID, "moe_route_reduce: expert output F32 or BF16");
  if (out_dtype != QS_BF16 && out_dtype != QS_F32) return fail(QS_ERR_INVALID, "moe_route_reduce: out F32 or BF16");
  if (T == 0) return QS_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (H % 8 == 0 && aligned(expert_out, 16) && aligned(out, 16)) {
    const dim3 grid((unsigned)T, (unsigned)cdiv(H, 2048));
#define QS_RED8(YT, OT) hipLaunchKernelGGL((k_moe_reduce8<YT, OT>), grid, dim3(256), 0, s, expert_out, coef, inverse, k, (int)H, out)
    if (y_dtype == QS_BF16 && out_dtype == QS_F32) QS_RED8(QS_BF16, QS_F32);
    else if (y_dtype == QS_BF16) QS_RED8(QS_BF16, QS_BF16);
    else if (out_dtype == QS_F32) QS_RED8(QS_F32, QS_F32);
    else QS_RED8(QS_F32, QS_BF16);
#undef QS_RED8
    return hip_check(hipGetLastError(), "k_moe_reduce8 launch");
  }
  const dim3 grid((unsigned)T, (unsigned)cdiv(H, 256));
#define QS_RED(YT, OT) hipLaunchKernelGGL((k_moe_reduce<YT, OT>), grid, dim3(256), 0, s, expert_out, coef, inverse, k, (int)H, out)
  if (y_dtype == QS_BF16 && out_dtype == QS_F32) QS_RED(QS_BF16, QS_F32);
  else if (y_dtype == QS_BF16) QS_RED(QS_BF16, QS_BF16);
  else if (out_dtype == QS_F32) QS_RED(QS_F32, QS_F32);
  else QS_RED(QS_F32, QS_BF16);
#undef QS_RED
  return hip_check(hipGetLastError(), "k_moe_reduce launch");
}

extern "C" int qs_moe_route_reduce(const void* expert_out, int y_dtype, const float* coef,
                                   const int64_t* inverse, int64_t T, int k, int64_t H,
                                   float* out, void* stream) {
  return qs_moe_route_reduce_to(expert_out, y_dtype, coef, inverse, T, k, H, out, QS_F32, stream);
}
