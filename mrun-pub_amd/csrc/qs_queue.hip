// Expert-major packet queues (the Expert Exchange contract) on gfx950.
//
// Kernels
//   k_queue_build   : one workgroup of 1024 threads compiles A router packets into
//                     expert-major ranges in STABLE order (a packet's rank among the
//                     earlier packets of its expert comes from wave ballots), so the queue
//                     equals a stable sort by expert, identical on every call.  Each packet
//                     carries its token, route slot, fp32 coefficient and its row's epoch and
//                     deadline.  A packet whose expert lies outside [0, E) is left out; the
//                     queue rows it frees at the end get token 0, expert -1, slot -1 and epoch
//                     INT64_MIN.
//   k_fill_i32      : fills an int32 array (in place of a memset, so that graph capture
//                     records a kernel node).
//   scatter         : a stable counting sort of the valid packets by token, then a reduce.
//                     valid[q] = (token in [0, rows) and epoch[q] == active[token[q]]), as the
//                     reference's index_add_ counts them (by token alone, whatever the route
//                     slot); k_scatter_count counts each row's valid packets,
//                     k_scan_exclusive turns the counts into row ranges, k_scatter_place drops
//                     each packet into its row's range, k_scatter_rank re-orders every range
//                     by ascending queue index (a packet's rank = the number of smaller indices
//                     in its range), and k_scatter_reduce sums each row's range in that order
//                     as acc = acc + fp32(float(y[q]) * coef[q]) from acc = 0 -- the order and
//                     roundings of the reference's index_add_ -- with no atomics in the sum,
//                     so the result is the same on every call.  Rows are a grid-stride loop.
#include "qs_common.h"

#include <limits.h>

namespace qs {
namespace {

constexpr int kQueueWaves = 16;
constexpr int kQueueMaxE = 512;

template <int IT>
__device__ __forceinline__ int64_t ld_index(const void* p, int64_t i) {
  if constexpr (IT == QS_I64) return static_cast<const int64_t*>(p)[i];
  else return static_cast<const int32_t*>(p)[i];
}

template <int WT>
__device__ __forceinline__ float ld_weight(const void* p, int64_t i) {
  if constexpr (WT == QS_F32) return static_cast<const float*>(p)[i];
  else if constexpr (WT == QS_BF16) return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  else return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}

struct QueueBuildArgs {
  const void* experts;       // [A] I32/I64
  const int64_t* tokens;     // [A] or null: packet a belongs to row a / top_k
  const int64_t* slots;      // [A] or null: route slot a % top_k
  const void* weights;       // [A] F32/BF16/F16
  const int64_t* row_epochs;     // [rows]
  const int64_t* row_deadlines;  // [rows]
  int A, top_k, E;
  int64_t rows;
  int64_t* token_ids;
  int64_t* expert_ids;
  int64_t* route_slots;
  float* coefficients;
  int64_t* epochs;
  int64_t* deadlines;
  void* starts;
  void* counts;
  bool counts_i64;
};

template <int IT, int WT>
__global__ __launch_bounds__(1024) void k_queue_build(QueueBuildArgs p) {
  __shared__ int cnt[kQueueWaves][kQueueMaxE];
  __shared__ int base[kQueueMaxE];
  __shared__ int total;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int E = p.E;
  for (int i = tid; i < kQueueWaves * kQueueMaxE; i += 1024) (&cnt[0][0])[i] = 0;
  __syncthreads();
  // wave w owns the contiguous packet range [lo, hi): packets keep their input order
  const int segs = (p.A + 63) / 64;
  const int per = (segs + kQueueWaves - 1) / kQueueWaves;
  const int lo = wave * per * 64;
  const int hi = min(p.A, (wave + 1) * per * 64);
  for (int i = lo + lane; i < hi; i += 64) {
    const int64_t e = ld_index<IT>(p.experts, i);
    if (e >= 0 && e < E) atomicAdd(&cnt[wave][(int)e], 1);
  }
  __syncthreads();
  if (tid < E) {
    int c = 0;
    for (int w = 0; w < kQueueWaves; ++w) c += cnt[w][tid];
    base[tid] = c;
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int e = 0; e < E; ++e) {
      const int c = base[e];
      if (p.counts_i64) {
        static_cast<int64_t*>(p.counts)[e] = c;
        static_cast<int64_t*>(p.starts)[e] = run;
      } else {
        static_cast<int32_t*>(p.counts)[e] = c;
        static_cast<int32_t*>(p.starts)[e] = run;
      }
      base[e] = run;
      run += c;
    }
    total = run;
  }
  __syncthreads();
  if (tid < E) {
    int run = base[tid];
    for (int w = 0; w < kQueueWaves; ++w) {
      const int c = cnt[w][tid];
      cnt[w][tid] = run;  // wave w's cursor for expert tid
      run += c;
    }
  }
  __syncthreads();
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  for (int s0 = lo; s0 < hi; s0 += 64) {
    const int i = s0 + lane;
    const bool in = i < hi;
    const int64_t e64 = in ? ld_index<IT>(p.experts, i) : -1;
    const bool ok = in && e64 >= 0 && e64 < E;
    const int e = ok ? (int)e64 : 0;
    uint64_t match = __ballot(ok);
    for (int b = 0; b < nbits; ++b) {
      const uint64_t bb = __ballot(ok && ((e >> b) & 1));
      match &= ((e >> b) & 1) ? bb : ~bb;
    }
    const uint64_t lower = lane ? (~0ull >> (64 - lane)) : 0ull;
    const int rank = __popcll(match & lower);
    const int n_same = __popcll(match);
    int dest = 0;
    if (ok) dest = cnt[wave][e] + rank;
    __builtin_amdgcn_wave_barrier();
    if (ok && rank == n_same - 1) cnt[wave][e] += n_same;
    __builtin_amdgcn_wave_barrier();
    if (ok) {
      const int64_t tok = p.tokens ? p.tokens[i] : (int64_t)(i / p.top_k);
      const int64_t slot = p.slots ? p.slots[i] : (int64_t)(i % p.top_k);
      const bool row_ok = tok >= 0 && tok < p.rows;
      p.token_ids[dest] = tok;
      p.expert_ids[dest] = e;
      p.route_slots[dest] = slot;
      p.coefficients[dest] = ld_weight<WT>(p.weights, i);
      p.epochs[dest] = row_ok ? p.row_epochs[tok] : LLONG_MIN;
      p.deadlines[dest] = row_ok ? p.row_deadlines[tok] : LLONG_MIN;
    }
  }
  for (int q = total + tid; q < p.A; q += 1024) {
    p.token_ids[q] = 0;
    p.expert_ids[q] = -1;
    p.route_slots[q] = -1;
    p.coefficients[q] = 0.f;
    p.epochs[q] = LLONG_MIN;
    p.deadlines[q] = LLONG_MIN;
  }
}

__global__ __launch_bounds__(256) void k_fill_i32(int32_t* __restrict__ dst, int64_t n, int32_t value) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) dst[i] = value;
}

// valid[q] and the number of valid packets per row
__global__ __launch_bounds__(256) void k_scatter_count(const int64_t* __restrict__ token_ids,
                                                       const int64_t* __restrict__ epochs,
                                                       const int64_t* __restrict__ active, int64_t A, int64_t rows,
                                                       uint8_t* __restrict__ valid, int32_t* __restrict__ counts) {
  for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < A; q += (int64_t)gridDim.x * 256) {
    const int64_t t = token_ids[q];
    const bool ok = t >= 0 && t < rows && epochs[q] == active[t];
    valid[q] = ok ? 1 : 0;
    if (ok) atomicAdd(&counts[t], 1);
  }
}

// In-place exclusive prefix sum of n int32 values, one workgroup: each thread sums a
// contiguous chunk, the chunk sums are scanned in LDS (Hillis-Steele), then each thread
// writes its chunk's prefixes.
__global__ __launch_bounds__(1024) void k_scan_exclusive(int32_t* __restrict__ v, int64_t n) {
  __shared__ int32_t buf[2][1024];
  const int tid = threadIdx.x;
  const int64_t chunk = (n + 1023) / 1024;
  const int64_t b = tid * chunk;
  const int64_t e = b + chunk < n ? b + chunk : n;
  int32_t sum = 0;
  for (int64_t i = b; i < e; ++i) sum += v[i];
  buf[0][tid] = sum;
  __syncthreads();
  int cur = 0;
  for (int off = 1; off < 1024; off <<= 1) {
    const int32_t add = tid >= off ? buf[cur][tid - off] : 0;
    buf[cur ^ 1][tid] = buf[cur][tid] + add;
    cur ^= 1;
    __syncthreads();
  }
  int32_t run = buf[cur][tid] - sum;  // exclusive prefix of this chunk
  for (int64_t i = b; i < e; ++i) {
    const int32_t c = v[i];
    v[i] = run;
    run += c;
  }
}

// each valid packet into its row's range (arrival order within the range)
__global__ __launch_bounds__(256) void k_scatter_place(const int64_t* __restrict__ token_ids,
                                                       const uint8_t* __restrict__ valid, int64_t A,
                                                       const int32_t* __restrict__ starts,
                                                       int32_t* __restrict__ cursor, int32_t* __restrict__ tmp) {
  for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < A; q += (int64_t)gridDim.x * 256) {
    if (!valid[q]) continue;
    const int64_t t = token_ids[q];
    tmp[starts[t] + atomicAdd(&cursor[t], 1)] = (int32_t)q;
  }
}

// each valid packet's rank among its row's packets (ascending queue index): the row's
// range in ascending queue order, whatever order the placement left
__global__ __launch_bounds__(256) void k_scatter_rank(const int64_t* __restrict__ token_ids,
                                                      const uint8_t* __restrict__ valid, int64_t A,
                                                      const int32_t* __restrict__ starts,
                                                      const int32_t* __restrict__ tmp, int32_t* __restrict__ order) {
  for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < A; q += (int64_t)gridDim.x * 256) {
    if (!valid[q]) continue;
    const int64_t t = token_ids[q];
    const int32_t b = starts[t], e = starts[t + 1];
    int32_t r = 0;
    for (int32_t j = b; j < e; ++j) r += tmp[j] < (int32_t)q ? 1 : 0;
    order[b + r] = (int32_t)q;
  }
}

// per row t (grid-stride over rows) and 256 hidden columns: the row's packets in
// ascending queue order, acc = acc + fp32(float(y[q]) * coef[q]) from 0
template <int YT>
__global__ __launch_bounds__(256) void k_scatter_reduce(const void* __restrict__ y, int64_t ldy,
                                                        const float* __restrict__ coef,
                                                        const int32_t* __restrict__ starts,
                                                        const int32_t* __restrict__ order, int64_t rows, int H,
                                                        float* __restrict__ out) {
  const int h = blockIdx.x * 256 + threadIdx.x;
  if (h >= H) return;
  for (int64_t t = blockIdx.y; t < rows; t += gridDim.y) {
    float acc = 0.f;
    const int32_t b = starts[t], e = starts[t + 1];
    for (int32_t j = b; j < e; ++j) {
      const int64_t q = order[j];
      float v;
      if constexpr (YT == QS_F32) v = static_cast<const float*>(y)[q * ldy + h];
      else if constexpr (YT == QS_BF16) v = bf16_bits_to_f32(static_cast<const uint16_t*>(y)[q * ldy + h]);
      else v = f16_bits_to_f32(static_cast<const uint16_t*>(y)[q * ldy + h]);
      acc = add_rn(acc, mul_rn(v, coef[q]));
    }
    out[t * H + h] = acc;
  }
}

unsigned grid_for(int64_t n) {
  const int64_t b = cdiv(n, 256);
  return (unsigned)(b < 1 ? 1 : (b < 65536 ? b : 65536));
}

}  // namespace
}  // namespace qs

using namespace qs;

extern "C" int qs_expert_queue_build(const void* experts, int expert_dtype, const int64_t* tokens,
                                     const int64_t* slots, const void* weights, int weight_dtype,
                                     const int64_t* row_epochs, const int64_t* row_deadlines, int64_t A,
                                     int top_k, int64_t rows, int E, int64_t* token_ids, int64_t* expert_ids,
                                     int64_t* route_slots, float* coefficients, int64_t* epochs,
                                     int64_t* deadlines, void* starts, void* counts, int count_dtype,
                                     void* stream) {
  if (!token_ids || !expert_ids || !route_slots || !coefficients || !epochs || !deadlines || !starts ||
      !counts || !row_epochs || !row_deadlines)
    return fail(QS_ERR_INVALID, "expert_queue_build: null pointer");
  if (A < 0 || top_k < 1 || rows < 1 || E < 1) return fail(QS_ERR_INVALID, "expert_queue_build: bad shape");
  if ((tokens == nullptr) != (slots == nullptr))
    return fail(QS_ERR_INVALID, "expert_queue_build: tokens and slots are given together or not at all");
  if (!tokens && A != rows * (int64_t)top_k)
    return fail(QS_ERR_INVALID, "expert_queue_build: dense packets need A == rows * top_k");
  if (A > 0 && (!experts || !weights)) return fail(QS_ERR_INVALID, "expert_queue_build: null pointer");
  if (E > kQueueMaxE) return fail(QS_ERR_LIMIT, "expert_queue_build: at most %d experts", kQueueMaxE);
  if (A > ((int64_t)1 << 28)) return fail(QS_ERR_LIMIT, "expert_queue_build: too many packets");
  if (count_dtype != QS_I32 && count_dtype != QS_I64)
    return fail(QS_ERR_INVALID, "expert_queue_build: counts I32 or I64");
  if (expert_dtype != QS_I32 && expert_dtype != QS_I64)
    return fail(QS_ERR_INVALID, "expert_queue_build: expert ids I32 or I64");
  if (weight_dtype != QS_F32 && weight_dtype != QS_BF16 && weight_dtype != QS_F16)
    return fail(QS_ERR_INVALID, "expert_queue_build: weights F32, BF16 or F16");
  QueueBuildArgs p{experts, tokens, slots, weights, row_epochs, row_deadlines, (int)A, top_k, E, rows,
                   token_ids, expert_ids, route_slots, coefficients, epochs, deadlines, starts, counts,
                   count_dtype == QS_I64};
  hipStream_t s = static_cast<hipStream_t>(stream);
#define QS_QB(IT, WT) hipLaunchKernelGGL((k_queue_build<IT, WT>), dim3(1), dim3(1024), 0, s, p)
  if (expert_dtype == QS_I64) {
    if (weight_dtype == QS_F32) QS_QB(QS_I64, QS_F32);
    else if (weight_dtype == QS_BF16) QS_QB(QS_I64, QS_BF16);
    else QS_QB(QS_I64, QS_F16);
  } else {
    if (weight_dtype == QS_F32) QS_QB(QS_I32, QS_F32);
    else if (weight_dtype == QS_BF16) QS_QB(QS_I32, QS_BF16);
    else QS_QB(QS_I32, QS_F16);
  }
#undef QS_QB
  return hip_check(hipGetLastError(), "k_queue_build launch");
}

// workspace (int32): starts[rows + 1] | cursor[rows] | tmp[A] | order[A]
extern "C" size_t qs_expert_queue_scatter_workspace_bytes(int64_t rows, int64_t A) {
  if (rows <= 0 || A < 0) return 0;
  return (size_t)(2 * rows + 1 + 2 * A) * sizeof(int32_t);
}

extern "C" int qs_expert_queue_scatter(const int64_t* token_ids, const float* coefficients, const int64_t* epochs,
                                       const int64_t* active_epochs, const void* expert_out, int out_dtype,
                                       int64_t ld_out, int64_t A, int64_t rows, int64_t H, void* workspace,
                                       size_t workspace_bytes, float* reduced, uint8_t* valid, void* stream) {
  if (!active_epochs || !reduced || !workspace ||
      (A > 0 && (!token_ids || !coefficients || !epochs || !expert_out || !valid)))
    return fail(QS_ERR_INVALID, "expert_queue_scatter: null pointer");
  if (A < 0 || rows < 1 || H < 1 || ld_out < H) return fail(QS_ERR_INVALID, "expert_queue_scatter: bad shape");
  if (H > INT_MAX || A >= INT_MAX || rows >= INT_MAX)
    return fail(QS_ERR_LIMIT, "expert_queue_scatter: packets, rows and hidden size below 2^31");
  if (workspace_bytes < qs_expert_queue_scatter_workspace_bytes(rows, A))
    return fail(QS_ERR_INVALID, "expert_queue_scatter: workspace smaller than qs_expert_queue_scatter_workspace_bytes()");
  if (out_dtype != QS_F32 && out_dtype != QS_BF16 && out_dtype != QS_F16)
    return fail(QS_ERR_INVALID, "expert_queue_scatter: expert outputs F32, BF16 or F16");
  hipStream_t s = static_cast<hipStream_t>(stream);
  int32_t* starts = static_cast<int32_t*>(workspace);
  int32_t* cursor = starts + rows + 1;
  int32_t* tmp = cursor + rows;
  int32_t* order = tmp + A;
  // counts (then starts, in place) and cursors start at zero: one fill kernel over both
  hipLaunchKernelGGL(k_fill_i32, dim3(grid_for(2 * rows + 1)), dim3(256), 0, s, starts, 2 * rows + 1, 0);
  if (A > 0) {
    hipLaunchKernelGGL(k_scatter_count, dim3(grid_for(A)), dim3(256), 0, s, token_ids, epochs, active_epochs, A,
                       rows, valid, starts);
    hipLaunchKernelGGL(k_scan_exclusive, dim3(1), dim3(1024), 0, s, starts, rows + 1);
    hipLaunchKernelGGL(k_scatter_place, dim3(grid_for(A)), dim3(256), 0, s, token_ids, valid, A, starts, cursor, tmp);
    hipLaunchKernelGGL(k_scatter_rank, dim3(grid_for(A)), dim3(256), 0, s, token_ids, valid, A, starts, tmp, order);
  }
  const dim3 grid((unsigned)cdiv(H, 256), (unsigned)(rows < 65535 ? rows : 65535));
  if (out_dtype == QS_F32)
    hipLaunchKernelGGL(k_scatter_reduce<QS_F32>, grid, dim3(256), 0, s, expert_out, ld_out, coefficients, starts, order, rows, (int)H, reduced);
  else if (out_dtype == QS_BF16)
    hipLaunchKernelGGL(k_scatter_reduce<QS_BF16>, grid, dim3(256), 0, s, expert_out, ld_out, coefficients, starts, order, rows, (int)H, reduced);
  else
    hipLaunchKernelGGL(k_scatter_reduce<QS_F16>, grid, dim3(256), 0, s, expert_out, ld_out, coefficients, starts, order, rows, (int)H, reduced);
  return hip_check(hipGetLastError(), "expert queue scatter launch");
}
