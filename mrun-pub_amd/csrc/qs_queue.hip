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
//   k_fill_i64      : fills an int64 array (in place of a memset, so that graph capture
//                     records a kernel node).
//   k_queue_inverse : per packet q: valid[q] = (epoch[q] == active[token[q]]) and
//                     inverse[token[q] * top_k + slot[q]] = q (the packet that carries route
//                     slot `slot` of that row).
//   k_queue_reduce  : per row t and 256 hidden columns: the row's valid packets, taken in
//                     ascending queue order, summed as acc = acc + fp32(float(y[q]) * coef[q])
//                     from acc = 0 -- the order and roundings of an index_add_ over the valid
//                     packets -- with no atomics, so the result is the same on every call.
#include "qs_common.h"

#include <limits.h>

namespace qs {
namespace {

constexpr int kQueueWaves = 16;
constexpr int kQueueMaxE = 512;
constexpr int kQueueMaxTopK = 64;

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

__global__ __launch_bounds__(256) void k_fill_i64(int64_t* __restrict__ dst, int64_t n, int64_t value) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) dst[i] = value;
}

__global__ __launch_bounds__(256) void k_queue_inverse(const int64_t* __restrict__ token_ids,
                                                       const int64_t* __restrict__ route_slots,
                                                       const int64_t* __restrict__ epochs,
                                                       const int64_t* __restrict__ active, int64_t A,
                                                       int64_t rows, int top_k, int64_t* __restrict__ inverse,
                                                       uint8_t* __restrict__ valid) {
  for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < A; q += (int64_t)gridDim.x * 256) {
    const int64_t t = token_ids[q];
    const int64_t s = route_slots[q];
    const bool in = t >= 0 && t < rows && s >= 0 && s < top_k;
    const bool ok = in && epochs[q] == active[t];
    valid[q] = ok ? 1 : 0;
    if (ok) inverse[t * top_k + s] = q;
  }
}

template <int YT>
__global__ __launch_bounds__(256) void k_queue_reduce(const void* __restrict__ y, int64_t ldy,
                                                      const float* __restrict__ coef,
                                                      const int64_t* __restrict__ inverse, int top_k,
                                                      int H, float* __restrict__ out) {
  __shared__ int64_t order[kQueueMaxTopK];
  __shared__ int n_valid;
  const int64_t t = blockIdx.y;
  if (threadIdx.x == 0) {
    // the row's packets in ascending queue order (insertion sort of at most top_k entries)
    int n = 0;
    for (int s = 0; s < top_k; ++s) {
      const int64_t q = inverse[t * top_k + s];
      if (q < 0) continue;
      int j = n++;
      while (j > 0 && order[j - 1] > q) {
        order[j] = order[j - 1];
        --j;
      }
      order[j] = q;
    }
    n_valid = n;
  }
  __syncthreads();
  const int h = blockIdx.x * 256 + threadIdx.x;
  if (h >= H) return;
  float acc = 0.f;
  for (int j = 0; j < n_valid; ++j) {
    const int64_t q = order[j];
    float v;
    if constexpr (YT == QS_F32) v = static_cast<const float*>(y)[q * ldy + h];
    else if constexpr (YT == QS_BF16) v = bf16_bits_to_f32(static_cast<const uint16_t*>(y)[q * ldy + h]);
    else v = f16_bits_to_f32(static_cast<const uint16_t*>(y)[q * ldy + h]);
    acc = add_rn(acc, mul_rn(v, coef[q]));
  }
  out[t * H + h] = acc;
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

extern "C" size_t qs_expert_queue_scatter_workspace_bytes(int64_t rows, int top_k) {
  if (rows <= 0 || top_k <= 0) return 0;
  return (size_t)(rows * top_k) * sizeof(int64_t);
}

extern "C" int qs_expert_queue_scatter(const int64_t* token_ids, const int64_t* route_slots,
                                       const float* coefficients, const int64_t* epochs,
                                       const int64_t* active_epochs, const void* expert_out, int out_dtype,
                                       int64_t ld_out, int64_t A, int64_t rows, int top_k, int64_t H,
                                       void* workspace, size_t workspace_bytes, float* reduced,
                                       uint8_t* valid, void* stream) {
  if (!active_epochs || !reduced || !workspace || (A > 0 && (!token_ids || !route_slots || !coefficients ||
                                                             !epochs || !expert_out || !valid)))
    return fail(QS_ERR_INVALID, "expert_queue_scatter: null pointer");
  if (A < 0 || rows < 1 || top_k < 1 || H < 1 || ld_out < H)
    return fail(QS_ERR_INVALID, "expert_queue_scatter: bad shape");
  if (top_k > kQueueMaxTopK) return fail(QS_ERR_LIMIT, "expert_queue_scatter: top_k at most %d", kQueueMaxTopK);
  if (H > INT_MAX || rows > 65535) return fail(QS_ERR_LIMIT, "expert_queue_scatter: at most 65535 rows");
  if (workspace_bytes < qs_expert_queue_scatter_workspace_bytes(rows, top_k))
    return fail(QS_ERR_INVALID, "expert_queue_scatter: workspace smaller than qs_expert_queue_scatter_workspace_bytes()");
  if (out_dtype != QS_F32 && out_dtype != QS_BF16 && out_dtype != QS_F16)
    return fail(QS_ERR_INVALID, "expert_queue_scatter: expert outputs F32, BF16 or F16");
  hipStream_t s = static_cast<hipStream_t>(stream);
  int64_t* inverse = static_cast<int64_t*>(workspace);
  const int64_t slots_total = rows * top_k;
  hipLaunchKernelGGL(k_fill_i64, dim3(grid_for(slots_total)), dim3(256), 0, s, inverse, slots_total, (int64_t)-1);
  if (A > 0)
    hipLaunchKernelGGL(k_queue_inverse, dim3(grid_for(A)), dim3(256), 0, s, token_ids, route_slots, epochs,
                       active_epochs, A, rows, top_k, inverse, valid);
  const dim3 grid((unsigned)cdiv(H, 256), (unsigned)rows);
  if (out_dtype == QS_F32)
    hipLaunchKernelGGL(k_queue_reduce<QS_F32>, grid, dim3(256), 0, s, expert_out, ld_out, coefficients, inverse, top_k, (int)H, reduced);
  else if (out_dtype == QS_BF16)
    hipLaunchKernelGGL(k_queue_reduce<QS_BF16>, grid, dim3(256), 0, s, expert_out, ld_out, coefficients, inverse, top_k, (int)H, reduced);
  else
    hipLaunchKernelGGL(k_queue_reduce<QS_F16>, grid, dim3(256), 0, s, expert_out, ld_out, coefficients, inverse, top_k, (int)H, reduced);
  return hip_check(hipGetLastError(), "expert queue scatter launch");
}
