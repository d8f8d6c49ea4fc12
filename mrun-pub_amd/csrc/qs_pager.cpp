// Pinned-host -> HBM page streamer (host code, HIP runtime API).
//
// A pager drives an HBM ring of `slots` equal-size slots (caller-owned device memory) and
// owns one copy stream at the default priority.  submit() copies a byte range of pinned
// host memory (a run of contiguous host pages) into a slot on the copy stream once the
// slot's "free" event (recorded by the last consumer) has fired, as transfers of at most
// max_transfer bytes: each hipMemcpyAsync carries a fixed cost, and 2 MiB transfers reach
// only about 60% of the link rate that 16 MiB and larger ones do.  seal() records the
// slot's "ready" event; acquire() makes a compute stream wait for "ready"; release()
// records "free" on the compute stream.  Only submit() can block the host, and only while
// the slot's last consumer is still queued on the GPU (the host is a whole ring ahead), so
// a slot is never overwritten while a kernel still reads it and never read before its
// copy has landed.
#include <hip/hip_runtime.h>

#include <new>
#include <vector>

#include "../../include/qstore_hip.h"

namespace qs {
int fail(int status, const char* fmt, ...);
int hip_check(hipError_t e, const char* what);
}  // namespace qs

using qs::fail;
using qs::hip_check;

struct qs_pager {
  size_t slot_bytes = 0;
  size_t max_transfer = 0;
  int slots = 0;
  char* arena = nullptr;  // caller-owned, slot_bytes * slots bytes
  hipStream_t copy = nullptr;
  std::vector<hipEvent_t> ready, freed;
  std::vector<int> used;  // a free event has been recorded at least once
};

extern "C" int qs_pager_create(void* device_arena, size_t slot_bytes, int slots,
                               size_t max_transfer, qs_pager** out) {
  if (!out || !device_arena || slot_bytes == 0 || slot_bytes % 256 || slots < 1 || slots > 65536 ||
      max_transfer == 0)
    return fail(QS_ERR_INVALID, "pager_create: bad arguments");
  qs_pager* p = new (std::nothrow) qs_pager();
  if (!p) return fail(QS_ERR_HIP, "pager_create: out of host memory");
  p->slot_bytes = slot_bytes;
  p->max_transfer = max_transfer;
  p->slots = slots;
  p->arena = static_cast<char*>(device_arena);
  int st = hip_check(hipStreamCreateWithFlags(&p->copy, hipStreamNonBlocking), "hipStreamCreate");
  p->ready.assign(slots, nullptr);
  p->freed.assign(slots, nullptr);
  p->used.assign(slots, 0);
  for (int i = 0; !st && i < slots; ++i) {
    st = hip_check(hipEventCreateWithFlags(&p->ready[i], hipEventDisableTiming), "hipEventCreate");
    if (!st) st = hip_check(hipEventCreateWithFlags(&p->freed[i], hipEventDisableTiming), "hipEventCreate");
  }
  if (st) {
    qs_pager_destroy(p);
    return st;
  }
  *out = p;
  return QS_OK;
}

extern "C" int qs_pager_destroy(qs_pager* p) {
  if (!p) return QS_OK;
  if (p->copy) hipStreamSynchronize(p->copy);
  for (auto e : p->ready)
    if (e) hipEventDestroy(e);
  for (auto e : p->freed)
    if (e) hipEventDestroy(e);
  if (p->copy) hipStreamDestroy(p->copy);
  delete p;
  return QS_OK;
}

extern "C" void* qs_pager_slot_ptr(qs_pager* p, int slot) {
  if (!p || slot < 0 || slot >= p->slots) return nullptr;
  return p->arena + p->slot_bytes * (size_t)slot;
}

extern "C" int qs_pager_submit(qs_pager* p, int slot, const void* host, size_t bytes,
                               size_t dst_offset) {
  if (!p || !host || slot < 0 || slot >= p->slots)
    return fail(QS_ERR_INVALID, "pager_submit: bad arguments");
  if (dst_offset + bytes > p->slot_bytes) return fail(QS_ERR_LIMIT, "pager_submit: range exceeds the slot");
  if (p->used[slot]) {
    // The slot's last consumer must be done before the copy overwrites it.  The wait is
    // taken on the host (a query, and a block only when the host is a whole ring ahead of
    // the GPU): a copy stream made to wait on a compute-stream event can stall the host
    // inside the following hipMemcpyAsync until that event fires, and the link then
    // idles between blocks.
    hipError_t q = hipEventQuery(p->freed[slot]);
    if (q == hipErrorNotReady) q = hipEventSynchronize(p->freed[slot]);
    int st = hip_check(q, "slot free event");
    if (st) return st;
  }
  char* dst = p->arena + p->slot_bytes * (size_t)slot + dst_offset;
  const char* src = static_cast<const char*>(host);
  for (size_t off = 0; off < bytes; off += p->max_transfer) {
    const size_t n = bytes - off < p->max_transfer ? bytes - off : p->max_transfer;
    int st = hip_check(hipMemcpyAsync(dst + off, src + off, n, hipMemcpyHostToDevice, p->copy), "hipMemcpyAsync");
    if (st) return st;
  }
  return QS_OK;
}

extern "C" int qs_pager_seal(qs_pager* p, int slot) {
  if (!p || slot < 0 || slot >= p->slots) return fail(QS_ERR_INVALID, "pager_seal: bad arguments");
  return hip_check(hipEventRecord(p->ready[slot], p->copy), "hipEventRecord(ready)");
}

extern "C" int qs_pager_acquire(qs_pager* p, int slot, void* compute_stream) {
  if (!p || slot < 0 || slot >= p->slots) return fail(QS_ERR_INVALID, "pager_acquire: bad arguments");
  return hip_check(hipStreamWaitEvent(static_cast<hipStream_t>(compute_stream), p->ready[slot], 0),
                   "hipStreamWaitEvent(ready)");
}

extern "C" int qs_pager_release(qs_pager* p, int slot, void* compute_stream) {
  if (!p || slot < 0 || slot >= p->slots) return fail(QS_ERR_INVALID, "pager_release: bad arguments");
  p->used[slot] = 1;
  return hip_check(hipEventRecord(p->freed[slot], static_cast<hipStream_t>(compute_stream)),
                   "hipEventRecord(free)");
}

// Batched forms for an expert layer's whole active set (about 128 slots per acquire).
// A slot whose ready event has already fired needs no stream wait: a wait on a completed
// event orders nothing, so skipping it keeps the same ordering with one packet fewer.
extern "C" int qs_pager_acquire_many(qs_pager* p, const int* slots, int n, void* compute_stream) {
  if (!p || n < 0 || (n > 0 && !slots)) return fail(QS_ERR_INVALID, "pager_acquire_many: bad arguments");
  for (int i = 0; i < n; ++i)
    if (slots[i] < 0 || slots[i] >= p->slots) return fail(QS_ERR_INVALID, "pager_acquire_many: slot out of range");
  auto stream = static_cast<hipStream_t>(compute_stream);
  for (int i = 0; i < n; ++i) {
    hipEvent_t ev = p->ready[slots[i]];
    hipError_t q = hipEventQuery(ev);
    if (q == hipSuccess) continue;
    if (q != hipErrorNotReady) return hip_check(q, "hipEventQuery(ready)");
    int st = hip_check(hipStreamWaitEvent(stream, ev, 0), "hipStreamWaitEvent(ready)");
    if (st) return st;
  }
  return QS_OK;
}

extern "C" int qs_pager_release_many(qs_pager* p, const int* slots, int n, void* compute_stream) {
  if (!p || n < 0 || (n > 0 && !slots)) return fail(QS_ERR_INVALID, "pager_release_many: bad arguments");
  for (int i = 0; i < n; ++i)
    if (slots[i] < 0 || slots[i] >= p->slots) return fail(QS_ERR_INVALID, "pager_release_many: slot out of range");
  for (int i = 0; i < n; ++i) {
    int st = qs_pager_release(p, slots[i], compute_stream);
    if (st) return st;
  }
  return QS_OK;
}

extern "C" int qs_pager_sync(qs_pager* p) {
  if (!p) return fail(QS_ERR_INVALID, "pager_sync: null pager");
  return hip_check(hipStreamSynchronize(p->copy), "hipStreamSynchronize(copy)");
}
