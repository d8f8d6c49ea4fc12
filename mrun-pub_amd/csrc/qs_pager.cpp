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

#include <algorithm>
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
  std::vector<hipEvent_t> ready;
  std::vector<char> ready_done;  // ready has been seen complete since the last seal
  // "free" events: one event per release batch, shared by the batch's slots and reference
  // counted, so a 128-slot release is one hipEventRecord; an event goes back to the pool
  // once no slot refers to it (it is never re-recorded while a slot still waits on it)
  std::vector<int> freed;  // slot -> event index, -1: never released or already waited on
  std::vector<hipEvent_t> events;
  std::vector<int> refs;
  std::vector<int> pool;
  // release_many's duplicate check: seen[slot] == stamp marks a slot of the current batch
  std::vector<unsigned> seen;
  unsigned stamp = 0;
};

namespace {
int take_event(qs_pager* p, int* out) {
  if (p->pool.empty()) {
    hipEvent_t e = nullptr;
    int st = hip_check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
    if (st) return st;
    p->events.push_back(e);
    p->refs.push_back(0);
    *out = (int)p->events.size() - 1;
  } else {
    *out = p->pool.back();
    p->pool.pop_back();
  }
  return QS_OK;
}

void drop_free_ref(qs_pager* p, int slot) {
  const int e = p->freed[slot];
  if (e < 0) return;
  if (--p->refs[e] == 0) p->pool.push_back(e);
  p->freed[slot] = -1;
}
}  // namespace

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
  p->ready_done.assign(slots, 1);  // never sealed: nothing to wait for
  p->freed.assign(slots, -1);
  p->seen.assign(slots, 0);
  for (int i = 0; !st && i < slots; ++i)
    st = hip_check(hipEventCreateWithFlags(&p->ready[i], hipEventDisableTiming), "hipEventCreate");
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
  for (auto e : p->events)
    if (e) hipEventDestroy(e);
  if (p->copy) hipStreamDestroy(p->copy);
  delete p;
  return QS_OK;
}

extern "C" void* qs_pager_slot_ptr(qs_pager* p, int slot) {
  if (!p || slot < 0 || slot >= p->slots) return nullptr;
  return p->arena + p->slot_bytes * (size_t)slot;
}

namespace {
// The slot's last consumer must be done before a copy overwrites it.  The wait is taken on
// the host (a query, and a block only when the host is a whole ring ahead of the GPU): a
// copy stream made to wait on a compute-stream event can stall the host inside the
// following hipMemcpyAsync until that event fires, and the link then idles between blocks.
int wait_slot_free(qs_pager* p, int slot) {
  if (p->freed[slot] < 0) return QS_OK;
  hipEvent_t ev = p->events[p->freed[slot]];
  hipError_t q = hipEventQuery(ev);
  if (q == hipErrorNotReady) q = hipEventSynchronize(ev);
  int st = hip_check(q, "slot free event");
  if (st) return st;
  drop_free_ref(p, slot);
  return QS_OK;
}

int copy_h2d(qs_pager* p, char* dst, const char* src, size_t bytes) {
  for (size_t off = 0; off < bytes; off += p->max_transfer) {
    const size_t n = bytes - off < p->max_transfer ? bytes - off : p->max_transfer;
    int st = hip_check(hipMemcpyAsync(dst + off, src + off, n, hipMemcpyHostToDevice, p->copy), "hipMemcpyAsync");
    if (st) return st;
  }
  return QS_OK;
}
}  // namespace

extern "C" int qs_pager_submit(qs_pager* p, int slot, const void* host, size_t bytes,
                               size_t dst_offset) {
  if (!p || !host || slot < 0 || slot >= p->slots)
    return fail(QS_ERR_INVALID, "pager_submit: bad arguments");
  if (dst_offset + bytes > p->slot_bytes) return fail(QS_ERR_LIMIT, "pager_submit: range exceeds the slot");
  int st = wait_slot_free(p, slot);
  if (st) return st;
  return copy_h2d(p, p->arena + p->slot_bytes * (size_t)slot + dst_offset, static_cast<const char*>(host), bytes);
}

// A run of whole slots from one contiguous host range: every slot's previous consumer is
// waited for, the range moves in max_transfer pieces (not one copy per slot), then every
// slot is sealed.  A layer change refills ~125 consecutive expert pages into consecutive
// slots, so its copies become a few large transfers.
extern "C" int qs_pager_submit_run(qs_pager* p, int slot, int count, const void* host) {
  if (!p || !host || slot < 0 || count < 1 || count > p->slots - slot)
    return fail(QS_ERR_INVALID, "pager_submit_run: bad arguments");
  for (int i = 0; i < count; ++i) {
    int st = wait_slot_free(p, slot + i);
    if (st) return st;
  }
  int st = copy_h2d(p, p->arena + p->slot_bytes * (size_t)slot, static_cast<const char*>(host),
                    p->slot_bytes * (size_t)count);
  if (st) return st;
  for (int i = 0; i < count; ++i) {
    p->ready_done[slot + i] = 0;
    st = hip_check(hipEventRecord(p->ready[slot + i], p->copy), "hipEventRecord(ready)");
    if (st) return st;
  }
  return QS_OK;
}

extern "C" int qs_pager_seal(qs_pager* p, int slot) {
  if (!p || slot < 0 || slot >= p->slots) return fail(QS_ERR_INVALID, "pager_seal: bad arguments");
  p->ready_done[slot] = 0;
  return hip_check(hipEventRecord(p->ready[slot], p->copy), "hipEventRecord(ready)");
}

// Batched forms for an expert layer's whole active set (about 128 slots per acquire).
// A slot whose ready event has already fired needs no stream wait: a wait on a completed
// event orders nothing, so skipping it keeps the same ordering with one packet fewer.  A
// slot seen complete once stays so until its next seal, so it costs no further query.
extern "C" int qs_pager_acquire_many(qs_pager* p, const int* slots, int n, void* compute_stream) {
  if (!p || n < 0 || (n > 0 && !slots)) return fail(QS_ERR_INVALID, "pager_acquire_many: bad arguments");
  for (int i = 0; i < n; ++i)
    if (slots[i] < 0 || slots[i] >= p->slots) return fail(QS_ERR_INVALID, "pager_acquire_many: slot out of range");
  auto stream = static_cast<hipStream_t>(compute_stream);
  for (int i = 0; i < n; ++i) {
    const int sl = slots[i];
    if (p->ready_done[sl]) continue;
    hipEvent_t ev = p->ready[sl];
    hipError_t q = hipEventQuery(ev);
    if (q == hipSuccess) {
      p->ready_done[sl] = 1;
      continue;
    }
    if (q != hipErrorNotReady) return hip_check(q, "hipEventQuery(ready)");
    int st = hip_check(hipStreamWaitEvent(stream, ev, 0), "hipStreamWaitEvent(ready)");
    if (st) return st;
  }
  return QS_OK;
}

// One "free" event recorded for the whole batch; each slot drops its previous event.  A
// slot listed twice is refused before anything changes: its second reference would drop
// the batch's own event to zero refs and return it to the pool while the slot still
// points at it.
extern "C" int qs_pager_release_many(qs_pager* p, const int* slots, int n, void* compute_stream) {
  if (!p || n < 0 || (n > 0 && !slots)) return fail(QS_ERR_INVALID, "pager_release_many: bad arguments");
  for (int i = 0; i < n; ++i)
    if (slots[i] < 0 || slots[i] >= p->slots) return fail(QS_ERR_INVALID, "pager_release_many: slot out of range");
  if (n == 0) return QS_OK;
  if (++p->stamp == 0) {  // the stamp wrapped: clear the marks once
    std::fill(p->seen.begin(), p->seen.end(), 0u);
    p->stamp = 1;
  }
  for (int i = 0; i < n; ++i) {
    if (p->seen[slots[i]] == p->stamp) return fail(QS_ERR_INVALID, "pager_release_many: slot %d listed twice", slots[i]);
    p->seen[slots[i]] = p->stamp;
  }
  int e = -1;
  int st = take_event(p, &e);
  if (st) return st;
  st = hip_check(hipEventRecord(p->events[e], static_cast<hipStream_t>(compute_stream)), "hipEventRecord(free)");
  if (st) {
    p->pool.push_back(e);
    return st;
  }
  for (int i = 0; i < n; ++i) {
    drop_free_ref(p, slots[i]);
    p->freed[slots[i]] = e;
    ++p->refs[e];
  }
  return QS_OK;
}

// Whether the copies last sealed into `slot` have landed (1) or not (0): a host-side
// query of the slot's ready event, for callers that reuse the host source of a copy.
extern "C" int qs_pager_slot_landed(qs_pager* p, int slot) {
  if (!p || slot < 0 || slot >= p->slots) return fail(QS_ERR_INVALID, "pager_slot_landed: bad arguments");
  if (p->ready_done[slot]) return 1;
  hipError_t q = hipEventQuery(p->ready[slot]);
  if (q == hipSuccess) {
    p->ready_done[slot] = 1;
    return 1;
  }
  return q == hipErrorNotReady ? 0 : hip_check(q, "hipEventQuery(ready)");
}

// Block the host until the copies last sealed into `slot` have landed.
extern "C" int qs_pager_wait_landed(qs_pager* p, int slot) {
  if (!p || slot < 0 || slot >= p->slots) return fail(QS_ERR_INVALID, "pager_wait_landed: bad arguments");
  if (p->ready_done[slot]) return QS_OK;
  int st = hip_check(hipEventSynchronize(p->ready[slot]), "hipEventSynchronize(ready)");
  if (!st) p->ready_done[slot] = 1;
  return st;
}

extern "C" int qs_pager_acquire(qs_pager* p, int slot, void* compute_stream) {
  if (!p || slot < 0 || slot >= p->slots) return fail(QS_ERR_INVALID, "pager_acquire: bad arguments");
  return qs_pager_acquire_many(p, &slot, 1, compute_stream);
}

extern "C" int qs_pager_release(qs_pager* p, int slot, void* compute_stream) {
  if (!p || slot < 0 || slot >= p->slots) return fail(QS_ERR_INVALID, "pager_release: bad arguments");
  return qs_pager_release_many(p, &slot, 1, compute_stream);
}

extern "C" int qs_pager_sync(qs_pager* p) {
  if (!p) return fail(QS_ERR_INVALID, "pager_sync: null pager");
  return hip_check(hipStreamSynchronize(p->copy), "hipStreamSynchronize(copy)");
}
