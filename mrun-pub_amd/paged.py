"""Paged int8 QStore: pinned host tier -> HBM slot ring -> fused HIP projections.

Mirrors the CUDA paged path of ``QStore`` with its successor-oracle prefetch ring
(src/mrun/engine/kernels/qstore.py:459-660 ``_RingSlot`` / ``_RingPrefetch``,
:800-833 ``enable_ring`` / ``disable_ring`` / ``ring_stats`` / ``ring_allocated_bytes``,
:1026-1097 ``weight`` / ``matmul`` / ``matmul_row_stable``).

Differences of design, same observable contract:

* Two host sides.  By default the host tier is ONE pinned allocation holding every qrow
  block as ``[codes][pad][scales]`` (each block 4096-aligned), filled once from the
  memory-mapped store: the pageable->pinned copy is paid once, so the steady state is
  bounded by the PCIe link alone.  For a store larger than pinned memory,
  ``staging_buffers=K`` keeps K pinned buffers only and re-stages every transfer from the
  mapping on worker threads, as the reference does (``MappedStagingTier``).
* The HBM side is a fixed ring of ``slots`` equal slots in one device allocation.  A
  block is a run of contiguous ``page_bytes`` (2 MiB) pages of the tier and travels as
  transfers of up to ``transfer_bytes`` (64 MiB, so one transfer per block) on the
  pager's copy stream (``csrc/qs_pager.cpp``): one 2 MiB copy per page would cap the
  link at about 60% of its rate; the compute stream waits on the slot's ready event,
  the fused kernel reads codes and scales in place from the slot, and the slot's free
  event is recorded right after.  The next copy into that slot is issued once the free
  event has fired: the host checks it, and blocks only when it has run a whole ring
  ahead of the GPU.  Taking that dependency on the copy stream instead stalls the host
  inside ``hipMemcpyAsync`` and leaves the link idle between blocks (35 vs 50 GB/s).
* A hit consumes the identical int8 codes and fp32 scales through the identical kernels
  as the resident ``DenseQStore``, so paged results equal resident results bit for bit.

The successor oracle is the reference's: ``observe(name)`` records ``last -> name`` and
prefetches the ``depth`` predicted successors; ``take(name)`` returns the prefetched
slot or ``None`` (miss).  A miss is served through the same ring (an immediate copy).
"""

from __future__ import annotations

import ctypes
import os
from collections import OrderedDict
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from . import _native as nat
from . import qrow as _qrow
from .dense_store import _DTYPES, DenseQStoreStats
from .qrow import CompactQRowPage
from .store import QStoreReader

PAGE_BYTES = 2 << 20
TRANSFER_BYTES = 64 << 20
IMPL_PAGED = "hip-gfx950-paged-ring-v1"


def _align(n: int, a: int) -> int:
    return (n + a - 1) // a * a


@dataclass(frozen=True)
class HostBlock:
    """Placement of one qrow block inside the pinned host tier (and inside a slot)."""

    name: str
    out_features: int
    in_features: int
    host_offset: int  # byte offset of the codes in the host tier
    scale_offset: int  # byte offset of the scales relative to the codes

    @property
    def span(self) -> int:
        """Bytes copied per transfer: codes, pad, scales."""
        return self.scale_offset + self.out_features * 4

    @property
    def compact_bytes(self) -> int:
        return self.out_features * self.in_features + self.out_features * 4


def _slot_layout(out: int, inn: int) -> int:
    return _align(out * inn, 256)


class PinnedHostTier:
    """Every qrow block of a store in one pinned host allocation."""

    def __init__(self, shapes: dict[str, tuple[int, int]]):
        self.blocks: dict[str, HostBlock] = {}
        off = 0
        for name, (out, inn) in shapes.items():
            so = _slot_layout(out, inn)
            self.blocks[name] = HostBlock(name, int(out), int(inn), off, so)
            off = _align(off + so + out * 4, 4096)
        self.nbytes = off
        self.host = torch.empty(max(off, 1), dtype=torch.uint8, pin_memory=True)

    def codes(self, name: str) -> np.ndarray:
        b = self.blocks[name]
        raw = self.host.numpy()[b.host_offset : b.host_offset + b.out_features * b.in_features]
        return raw.view(np.int8).reshape(b.out_features, b.in_features)

    def scales(self, name: str) -> np.ndarray:
        b = self.blocks[name]
        a = b.host_offset + b.scale_offset
        return self.host.numpy()[a : a + b.out_features * 4].view(np.float32)

    def put(self, name: str, codes, scales) -> None:
        """Write one block's codes ``[out, in]`` int8 and scales ``[out]`` fp32."""
        b = self.blocks[name]
        if isinstance(codes, torch.Tensor):
            dst = self.host[b.host_offset : b.host_offset + b.out_features * b.in_features]
            dst.copy_(codes.reshape(-1).view(torch.uint8))
            a = b.host_offset + b.scale_offset
            self.host[a : a + b.out_features * 4].copy_(scales.reshape(-1).contiguous().view(torch.uint8))
            return
        np.copyto(self.codes(name), np.asarray(codes, dtype=np.int8).reshape(b.out_features, b.in_features))
        np.copyto(self.scales(name), np.asarray(scales, dtype=np.float32).reshape(-1))

    @classmethod
    def from_reader(cls, reader: QStoreReader) -> "PinnedHostTier":
        names = reader.qrow_names()
        shapes = {n: tuple(int(v) for v in reader.blocks[n]["shape"]) for n in names}
        tier = cls(shapes)
        for n in names:
            codes, scales = reader.qrow(n)
            tier.put(n, codes, scales)
        return tier

    @classmethod
    def from_pages(cls, pages: dict[str, CompactQRowPage]) -> "PinnedHostTier":
        tier = cls({n: (p.out_features, p.in_features) for n, p in pages.items()})
        for n, p in pages.items():
            tier.put(n, p.codes, p.scales)
        return tier

    @property
    def max_slot_bytes(self) -> int:
        return max((_align(b.span, 256) for b in self.blocks.values()), default=256)


class MappedStagingTier:
    """Bounded pinned staging between a memory-mapped store and the HBM ring.

    The bounded mode of the paged path, for stores that do not fit in pinned memory (the
    reference's ring stages every block this way, qstore.py:613-659): ``buffers`` pinned
    buffers of the largest block's slot span, allocated once on the calling thread.
    ``fill(j, name)`` copies one block's codes and scales from the store's mapping into
    buffer ``j`` in the slot layout ``[codes][pad to 256][scales]`` on a worker thread,
    the codes in ``chunk_bytes`` pieces over ``copy_threads`` threads (the copies release
    the interpreter lock, so the pieces run in parallel); the ring then issues the H2D
    from that buffer.  Only the caller's thread talks to the pager.

    Defaults, from a sweep of the config-2 decode pass on a 16-CPU host (H2D GB/s in the
    bounded mode): 4 MiB pieces over 8 threads 27.5 (12 threads 28.7); 8 MiB pieces 21.1
    whatever the thread count (a block of at most 13.8 MB is two pieces); 2 MiB 26.1
    (8 threads) falling with more threads; 1 MiB 16.9.
    """

    def __init__(self, reader: QStoreReader, *, buffers: int = 3, copy_threads: int | None = None,
                 chunk_bytes: int = 4 << 20):
        from concurrent.futures import ThreadPoolExecutor

        if copy_threads is None:
            copy_threads = min(8, max(1, (os.cpu_count() or 2) // 2))
        if buffers < 1 or copy_threads < 1 or chunk_bytes < 1:
            raise ValueError("staging needs at least one buffer, one copy thread and a positive chunk")
        self.reader = reader
        self.blocks: dict[str, HostBlock] = {}
        for name in reader.qrow_names():
            out, inn = (int(v) for v in reader.blocks[name]["shape"])
            self.blocks[name] = HostBlock(name, out, inn, 0, _slot_layout(out, inn))
        self.buffer_bytes = _align(max((b.span for b in self.blocks.values()), default=256), 4096)
        self.buffers = [torch.empty(self.buffer_bytes, dtype=torch.uint8, pin_memory=True) for _ in range(buffers)]
        self.nbytes = self.buffer_bytes * len(self.buffers)
        self.chunk_bytes = int(chunk_bytes)
        self._worker = ThreadPoolExecutor(max_workers=1, thread_name_prefix="qstore-stage")
        self._copiers = ThreadPoolExecutor(max_workers=int(copy_threads), thread_name_prefix="qstore-stage-cp")
        self.stats = {"staged_blocks": 0, "staged_bytes": 0}

    @property
    def max_slot_bytes(self) -> int:
        return max((_align(b.span, 256) for b in self.blocks.values()), default=256)

    def codes(self, name: str) -> np.ndarray:
        return self.reader.qrow(name)[0]

    def scales(self, name: str) -> np.ndarray:
        return self.reader.qrow(name)[1]

    def buffer_ptr(self, j: int) -> int:
        return self.buffers[j].data_ptr()

    def _copy(self, j: int, name: str) -> None:
        b = self.blocks[name]
        codes, scales = self.reader.qrow(name)
        dst = self.buffers[j].numpy()
        n = b.out_features * b.in_features
        src = np.asarray(codes).reshape(-1).view(np.uint8)
        pieces = [(a, min(n, a + self.chunk_bytes)) for a in range(0, n, self.chunk_bytes)]
        if len(pieces) > 2:
            for f in [self._copiers.submit(np.copyto, dst[a:e], src[a:e]) for a, e in pieces]:
                f.result()
        else:
            np.copyto(dst[:n], src)
        sc = np.asarray(scales, dtype=np.float32).reshape(-1).view(np.uint8)
        np.copyto(dst[b.scale_offset:b.scale_offset + sc.size], sc)
        self.stats["staged_blocks"] += 1
        self.stats["staged_bytes"] += b.span

    def fill(self, j: int, name: str):
        """Start copying block ``name`` into buffer ``j``; returns its future."""
        return self._worker.submit(self._copy, j, name)

    def close(self) -> None:
        self._worker.shutdown(wait=True)
        self._copiers.shutdown(wait=True)


class RingPrefetch:
    """Successor-oracle prefetch ring over HBM slots (qstore.py:486-660 ``_RingPrefetch``).

    With a ``PinnedHostTier`` every transfer reads the tier in place.  With a
    ``MappedStagingTier`` a block first goes through one of its pinned buffers: a prefetch
    starts the buffer fill on the staging worker and its H2D is issued by the first ring
    call after the fill has finished (or by ``take`` of that block, which waits for it);
    a buffer is refilled only after the H2D that read it has landed.
    """

    def __init__(self, tier: PinnedHostTier, device: torch.device, *, slots: int = 3, depth: int = 2,
                 page_bytes: int = PAGE_BYTES, transfer_bytes: int = TRANSFER_BYTES):
        if device.type != "cuda":
            raise RuntimeError("ring prefetch requires a HIP device")
        self.tier = tier
        self.device = device
        self.depth = max(1, int(depth))
        self.n_slots = max(2, int(slots))
        self.slot_bytes = tier.max_slot_bytes
        self.page_bytes = int(page_bytes)
        self.transfer_bytes = int(transfer_bytes)
        if self.page_bytes <= 0 or self.transfer_bytes <= 0:
            raise ValueError("page_bytes and transfer_bytes must be positive")
        self.arena = torch.empty(self.slot_bytes * self.n_slots, dtype=torch.uint8, device=device)
        handle = ctypes.c_void_p()
        with torch.cuda.device(device):
            nat.call("qs_pager_create", nat.ptr(self.arena), self.slot_bytes, self.n_slots, self.transfer_bytes,
                     ctypes.byref(handle))
        self._pager = handle
        self.held = [0] * self.n_slots
        self.staging = tier if isinstance(tier, MappedStagingTier) else None
        n_buf = len(self.staging.buffers) if self.staging is not None else 0
        # staging buffer j: None (free), ("fill", name) while its copy runs, or ("h2d", slot)
        # until the transfer that reads it has landed
        self._buf_state: list = [None] * n_buf
        self._pending: OrderedDict[str, tuple[int, object, int]] = OrderedDict()  # name -> (buffer, fill, slot)
        self.inflight: OrderedDict[str, int] = OrderedDict()
        self.successor: dict[str, str] = {}
        self.last_access: str | None = None
        self.stats = {
            "hits": 0,
            "misses": 0,
            "prefetches": 0,
            "prefetch_bytes": 0,
            "evicted_unused": 0,
            "successor_entries": 0,
            "h2d_bytes": 0,
            "h2d_pages": 0,
            "staging_waits": 0,
        }

    # -- lifecycle -----------------------------------------------------------------
    def close(self) -> None:
        for _, fill, _ in self._pending.values():
            fill.result()
        self._pending.clear()
        if self._pager is not None:
            torch.cuda.current_stream(self.device).synchronize()
            nat.call("qs_pager_destroy", self._pager)
            self._pager = None
        self.inflight.clear()
        self.arena = None

    def allocated_bytes(self) -> int:
        return 0 if self.arena is None else int(self.arena.numel())

    # -- serving -------------------------------------------------------------------
    def _page(self, slot: int, name: str) -> CompactQRowPage:
        b = self.tier.blocks[name]
        base = slot * self.slot_bytes
        codes = self.arena[base : base + b.out_features * b.in_features].view(torch.int8)
        codes = codes.view(b.out_features, b.in_features)
        a = base + b.scale_offset
        scales = self.arena[a : a + b.out_features * 4].view(torch.float32)
        return CompactQRowPage(name, 0, b.out_features, b.in_features, codes, scales)

    def take(self, name: str) -> CompactQRowPage | None:
        """Prefetched page for ``name`` (ordered after its copy on the current stream) or None."""
        self._pump()
        slot = self.inflight.pop(name, None)
        if slot is None:
            self.stats["misses"] += 1
            return None
        self.stats["hits"] += 1
        if name in self._pending:  # its fill is still running: wait for it, then copy
            j, fill, _ = self._pending.pop(name)
            fill.result()
            self._send_staged(j, slot, name)
        return self._hold(slot, name)

    def load(self, name: str) -> CompactQRowPage:
        """Miss path: copy ``name`` into a slot now and hand it out."""
        slot = self._issue(name)
        self.inflight.pop(name, None)
        if name in self._pending:
            j, fill, _ = self._pending.pop(name)
            fill.result()
            self._send_staged(j, slot, name)
        return self._hold(slot, name)

    def _hold(self, slot: int, name: str) -> CompactQRowPage:
        stream = torch.cuda.current_stream(self.device).cuda_stream
        nat.call("qs_pager_acquire", self._pager, slot, stream)
        self.held[slot] += 1
        return self._page(slot, name)

    def release(self, page: CompactQRowPage) -> None:
        """Consumer finished queueing its reads of ``page`` on the current stream."""
        slot = (page.codes.data_ptr() - self.arena.data_ptr()) // self.slot_bytes
        if not 0 <= slot < self.n_slots or self.held[slot] <= 0:
            raise RuntimeError(f"page {page.name!r} is not held from this ring")
        stream = torch.cuda.current_stream(self.device).cuda_stream
        nat.call("qs_pager_release", self._pager, slot, stream)
        self.held[slot] -= 1

    def observe(self, name: str) -> None:
        """Record access order and prefetch the predicted successors (qstore.py:561-573)."""
        self._pump()
        if self.last_access is not None and self.last_access != name:
            self.successor[self.last_access] = name
            self.stats["successor_entries"] = len(self.successor)
        self.last_access = name
        chain, nxt = [], name
        for _ in range(self.depth):
            nxt = self.successor.get(nxt)
            if nxt is None:
                break
            chain.append(nxt)
        wanted = set(chain)
        for nxt in chain:
            if nxt in self.inflight or nxt not in self.tier.blocks:
                continue
            slot = self._free_slot(protect=wanted)
            if slot is None:
                return
            if self.staging is not None:
                j = self._free_buffer(block=False)
                if j is None:  # every buffer is being filled: no prefetch this time
                    return
                self._start_fill(j, slot, nxt)
            else:
                self._submit(slot, nxt)
            self.stats["prefetches"] += 1
            self.stats["prefetch_bytes"] += self.tier.blocks[nxt].compact_bytes

    # -- staging -------------------------------------------------------------------
    def _free_slot(self, protect: set[str] = frozenset()) -> int | None:
        busy = set(self.inflight.values())
        for s in range(self.n_slots):
            if s not in busy and not self.held[s]:
                return s
        # oldest unconsumed prefetch outside the predicted chain: a mispredict
        for key, s in list(self.inflight.items()):
            if not self.held[s] and key not in protect:
                self.inflight.pop(key)
                if key in self._pending:  # its fill may still be running: let it end, unsent
                    j, fill, _ = self._pending.pop(key)
                    fill.result()
                    self._buf_state[j] = None
                self.stats["evicted_unused"] += 1
                return s
        return None

    # -- bounded staging (MappedStagingTier) -----------------------------------------------
    def _start_fill(self, j: int, slot: int, name: str) -> None:
        self._buf_state[j] = ("fill", name)
        self._pending[name] = (j, self.staging.fill(j, name), slot)
        self.inflight[name] = slot

    def _send_staged(self, j: int, slot: int, name: str) -> None:
        """H2D of a filled staging buffer into its slot; the buffer stays busy until it lands."""
        b = self.tier.blocks[name]
        nat.call("qs_pager_submit", self._pager, slot, self.staging.buffer_ptr(j), b.span, 0)
        nat.call("qs_pager_seal", self._pager, slot)
        self._buf_state[j] = ("h2d", slot)
        self.stats["h2d_bytes"] += b.span
        self.stats["h2d_pages"] += -(-b.span // self.page_bytes)

    def _pump(self) -> None:
        """Issue the H2D of every prefetch whose buffer fill has finished (in order)."""
        for name, (j, fill, slot) in list(self._pending.items()):
            if not fill.done():
                break
            fill.result()
            del self._pending[name]
            self._send_staged(j, slot, name)

    def _free_buffer(self, *, block: bool) -> int | None:
        """A staging buffer that may be refilled: a free one, else one whose transfer has
        landed; with ``block``, wait for the oldest transfer (or fill) to end."""
        for j, st in enumerate(self._buf_state):
            if st is None:
                return j
        for j, st in enumerate(self._buf_state):
            if st[0] == "h2d" and nat.load().qs_pager_slot_landed(self._pager, st[1]) == 1:
                self._buf_state[j] = None
                return j
        if not block:
            return None
        self.stats["staging_waits"] += 1
        for j, st in enumerate(self._buf_state):
            if st[0] == "h2d":
                nat.call("qs_pager_wait_landed", self._pager, st[1])
                self._buf_state[j] = None
                return j
        # every buffer is filling for a prefetch: send the oldest, then wait for it to land
        name, (j, fill, slot) = next(iter(self._pending.items()))
        fill.result()
        del self._pending[name]
        self._send_staged(j, slot, name)
        nat.call("qs_pager_wait_landed", self._pager, slot)
        self._buf_state[j] = None
        return j

    def _issue(self, name: str) -> int:
        slot = self.inflight.get(name)
        if slot is not None:
            return slot
        slot = self._free_slot()
        if slot is None:
            raise RuntimeError("every ring slot is held by an unreleased page")
        self._submit(slot, name)
        return slot

    def _submit(self, slot: int, name: str) -> None:
        if self.staging is not None:  # a miss: stage it now and send it
            j = self._free_buffer(block=True)
            self._buf_state[j] = ("fill", name)
            self.staging.fill(j, name).result()
            self.inflight[name] = slot
            self._send_staged(j, slot, name)
            return
        b = self.tier.blocks[name]
        src = self.tier.host.data_ptr() + b.host_offset
        nat.call("qs_pager_submit", self._pager, slot, src, b.span, 0)
        nat.call("qs_pager_seal", self._pager, slot)
        self.inflight[name] = slot
        self.stats["h2d_bytes"] += b.span
        self.stats["h2d_pages"] += -(-b.span // self.page_bytes)


class PagedQStore:
    """int8 QStore served from pinned host memory through the HBM slot ring.

    Store surface as ``QStore`` (qstore.py:1008-1185): ``has``, ``fp32``, ``weight``,
    ``matmul``, ``matmul_row_stable``, ``row_blocks``, ``close``, plus the ring controls
    ``enable_ring`` / ``disable_ring`` / ``ring_stats`` / ``ring_allocated_bytes`` and the
    DenseQStore extra ``fused_swiglu``.  With the ring disabled every block is a miss
    (copied on demand through the same slots), which is the reference's plain paged path.
    """

    def __init__(
        self,
        store: QStoreReader | PinnedHostTier | str | Path,
        *,
        device: str | torch.device = "cuda",
        compute_dtype: str | None = "bf16",
        slots: int = 3,
        depth: int = 2,
        page_bytes: int = PAGE_BYTES,
        transfer_bytes: int = TRANSFER_BYTES,
        enable_prefetch_ring: bool = True,
        staging_buffers: int | None = None,
    ) -> None:
        """``staging_buffers=None``: every qrow block is copied once into one pinned host tier
        (the store must fit in pinned memory).  ``staging_buffers=K``: bounded mode -- only K
        pinned buffers of the largest block, refilled from the store's mapping for every
        transfer (a store of any size)."""
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("PagedQStore requires a HIP (cuda) device")
        if compute_dtype not in _DTYPES:
            raise ValueError("compute_dtype must be fp32, bf16 or fp16")
        self.compute_dtype = _DTYPES[compute_dtype]
        self.reader: QStoreReader | None = None
        if isinstance(store, (PinnedHostTier, MappedStagingTier)):
            if staging_buffers is not None:
                raise ValueError("staging_buffers applies to a store directory or reader, not a host tier")
            self.tier = store
            self.reader = store.reader if isinstance(store, MappedStagingTier) else None
        else:
            self.reader = store if isinstance(store, QStoreReader) else QStoreReader(store)
            if staging_buffers is None:
                self.tier = PinnedHostTier.from_reader(self.reader)
            else:
                self.tier = MappedStagingTier(self.reader, buffers=int(staging_buffers))
        self.ring = RingPrefetch(self.tier, self.device, slots=slots, depth=depth, page_bytes=page_bytes,
                                 transfer_bytes=transfer_bytes)
        self.prefetch = bool(enable_prefetch_ring)
        self.stats = DenseQStoreStats()

    # ---- ring controls ----------------------------------------------------------------
    def enable_ring(self, *, slots: int | None = None, depth: int = 2) -> None:
        if slots is not None and max(2, int(slots)) != self.ring.n_slots:
            self.ring.close()
            self.ring = RingPrefetch(self.tier, self.device, slots=slots, depth=depth, page_bytes=self.ring.page_bytes,
                                     transfer_bytes=self.ring.transfer_bytes)
        self.ring.depth = max(1, int(depth))
        self.prefetch = True

    def disable_ring(self) -> None:
        self.prefetch = False

    def ring_stats(self) -> dict[str, int] | None:
        return dict(self.ring.stats) if self.prefetch else None

    def ring_allocated_bytes(self) -> int:
        return self.ring.allocated_bytes() + self.tier.nbytes

    # ---- store surface ------------------------------------------------------------------
    def _physical(self, name: str) -> str:
        if self.reader is not None:
            key = str(name)
            seen: set[str] = set()
            while True:
                if key in seen:
                    raise RuntimeError(f"cyclic QStore alias at {name!r}")
                seen.add(key)
                blk = self.reader.blocks.get(key)
                if blk is None:
                    raise KeyError(f"QStore has no block {key!r}")
                if "alias" not in blk:
                    break
                key = str(blk["alias"])
        else:
            key = str(name)
        if key not in self.tier.blocks:
            raise KeyError(f"QStore has no qrow block {name!r}")
        return key

    def has(self, name: str) -> bool:
        if self.reader is not None:
            return self.reader.has(name)
        return str(name) in self.tier.blocks

    def fp32(self, name: str) -> torch.Tensor:
        if self.reader is None:
            raise KeyError(f"QStore has no fp32 block {name!r}")
        return torch.from_numpy(self.reader.fp32(name)).to(self.device)

    def block_kind(self, name: str) -> str | None:
        """``"qrow"`` / ``"fp32"`` of a block after alias resolution."""
        if self.reader is not None:
            return self.reader.block_kind(name)
        return "qrow" if str(name) in self.tier.blocks else None

    def embed_rows(self, name: str, ids) -> torch.Tensor:
        """fp32 rows ``ids`` of a qrow block, ``[*ids.shape, in]`` (qstore.py:1099-1128).  Only
        the selected rows leave the pinned host tier; the ring is not involved."""
        key = self._physical(name)
        codes, scales = self.tier.codes(key), self.tier.scales(key)
        flat, shape = _qrow.normalize_row_ids(ids, int(codes.shape[0]))
        uniq, inverse = np.unique(flat.reshape(-1), return_inverse=True)
        c = torch.from_numpy(np.ascontiguousarray(codes[uniq])).to(self.device)
        sc = torch.from_numpy(np.ascontiguousarray(scales[uniq])).to(self.device)
        return _qrow.qrow_embed_rows(c, sc, inverse.reshape(shape))

    def _acquire(self, name: str) -> CompactQRowPage:
        key = self._physical(name)
        page = self.ring.take(key) if self.prefetch else None
        if self.prefetch:
            self.ring.observe(key)
        if page is None:
            page = self.ring.load(key)
            self.stats.page_loads += 1
        else:
            self.stats.cache_hits += 1
        self.stats.compact_h2d_bytes += page.compact_bytes
        return page

    def _count(self, page: CompactQRowPage) -> None:
        self.stats.projection_calls += 1
        self.stats.native_projection_calls += 1
        self.stats.compact_logical_bytes += page.compact_bytes
        self.stats.expanded_compute_bytes_avoided += page.expanded_compute_bytes(self.compute_dtype)

    def weight(self, name: str) -> torch.Tensor:
        page = self._acquire(name)
        try:
            return _qrow.qrow_dequant(page.codes, page.scales, self.compute_dtype)
        finally:
            self.ring.release(page)

    def matmul(self, name: str, x: torch.Tensor) -> torch.Tensor:
        page = self._acquire(name)
        try:
            if x.dtype != self.compute_dtype:
                x = x.to(self.compute_dtype)
            y, _tag = _qrow.fused_qrow_matmul(page, x)
        finally:
            self.ring.release(page)
        self._count(page)
        return y

    def matmul_row_stable(self, name: str, x: torch.Tensor) -> torch.Tensor:
        if x.ndim < 2 or int(x.shape[0]) <= 0:
            raise ValueError("row-stable matmul input must have a leading request axis")
        page = self._acquire(name)
        try:
            if x.dtype != self.compute_dtype:
                x = x.to(self.compute_dtype)
            y = _qrow.qrow_matmul(page.codes, page.scales, x, row_stable=True)
        finally:
            self.ring.release(page)
        self._count(page)
        return y

    def fused_swiglu(self, gate_name: str, up_name: str, x: torch.Tensor) -> tuple[torch.Tensor, str]:
        g = self._acquire(gate_name)
        try:
            u = self._acquire(up_name)
            try:
                y, tag = _qrow.fused_qrow_swiglu(g, u, x)
            finally:
                self.ring.release(u)
        finally:
            self.ring.release(g)
        self._count(g)
        self._count(u)
        self.stats.paired_swiglu_calls += 1
        return y, tag

    def row_blocks(self, name: str, bs: int = 8192):
        W = self.weight(name)
        for start in range(0, W.shape[0], bs):
            end = min(start + bs, W.shape[0])
            yield start, end, W[start:end]

    def synchronize(self) -> None:
        nat.call("qs_pager_sync", self.ring._pager)
        torch.cuda.current_stream(self.device).synchronize()

    def close(self) -> None:
        if self.ring is not None:
            self.ring.close()
        self.ring = None
        if isinstance(self.tier, MappedStagingTier):
            self.tier.close()
