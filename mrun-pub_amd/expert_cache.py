"""Paged int8 experts: page store, pinned host tier and HBM slot cache with route prefetch.

Mirrors the Qwen3 MoE page tier of the reference (src/mrun/engine/qwen3_moe_cuda.py):

* ``PackedInt8ExpertStore`` -- ``PackedFP8ExpertStore`` (:780-840): one flat file of
  ``[layers * experts, page_stride]`` pages in the ``ExpertPageLayout`` (:187-233) with
  1-byte int8 codes and fp32 row scales; ``global_page`` / ``gather`` / ``view_pages``.
* ``HostPageTier`` (:878-981): a budgeted pinned copy of pages, filled by one sequential
  ``warm()`` pass or admitted on first miss, never evicted.
* ``ExpertPageCache`` (:1221-1820): a device cache of ``capacity`` page slots with the
  reference's ``global-lru-v1`` / ``layer-frequency-lru-v1`` eviction, decode protection,
  the ``slot-indirect-v1`` binding (routed groups address cache slots directly through the
  grouped GEMM's ``group_slots``) and the ``compact-copy-v1`` binding, and opt-in
  route-history prefetch of the previous step's routes for layer + 1.

Design for the device: the cache arena is the slot array of a ``qs_pager`` (csrc/
qs_pager.cpp).  A miss is one H2D transfer straight from the pinned tier page into its
cache slot (no staging copy when the tier holds the page), on the pager's copy stream;
the compute stream waits on that slot's ready event; the slot's free event is recorded
after the kernels that read it, and a later fill of that slot waits for it on the host.
Route prefetches are the same transfers issued one layer early.
"""

from __future__ import annotations

import ctypes
import json
import os
from collections import Counter, OrderedDict
from dataclasses import dataclass, fields
from pathlib import Path
from typing import Any

import numpy as np
import torch

from . import _native as nat
from .moe import ExpertPageLayout, Int8ExpertLayer

STORE_SCHEMA = "mrun-hip-int8-expert-store-v1"
STORE_CODEC = "int8-qrow-experts-v1"
STORE_FILE = "experts.pages"

GLOBAL_LRU_CACHE_POLICY = "global-lru-v1"
LAYER_FREQUENCY_CACHE_POLICY = "layer-frequency-lru-v1"
SUPPORTED_CACHE_POLICIES = frozenset({GLOBAL_LRU_CACHE_POLICY, LAYER_FREQUENCY_CACHE_POLICY})
COMPACT_PAGE_BINDING_POLICY = "compact-copy-v1"
SLOT_INDIRECT_PAGE_BINDING_POLICY = "slot-indirect-v1"
DEFAULT_PAGE_BINDING_POLICY = SLOT_INDIRECT_PAGE_BINDING_POLICY
SUPPORTED_PAGE_BINDING_POLICIES = frozenset({COMPACT_PAGE_BINDING_POLICY, SLOT_INDIRECT_PAGE_BINDING_POLICY})
TRANSFER_BYTES = 64 << 20


# ---- page store -----------------------------------------------------------------------------


def write_int8_expert_store(store_dir: str | Path, gate_up, gate_up_scales, down, down_scales) -> Path:
    """Write ``[L,E,2I,H]`` int8 / ``[L,E,2I]`` f32 / ``[L,E,H,I]`` int8 / ``[L,E,H]`` f32 arrays
    as one page file plus ``manifest.json``; returns the store directory."""
    gate_up = np.asarray(gate_up, dtype=np.int8)
    down = np.asarray(down, dtype=np.int8)
    gate_up_scales = np.asarray(gate_up_scales, dtype=np.float32)
    down_scales = np.asarray(down_scales, dtype=np.float32)
    L, E, two_i, H = gate_up.shape
    I = two_i // 2
    if two_i != 2 * I or down.shape != (L, E, H, I) or gate_up_scales.shape != (L, E, two_i) \
            or down_scales.shape != (L, E, H):
        raise ValueError("expert arrays disagree on [layers, experts, 2I, H] / [layers, experts, H, I]")
    layout = ExpertPageLayout.create(H, I)
    root = Path(store_dir)
    root.mkdir(parents=True, exist_ok=True)
    pages = np.lib.format.open_memmap(root / (STORE_FILE + ".npy"), mode="w+", dtype=np.uint8,
                                      shape=(L * E, layout.page_stride))
    for layer in range(L):
        for expert in range(E):
            row = pages[layer * E + expert]
            row[:] = 0
            lo = layout.gate_up_codes_offset
            row[lo:lo + layout.gate_up_codes_bytes] = gate_up[layer, expert].reshape(-1).view(np.uint8)
            lo = layout.gate_up_scales_offset
            row[lo:lo + layout.gate_up_scales_bytes] = gate_up_scales[layer, expert].view(np.uint8)
            lo = layout.down_codes_offset
            row[lo:lo + layout.down_codes_bytes] = down[layer, expert].reshape(-1).view(np.uint8)
            lo = layout.down_scales_offset
            row[lo:lo + layout.down_scales_bytes] = down_scales[layer, expert].view(np.uint8)
    pages.flush()
    del pages
    manifest = {
        "schema_version": STORE_SCHEMA,
        "codec": STORE_CODEC,
        "layout": layout.as_dict(),
        "layers": int(L),
        "num_experts": int(E),
        "data_file": STORE_FILE + ".npy",
    }
    (root / "manifest.json").write_text(json.dumps(manifest, indent=1, sort_keys=True), encoding="utf-8")
    return root


class PackedInt8ExpertStore:
    """``[layers * experts, page_stride]`` int8 expert pages on disk (memory-mapped)."""

    def __init__(self, store_dir: str | Path):
        self.store_dir = Path(store_dir)
        self.manifest = json.loads((self.store_dir / "manifest.json").read_text(encoding="utf-8"))
        if self.manifest.get("schema_version") != STORE_SCHEMA:
            raise ValueError("unsupported int8 expert store schema")
        if self.manifest.get("codec") != STORE_CODEC:
            raise ValueError("unsupported int8 expert store codec")
        self.layout = ExpertPageLayout.from_dict(self.manifest["layout"])
        self.layers = int(self.manifest["layers"])
        self.experts = int(self.manifest["num_experts"])
        self.data_path = self.store_dir / self.manifest["data_file"]
        self._pages: np.ndarray | None = None
        pages = self._ensure_pages()
        if pages.shape != (self.layers * self.experts, self.layout.page_stride):
            raise ValueError("expert page file does not match the manifest")

    def _ensure_pages(self) -> np.ndarray:
        if self._pages is None:
            self._pages = np.load(self.data_path, mmap_mode="r", allow_pickle=False)
        return self._pages

    def global_page(self, layer: int, expert: int) -> int:
        return layer * self.experts + expert

    def page(self, gid: int) -> np.ndarray:
        return self._ensure_pages()[gid]

    def gather(self, layer: int, expert_ids: list[int], target: torch.Tensor) -> None:
        if not expert_ids:
            return
        if target.device.type != "cpu" or target.dtype != torch.uint8:
            raise ValueError("expert page staging target must be a CPU uint8 tensor")
        view = target[: len(expert_ids)].numpy()
        rows = layer * self.experts + np.asarray(expert_ids, dtype=np.int64)
        np.take(self._ensure_pages(), rows, axis=0, out=view)

    def view_pages(self, raw: torch.Tensor) -> Int8ExpertLayer:
        """Expert-page views ``gate_up / gate_up_scales / down / down_scales`` over ``raw``
        ``[groups, page_stride]`` (no copies)."""
        if raw.dtype != torch.uint8 or raw.ndim != 2 or raw.shape[1] != self.layout.page_stride:
            raise ValueError("expert pages must be uint8 [groups, page_stride]")
        return Int8ExpertLayer(raw.reshape(-1), self.layout, int(raw.shape[0]))

    def release(self) -> None:
        self._pages = None


class HostPageTier:
    """Budgeted pinned host copy of expert pages (fill once, no eviction)."""

    def __init__(self, store: PackedInt8ExpertStore, *, host_cache_mb: float, try_pin: bool = True):
        self.store = store
        stride = store.layout.page_stride
        total_pages = store.layers * store.experts
        capacity = min(total_pages, int(float(host_cache_mb) * 1e6) // stride)
        if capacity < 1:
            raise ValueError("host_cache_mb smaller than one expert page")
        self.capacity = capacity
        self.pinned = False
        buf = None
        if try_pin:
            try:
                buf = torch.empty((capacity, stride), dtype=torch.uint8, pin_memory=True)
                self.pinned = True
            except RuntimeError:
                buf = None
        if buf is None:
            buf = torch.empty((capacity, stride), dtype=torch.uint8)
        self.buf = buf
        self._buf_np = buf.numpy()
        self._rows = np.full(total_pages, -1, dtype=np.int64)
        self._next_row = 0
        self.stats = {"capacity_pages": capacity, "pinned": self.pinned, "warmed_pages": 0,
                      "served_pages": 0, "admitted_pages": 0, "disk_pages": 0}

    def warm(self) -> dict[str, Any]:
        """Fill rows [next, capacity) with pages [next, capacity) in one sequential pass."""
        pages = self.store._ensure_pages()
        start, stop = self._next_row, self.capacity
        chunk = max(1, (256 << 20) // self.store.layout.page_stride)
        for lo in range(start, stop, chunk):
            hi = min(stop, lo + chunk)
            self._buf_np[lo:hi] = pages[lo:hi]
        self._rows[start:stop] = np.arange(start, stop, dtype=np.int64)
        self._next_row = stop
        self.stats["warmed_pages"] = stop
        return dict(self.stats)

    def host_page(self, layer: int, expert: int) -> torch.Tensor | None:
        """The tier's row for a page (admitting it while capacity remains), else None."""
        gid = self.store.global_page(layer, expert)
        row = int(self._rows[gid])
        if row >= 0:
            self.stats["served_pages"] += 1
            return self.buf[row]
        if self._next_row >= self.capacity:
            self.stats["disk_pages"] += 1
            return None
        row = self._next_row
        self._next_row += 1
        np.copyto(self._buf_np[row], self.store.page(gid))
        self._rows[gid] = row
        self.stats["admitted_pages"] += 1
        return self.buf[row]

    def gather(self, layer: int, expert_ids: list[int], target: torch.Tensor) -> None:
        """Fill ``target[:len(expert_ids)]`` from the tier where present, disk otherwise."""
        view = target[: len(expert_ids)].numpy()
        for i, expert in enumerate(expert_ids):
            page = self.host_page(layer, expert)
            np.copyto(view[i], page.numpy() if page is not None else
                      self.store.page(self.store.global_page(layer, expert)))


# ---- slot policy (host logic) ---------------------------------------------------------------


@dataclass
class PageCacheStats:
    """Counters of qwen3_moe_cuda.py:983-1030 that this cache maintains."""

    page_requests: int = 0
    page_hits: int = 0
    page_misses: int = 0
    host_to_device_bytes: int = 0
    layer_acquires: int = 0
    active_experts_sum: int = 0
    evictions: int = 0
    same_layer_evictions: int = 0
    over_quota_evictions: int = 0
    fallback_evictions: int = 0
    decode_protected_promotions: int = 0
    decode_protected_demotions: int = 0

    def as_dict(self) -> dict[str, Any]:
        out = {f.name: getattr(self, f.name) for f in fields(self)}
        out["hit_rate"] = self.page_hits / max(1, self.page_requests)
        out["host_to_device_gb"] = self.host_to_device_bytes / 1e9
        out["mean_active_experts"] = self.active_experts_sum / max(1, self.layer_acquires)
        return out


class SlotPolicy:
    """Which cache slot holds which (layer, expert) page, and which page to evict.

    ``global-lru-v1`` evicts the least recently used unprotected page;
    ``layer-frequency-lru-v1`` first evicts within the incoming layer once it is at its
    quota, then any layer above its quota, then falls back to global LRU
    (qwen3_moe_cuda.py:1415-1488).  Pages requested by the current acquire are never
    evicted; decode-protected pages lose protection when evicted.
    """

    def __init__(self, capacity: int, layers: int, policy: str, stats: PageCacheStats, on_change=None):
        if policy not in SUPPORTED_CACHE_POLICIES:
            raise ValueError(f"unsupported expert cache policy {policy!r}; "
                             f"expected one of {sorted(SUPPORTED_CACHE_POLICIES)}")
        self.capacity = capacity
        self.policy = policy
        self.stats = stats
        self.entries: OrderedDict[tuple[int, int], int] = OrderedDict()
        self.decode_protected: set[tuple[int, int]] = set()
        self.free_slots = list(range(capacity - 1, -1, -1))
        quota, remainder = divmod(capacity, layers)
        self.layer_quotas = tuple(quota + (1 if layer < remainder else 0) for layer in range(layers))
        self.layer_entry_counts = [0] * layers
        # on_change(key, slot): key now lives in slot (-1: key left the cache)
        self.on_change = on_change

    def reset(self) -> None:
        if self.on_change is not None:
            for key in self.entries:
                self.on_change(key, -1)
        self.entries.clear()
        self.decode_protected.clear()
        self.free_slots = list(range(self.capacity - 1, -1, -1))
        self.layer_entry_counts = [0] * len(self.layer_entry_counts)

    def victim(self, incoming_layer: int, protected) -> tuple[tuple[int, int] | None, str]:
        """The page to evict for a page of ``incoming_layer`` and the statistics counter it
        counts under, from one scan of the pages in LRU order (oldest first), skipping
        ``protected`` (the current acquire's pages):

        * global LRU: the oldest page (``fallback_evictions``);
        * layer-frequency LRU: the oldest page of the incoming layer when that layer holds
          at least its quota (``same_layer_evictions``), else the oldest page of any layer
          above its quota (``over_quota_evictions``), else the oldest page
          (``fallback_evictions``).

        ``None`` when every cached page is protected."""
        counts, quotas = self.layer_entry_counts, self.layer_quotas
        layer_full = counts[incoming_layer] >= quotas[incoming_layer]
        oldest = over = None
        for key in self.entries:
            if key in protected:
                continue
            if self.policy == GLOBAL_LRU_CACHE_POLICY:
                return key, "fallback_evictions"
            if layer_full and key[0] == incoming_layer:
                return key, "same_layer_evictions"  # the rule that ranks first decides at once
            if oldest is None:
                oldest = key
            if over is None and counts[key[0]] > quotas[key[0]]:
                over = key
        if over is not None:
            return over, "over_quota_evictions"
        return oldest, "fallback_evictions"

    def reserve(self, key, protected) -> int:
        """A slot for ``key`` (a free one, else the victim's), recorded as most recently used."""
        if self.free_slots:
            slot = self.free_slots.pop()
        else:
            victim, counter = self.victim(key[0], protected)
            if victim is None:
                raise RuntimeError("no expert page can be evicted: every cached page belongs to the active set")
            slot = self._evict(victim, counter)
        self.entries[key] = slot
        self.layer_entry_counts[key[0]] += 1
        if self.on_change is not None:
            self.on_change(key, slot)
        return slot

    def _evict(self, victim, counter: str) -> int:
        slot = self.entries.pop(victim)
        self.layer_entry_counts[victim[0]] -= 1
        if victim in self.decode_protected:  # a protected page loses protection with its slot
            self.decode_protected.discard(victim)
            self.stats.decode_protected_demotions += 1
        self.stats.evictions += 1
        setattr(self.stats, counter, getattr(self.stats, counter) + 1)
        if self.on_change is not None:
            self.on_change(victim, -1)
        return slot


# ---- device cache ---------------------------------------------------------------------------


class ExpertPageCache:
    """HBM cache of expert pages with slot binding for the grouped int8 GEMM."""

    def __init__(
        self,
        store: PackedInt8ExpertStore,
        *,
        device: str | torch.device,
        cache_mb: float,
        max_active_pages: int,
        host_tier: HostPageTier | None = None,
        route_prefetch: bool | None = None,
        cache_policy: str | None = None,
        page_binding_policy: str | None = None,
    ):
        self.store = store
        self.layout = store.layout
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("ExpertPageCache requires a HIP (cuda) device")
        self.host_tier = host_tier
        if route_prefetch is None:
            route_prefetch = os.environ.get("MRUN_QWEN3_MOE_ROUTE_PREFETCH", "").strip() not in ("", "0")
        self.route_prefetch = bool(route_prefetch)
        policy = cache_policy if cache_policy is not None else \
            os.environ.get("MRUN_QWEN3_MOE_CACHE_POLICY", GLOBAL_LRU_CACHE_POLICY)
        binding = page_binding_policy if page_binding_policy is not None else \
            os.environ.get("MRUN_QWEN3_MOE_PAGE_BINDING_POLICY", DEFAULT_PAGE_BINDING_POLICY)
        self.page_binding_policy = str(binding).strip().lower()
        if self.page_binding_policy not in SUPPORTED_PAGE_BINDING_POLICIES:
            raise ValueError(f"unsupported expert page binding policy {self.page_binding_policy!r}; "
                             f"expected one of {sorted(SUPPORTED_PAGE_BINDING_POLICIES)}")
        stride = self.layout.page_stride
        requested = int(float(cache_mb) * 1e6) // stride
        self.capacity = min(store.layers * store.experts, max(int(max_active_pages), requested))
        self.max_active_pages = int(max_active_pages)
        self._stats = PageCacheStats()
        # device route -> slot table: slot_table[layer, expert] = cache slot or -1, kept equal
        # to the policy's entries (host mirror updated on every change, dirty rows copied
        # to the device before a kernel reads them)
        self._slot_host = np.full((store.layers, store.experts), -1, dtype=np.int32)
        self.slot_table = torch.full((store.layers, store.experts), -1, dtype=torch.int32, device=self.device)
        self._dirty_layers: set[int] = set()
        self._layer_slot_arrays: dict[int, Any] = {}
        # routes of device-table layers whose bookkeeping has not been applied yet
        self._deferred: list[tuple[int, torch.Tensor, bool]] = []
        self.device_table_stats = {"device_table_layers": 0, "deferred_drains": 0}
        self.policy = SlotPolicy(self.capacity, store.layers, str(policy).strip().lower(), self._stats,
                                 on_change=self._slot_changed)
        self.cache_policy = self.policy.policy
        self.cache = torch.empty((self.capacity, stride), dtype=torch.uint8, device=self.device)
        # pinned staging for pages the host tier does not hold (read from the store file)
        self.stage = torch.empty((self.max_active_pages, stride), dtype=torch.uint8, pin_memory=True)
        self.compact = torch.empty((self.max_active_pages, stride), dtype=torch.uint8, device=self.device) \
            if self.page_binding_policy == COMPACT_PAGE_BINDING_POLICY else None
        handle = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            nat.call("qs_pager_create", nat.ptr(self.cache), stride, self.capacity, TRANSFER_BYTES,
                     ctypes.byref(handle))
        self._pager = handle
        self._pending_release: list[int] = []
        self._stage_in_flight = False
        self._prev_routes: dict[int, list[int]] = {}
        self._prefetched: set[tuple[int, int]] = set()  # prefetched pages no acquire has used yet
        self.prefetch_stats = {"prefetched_pages": 0, "prefetch_rounds": 0, "wasted_prefetches": 0}

    # -- reference surface ------------------------------------------------------------------
    @property
    def stats(self) -> PageCacheStats:
        self._drain_deferred()
        return self._stats

    @property
    def entries(self) -> OrderedDict:
        self._drain_deferred()
        return self.policy.entries

    @property
    def decode_protected(self) -> set:
        self._drain_deferred()
        return self.policy.decode_protected

    @property
    def device_bytes(self) -> int:
        n = self.cache.numel() + (self.compact.numel() if self.compact is not None else 0)
        return int(n)

    def reset(self, *, clear_pages: bool) -> None:
        self.synchronize()
        self._deferred.clear()
        self._stats.__init__()
        self.prefetch_stats = {"prefetched_pages": 0, "prefetch_rounds": 0, "wasted_prefetches": 0}
        self._prev_routes.clear()
        self._prefetched.clear()
        if clear_pages:
            self.policy.reset()

    def acquire_slot_binding(self, layer: int, top_indices: torch.Tensor, *, protect: bool = False):
        """``(selected_experts, page views of the whole cache, slots)``: routed groups address
        their cache slots directly (the grouped GEMM's ``group_slots``)."""
        selected, slots = self._acquire_resident(layer, top_indices, protect=protect)
        return selected, self.store.view_pages(self.cache), slots

    def acquire_layer_table(self, layer: int, top_indices: torch.Tensor, *, protect: bool = False):
        """Fast binding for a layer whose every expert page is resident: ``(page views of
        the whole cache, slot_table[layer])``, a device int32 ``[experts]`` row that the
        grouped GEMMs index by expert id, or ``None`` when some page of the layer is not
        in the cache (then use ``acquire_slot_binding``).

        No host synchronisation: the routes are kept on the device and their bookkeeping
        (LRU touches in admission order, decode protection, hit statistics) is applied, in
        call order, before the next decision that depends on it -- the next acquire that
        may evict, or any read of ``stats`` / ``entries`` / ``decode_protected``.  With
        every page of the layer resident nothing is filled or evicted, so the deferred
        updates leave the cache in the state the synchronous path would have left it in.
        Route prefetch reads the routes on the host, so it turns this binding off, and so
        does the compact-copy binding policy."""
        if (self.route_prefetch or self.page_binding_policy != SLOT_INDIRECT_PAGE_BINDING_POLICY
                or self.policy.layer_entry_counts[int(layer)] != self.store.experts):
            return None
        layer = int(layer)
        self.release()
        self._push_slot_table()
        arr = self._layer_slot_arrays.get(layer)
        if arr is None:
            arr = self._layer_slot_arrays[layer] = (ctypes.c_int * self.store.experts)(*self._slot_host[layer].tolist())
        nat.call("qs_pager_acquire_many", self._pager, arr, self.store.experts, nat.stream_of(self.device))
        self._pending_release = arr
        self._deferred.append((layer, top_indices.detach().reshape(-1).clone(), bool(protect)))
        self.device_table_stats["device_table_layers"] += 1
        if len(self._deferred) >= 64:  # bound the device copies held
            self._drain_deferred()
        return self.store.view_pages(self.cache), self.slot_table[layer]

    def acquire(self, layer: int, top_indices: torch.Tensor, *, protect: bool = False):
        """``(selected_experts, page views of a compact copy)`` (the compact binding)."""
        selected, slots = self._acquire_resident(layer, top_indices, protect=protect)
        if self.compact is None:
            self.compact = torch.empty((self.max_active_pages, self.layout.page_stride), dtype=torch.uint8,
                                       device=self.device)
        n = int(selected.numel())
        torch.index_select(self.cache, 0, slots, out=self.compact[:n])
        return selected, self.store.view_pages(self.compact[:n])

    def release(self) -> None:
        """Mark the pages of the last acquire free once the work queued so far on the current
        stream is done (also done implicitly by the next acquire)."""
        pend = self._pending_release
        if len(pend):
            slots = pend if isinstance(pend, ctypes.Array) else (ctypes.c_int * len(pend))(*pend)
            nat.call("qs_pager_release_many", self._pager, slots, len(slots), nat.stream_of(self.device))
        self._pending_release = []

    def preload(self, layers=None) -> int:
        """Fill every page of ``layers`` (default: all) that is not resident, in layer order,
        as far as the cache holds them without evicting a page of a layer preloaded here.
        Returns the number of pages filled.  A layer whose pages are then all resident
        takes the device slot-table binding from its next call on."""
        self.release()
        self._drain_deferred()
        todo = range(self.store.layers) if layers is None else [int(l) for l in layers]
        guard: set[tuple[int, int]] = set()
        filled = 0
        for layer in todo:
            keys = [(layer, e) for e in range(self.store.experts)]
            guard.update(keys)
            missing = [k for k in keys if k not in self.policy.entries]
            for i in range(0, len(missing), self.max_active_pages):
                fills = []
                for key in missing[i:i + self.max_active_pages]:
                    try:
                        fills.append((key[1], self.policy.reserve(key, guard)))
                    except RuntimeError:
                        break  # full: the rest stays demand-filled
                if fills:
                    self._fill(layer, fills)
                    filled += len(fills)
                if len(fills) < len(missing[i:i + self.max_active_pages]):
                    return filled
        return filled

    def synchronize(self) -> None:
        nat.call("qs_pager_sync", self._pager)

    def close(self) -> None:
        if self._pager is not None:
            self.synchronize()
            nat.call("qs_pager_destroy", self._pager)
            self._pager = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- internals ----------------------------------------------------------------------------
    def _slot_changed(self, key, slot: int) -> None:
        if slot < 0 and key in self._prefetched:
            self._prefetched.discard(key)
            self.prefetch_stats["wasted_prefetches"] += 1  # evicted before any acquire used it
        layer, expert = key
        self._slot_host[layer, expert] = slot
        self._dirty_layers.add(int(layer))
        self._layer_slot_arrays.pop(int(layer), None)

    def _push_slot_table(self) -> None:
        """Copy changed rows of the slot table to the device (ordered on the current stream
        before the kernels that read them; the copy is taken from the host mirror at the
        call, so later changes of the mirror do not race with it)."""
        for layer in sorted(self._dirty_layers):
            self.slot_table[layer].copy_(torch.from_numpy(self._slot_host[layer].copy()))
        self._dirty_layers.clear()

    def _drain_deferred(self) -> None:
        """Apply the bookkeeping of device-table layers in call order (one host sync)."""
        if not self._deferred:
            return
        pending, self._deferred = self._deferred, []
        flat = torch.cat([r for _, r, _ in pending]).cpu().tolist()
        self.device_table_stats["deferred_drains"] += 1
        pos = 0
        for layer, routes, protect in pending:
            n = int(routes.numel())
            self._touch(layer, flat[pos:pos + n], protect)
            pos += n

    def _admission(self, layer: int, routed: list[int]):
        frequencies = Counter(routed)
        expert_ids = sorted(frequencies)
        keys = [(int(layer), e) for e in expert_ids]
        admission = keys
        if self.cache_policy == LAYER_FREQUENCY_CACHE_POLICY:
            admission = sorted(keys, key=lambda k: (frequencies[k[1]], k[1]))
        return expert_ids, keys, admission

    def _touch(self, layer: int, routed: list[int], protect: bool) -> None:
        """Bookkeeping of an acquire whose pages were all resident (no fills)."""
        _, keys, admission = self._admission(layer, [e for e in routed if 0 <= e < self.store.experts])
        self._prefetched.difference_update(keys)
        for key in admission:
            self.policy.entries.move_to_end(key)
        self._stats.page_requests += len(keys)
        self._stats.page_hits += len(keys)
        self._stats.layer_acquires += 1
        self._stats.active_experts_sum += len(keys)
        if protect:
            new = set(keys) - self.policy.decode_protected
            self.policy.decode_protected.update(keys)
            self._stats.decode_protected_promotions += len(new)

    def _fill(self, layer: int, misses: list[tuple[int, int]]) -> None:
        """One H2D transfer per missing page into its slot (pager copy stream)."""
        stride = self.layout.page_stride
        staged: list[tuple[int, int]] = []
        for expert, slot in misses:
            src = self.host_tier.host_page(layer, expert) if self.host_tier is not None else None
            if src is not None and self.host_tier.pinned:
                nat.call("qs_pager_submit", self._pager, slot, src.data_ptr(), stride, 0)
                nat.call("qs_pager_seal", self._pager, slot)
            else:
                staged.append((expert, slot))
        if staged:
            if self._stage_in_flight:  # the previous staging copies must have landed
                self.synchronize()
            rows = [e for e, _ in staged]
            if self.host_tier is not None:
                self.host_tier.gather(layer, rows, self.stage)
            else:
                self.store.gather(layer, rows, self.stage)
            for i, (_, slot) in enumerate(staged):
                nat.call("qs_pager_submit", self._pager, slot, self.stage[i].data_ptr(), stride, 0)
                nat.call("qs_pager_seal", self._pager, slot)
            self._stage_in_flight = True
        self._stats.host_to_device_bytes += len(misses) * stride

    def _acquire_resident(self, layer: int, top_indices: torch.Tensor, *, protect: bool):
        self.release()  # the previous acquire's kernels are queued: its slots may be refilled after them
        self._drain_deferred()  # earlier device-table layers' LRU touches precede any eviction here
        routed = top_indices.detach().reshape(-1).cpu().tolist()
        expert_ids, keys, admission = self._admission(layer, routed)
        if len(expert_ids) > self.max_active_pages:
            raise RuntimeError(f"active expert set {len(expert_ids)} exceeds staging limit {self.max_active_pages}")
        protected = set(keys)
        self._prefetched.difference_update(keys)
        misses: list[tuple[int, int]] = []
        for key in admission:
            if key in self.policy.entries:
                self.policy.entries.move_to_end(key)
                continue
            misses.append((key[1], self.policy.reserve(key, protected)))
        if misses:
            self._fill(int(layer), misses)
        slot_list = [self.policy.entries[k] for k in keys]
        if slot_list:
            nat.call("qs_pager_acquire_many", self._pager, (ctypes.c_int * len(slot_list))(*slot_list),
                     len(slot_list), nat.stream_of(self.device))
        self._pending_release = list(slot_list)
        self._stats.page_requests += len(keys)
        self._stats.page_misses += len(misses)
        self._stats.page_hits += len(keys) - len(misses)
        self._stats.layer_acquires += 1
        self._stats.active_experts_sum += len(keys)
        if protect:
            new = set(keys) - self.policy.decode_protected
            self.policy.decode_protected.update(keys)
            self._stats.decode_protected_promotions += len(new)
        if self.route_prefetch:
            self._prefetch_next_layer(int(layer), protected)
            self._prev_routes[int(layer)] = expert_ids
        selected = torch.tensor(expert_ids, dtype=torch.long, device=self.device)
        slots = torch.tensor(slot_list, dtype=torch.long, device=self.device)
        return selected, slots

    def _prefetch_next_layer(self, layer: int, protected: set) -> None:
        """Stage the previous step's routes for layer + 1 (qwen3_moe_cuda.py:1778-1815).

        Unlike the reference, the pages reserved in one round protect each other: the
        reference's round can evict a page it prefetched a moment earlier (a wasted
        transfer).  Results never depend on which pages are cached; prefetched pages that
        are evicted before any acquire uses them are counted as ``wasted_prefetches``."""
        nxt = layer + 1
        predicted = self._prev_routes.get(nxt)
        if not predicted:
            return
        wanted = [e for e in predicted if (nxt, e) not in self.policy.entries][: self.max_active_pages]
        fills: list[tuple[int, int]] = []
        guard = set(protected)
        for expert in wanted:
            key = (nxt, expert)
            try:
                fills.append((expert, self.policy.reserve(key, guard)))
            except RuntimeError:
                break  # the cache is saturated by the active set
            guard.add(key)
            self._prefetched.add(key)
        if not fills:
            return
        self._fill(nxt, fills)
        self.prefetch_stats["prefetched_pages"] += len(fills)
        self.prefetch_stats["prefetch_rounds"] += 1
