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
import hashlib
import json
import os
import time
from collections import Counter, OrderedDict
from dataclasses import dataclass, field, fields
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
CACHE_FILL_PREFILL_PAGE_POLICY = "cache-fill-v1"
TRANSIENT_FREQUENCY_PREFILL_PAGE_POLICY = "transient-frequency-v1"
SUPPORTED_PREFILL_PAGE_POLICIES = frozenset({CACHE_FILL_PREFILL_PAGE_POLICY, TRANSIENT_FREQUENCY_PREFILL_PAGE_POLICY})
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


def _npy_data_offset_and_shape(path: Path) -> tuple[int, tuple[int, ...], np.dtype]:
    """Byte offset of the array data in an ``.npy`` file, and its shape and dtype, from the
    header alone (the pages are never touched)."""
    with open(path, "rb") as fh:
        major, _ = np.lib.format.read_magic(fh)
        read_header = np.lib.format.read_array_header_1_0 if major == 1 else np.lib.format.read_array_header_2_0
        shape, fortran, dtype = read_header(fh)
        if fortran:
            raise ValueError("expert page file must be C-ordered")
        return fh.tell(), tuple(int(v) for v in shape), np.dtype(dtype)


def _validated_manifest(root: Path) -> dict[str, Any]:
    """The store manifest, after every field this reader relies on has been checked."""
    try:
        manifest = json.loads((root / "manifest.json").read_text(encoding="utf-8"))
    except (OSError, json.JSONDecodeError) as exc:
        raise ValueError(f"int8 expert store at {root} has no readable manifest.json") from exc
    expected = {"schema_version": STORE_SCHEMA, "codec": STORE_CODEC, "data_file": STORE_FILE + ".npy"}
    for key, want in expected.items():
        if manifest.get(key) != want:
            raise ValueError(f"int8 expert store {key} {manifest.get(key)!r} is not {want!r}")
    for key in ("layers", "num_experts"):
        value = manifest.get(key)
        if isinstance(value, bool) or not isinstance(value, int) or value < 1:
            raise ValueError(f"int8 expert store {key} must be a positive integer")
    return manifest


class PackedInt8ExpertStore:
    """Expert pages on disk for the HBM slot cache.

    One ``.npy`` array ``uint8 [layers * experts, page_stride]`` holds page ``layer *
    experts + expert`` in the ``ExpertPageLayout``; ``manifest.json`` names the schema,
    codec, geometry and layout.  Opening reads the manifest and the array header only; the
    pages are memory-mapped on first use.  Public surface of the reference's packed expert
    store (qwen3_moe_cuda.py:780-840): ``layout``, ``layers``, ``experts``, ``global_page``,
    ``gather``, ``view_pages``, ``release``; the file format is this build's own.
    """

    def __init__(self, store_dir: str | Path):
        self.store_dir = Path(store_dir)
        self.manifest = _validated_manifest(self.store_dir)
        self.layout = ExpertPageLayout.from_dict(self.manifest["layout"])
        self.layers = int(self.manifest["layers"])
        self.experts = int(self.manifest["num_experts"])
        self.data_path = self.store_dir / self.manifest["data_file"]
        if not self.data_path.is_file():
            raise ValueError(f"int8 expert store page file {self.data_path} is missing")
        self.data_offset, shape, dtype = _npy_data_offset_and_shape(self.data_path)
        want = (self.layers * self.experts, self.layout.page_stride)
        if shape != want or dtype != np.uint8:
            raise ValueError(f"expert page file holds {dtype} {shape}, the manifest describes uint8 {want}")
        self._mapped: np.ndarray | None = None

    @property
    def page_count(self) -> int:
        return self.layers * self.experts

    def _pages(self) -> np.ndarray:
        if self._mapped is None:
            self._mapped = np.load(self.data_path, mmap_mode="r", allow_pickle=False)
        return self._mapped

    def global_page(self, layer: int, expert: int) -> int:
        if not (0 <= layer < self.layers and 0 <= expert < self.experts):
            raise IndexError(f"expert page ({layer}, {expert}) outside {self.layers} x {self.experts}")
        return layer * self.experts + expert

    def page(self, gid: int) -> np.ndarray:
        """Page ``gid`` as a read-only view of the mapping."""
        return self._pages()[gid]

    def gather(self, layer: int, expert_ids: list[int], target: torch.Tensor) -> None:
        """Copy the pages of ``expert_ids`` (one layer) into ``target[:len(expert_ids)]``.
        Runs of consecutive page ids are copied as one slice each, so a sorted expert list
        reads the file sequentially."""
        count = len(expert_ids)
        if count == 0:
            return
        stride = self.layout.page_stride
        if (target.device.type != "cpu" or target.dtype != torch.uint8 or target.ndim != 2
                or int(target.shape[1]) != stride or int(target.shape[0]) < count):
            raise ValueError(f"expert page gather needs a host uint8 [>= {count}, {stride}] target")
        ids = [self.global_page(layer, int(e)) for e in expert_ids]
        dst = target.numpy()
        pages = self._pages()
        run = 0
        for i in range(1, count + 1):
            if i == count or ids[i] != ids[i - 1] + 1:
                dst[run:i] = pages[ids[run]:ids[i - 1] + 1]
                run = i

    def view_pages(self, raw: torch.Tensor) -> Int8ExpertLayer:
        """Expert-page views ``gate_up / gate_up_scales / down / down_scales`` over ``raw``
        ``[groups, page_stride]`` (no copies)."""
        if raw.dtype != torch.uint8 or raw.ndim != 2 or raw.shape[1] != self.layout.page_stride:
            raise ValueError("expert pages must be uint8 [groups, page_stride]")
        return Int8ExpertLayer(raw.reshape(-1), self.layout, int(raw.shape[0]))

    def release(self) -> None:
        """Drop the mapping (it is re-created on the next read)."""
        self._mapped = None


def _host_rows(rows: int, width: int, pin: bool) -> tuple[torch.Tensor, bool]:
    """``uint8 [rows, width]`` host memory, page-locked when ``pin`` and the runtime grants
    it, else pageable; returns the tensor and whether it is pinned."""
    if pin:
        try:
            return torch.empty((rows, width), dtype=torch.uint8, pin_memory=True), True
        except RuntimeError:
            pass
    return torch.empty((rows, width), dtype=torch.uint8), False


class HostPageTier:
    """Fill-once host copy of expert pages between the HBM cache and the store file.

    A pinned arena of ``host_cache_mb`` worth of page rows (pageable if pinning is refused).
    Rows are handed out in order and never reclaimed: ``warm()`` streams the store's
    leading pages into the free rows with large sequential file reads, and a page first
    met later takes the next free row while any is left; pages beyond the budget are read
    from the store on every miss.  A pinned tier row is the source of the pager's H2D
    transfer directly.  Public surface and statistics keys of the reference's host tier
    (qwen3_moe_cuda.py:878-981).
    """

    WARM_READ_BYTES = 256 << 20

    def __init__(self, store: PackedInt8ExpertStore, *, host_cache_mb: float, try_pin: bool = True):
        self.store = store
        stride = store.layout.page_stride
        budget = int(float(host_cache_mb) * 1e6) // stride
        if budget < 1:
            raise ValueError("host_cache_mb smaller than one expert page")
        self.capacity = min(store.page_count, budget)
        self.buf, self.pinned = _host_rows(self.capacity, stride, try_pin)
        self._row_of_page = np.full(store.page_count, -1, dtype=np.int64)
        self._used_rows = 0
        self.stats = {"capacity_pages": self.capacity, "pinned": self.pinned, "warmed_pages": 0,
                      "warm_seconds": 0.0, "served_pages": 0, "admitted_pages": 0, "disk_pages": 0}

    def warm(self) -> dict[str, Any]:
        """Read pages ``[used, capacity)`` of the store into the same rows with unbuffered
        sequential reads straight into the arena (no mapping: the tier is the only copy in
        this process's memory)."""
        t0 = time.perf_counter()
        stride = self.store.layout.page_stride
        first = self._used_rows
        arena = memoryview(self.buf.numpy().reshape(-1))
        end = self.capacity * stride
        pos = first * stride
        with open(self.store.data_path, "rb", buffering=0) as fh:
            fh.seek(self.store.data_offset + pos)
            while pos < end:
                got = fh.readinto(arena[pos:min(end, pos + self.WARM_READ_BYTES)])
                if not got:
                    break
                pos += got
        last = pos // stride
        self._row_of_page[first:last] = np.arange(first, last, dtype=np.int64)
        self._used_rows = last
        self.stats["warmed_pages"] = last
        self.stats["warm_seconds"] = time.perf_counter() - t0
        return dict(self.stats)

    def host_page(self, layer: int, expert: int) -> torch.Tensor | None:
        """The tier row holding a page, admitting the page into a free row when it is not
        held yet; ``None`` when it is not held and no row is free (read it from the store)."""
        gid = self.store.global_page(layer, expert)
        row = int(self._row_of_page[gid])
        if row >= 0:
            self.stats["served_pages"] += 1
            return self.buf[row]
        self.stats["disk_pages"] += 1
        if self._used_rows == self.capacity:
            return None
        row, self._used_rows = self._used_rows, self._used_rows + 1
        self.buf[row].numpy()[:] = self.store.page(gid)
        self._row_of_page[gid] = row
        self.stats["admitted_pages"] += 1
        return self.buf[row]

    def gather(self, layer: int, expert_ids: list[int], target: torch.Tensor) -> None:
        """Fill ``target[:len(expert_ids)]`` with the pages: tier rows where held (admitting
        new pages while rows are free), the store for the rest."""
        dst = target[: len(expert_ids)].numpy()
        from_store: list[tuple[int, int]] = []
        for i, expert in enumerate(expert_ids):
            row = self.host_page(layer, int(expert))
            if row is None:
                from_store.append((i, int(expert)))
            else:
                dst[i] = row.numpy()
        for i, expert in from_store:
            dst[i] = self.store.page(self.store.global_page(layer, expert))


# ---- page trace (host logic) ----------------------------------------------------------------

PAGE_TRACE_SCHEMA = "mrun-qwen3-moe-page-trace-v1"
PAGE_TRACE_HARD_MAX_EVENTS = 250_000
PAGE_TRACE_HARD_MAX_REQUESTS = 2_000_000
PAGE_TRACE_HARD_MAX_MANIFEST_BYTES = 32 * 1024 * 1024


class PageTraceLimitError(RuntimeError):
    """A page-trace cap would be exceeded; raised before the acquire changes the cache."""


Qwen3MoePageTraceLimitError = PageTraceLimitError  # the reference's name for the same error


def _canonical_json(value: Any) -> bytes:
    return json.dumps(value, sort_keys=True, separators=(",", ":")).encode("utf-8")


def _trace_cap(value: Any, name: str, hard: int) -> int:
    if isinstance(value, bool) or not isinstance(value, int) or value <= 0:
        raise ValueError(f"{name} must be a positive integer")
    if value > hard:
        raise ValueError(f"{name} cannot exceed hard maximum {hard:,}")
    return int(value)


class PageTrace:
    """Bounded record of the page requests an expert cache served, in the reference's
    ``mrun-qwen3-moe-page-trace-v1`` manifest (qwen3_moe_cuda.py:1039-1220).

    One event per acquire: its phase (``prefill`` / ``decode``), a step counted per (phase,
    layer), the layer, and the sorted unique experts with their route counts.  Nothing
    else is kept (no activations, no tokens).  The manifest is canonical JSON (sorted keys,
    no spaces) with ``trace_sha256`` = SHA-256 of the manifest without that field.  Its
    size is tracked exactly as events arrive, so the event, request and byte caps are
    checked before anything is recorded."""

    def __init__(self, *, layer_count: int, page_bytes: int, max_events: int = PAGE_TRACE_HARD_MAX_EVENTS,
                 max_requests: int = PAGE_TRACE_HARD_MAX_REQUESTS,
                 max_manifest_bytes: int = PAGE_TRACE_HARD_MAX_MANIFEST_BYTES):
        self.layer_count = int(layer_count)
        self.page_bytes = int(page_bytes)
        self.caps = {
            "events": _trace_cap(max_events, "page_trace_max_events", PAGE_TRACE_HARD_MAX_EVENTS),
            "page_requests": _trace_cap(max_requests, "page_trace_max_requests", PAGE_TRACE_HARD_MAX_REQUESTS),
            "manifest_bytes": _trace_cap(max_manifest_bytes, "page_trace_max_manifest_bytes",
                                         PAGE_TRACE_HARD_MAX_MANIFEST_BYTES),
        }
        # size of the manifest with no events and a hash in place: the fixed part
        self._base_bytes = len(_canonical_json({**self._core([]), "trace_sha256": "0" * 64}))
        if self._base_bytes > self.caps["manifest_bytes"]:
            raise ValueError("page_trace_max_manifest_bytes cannot hold the empty compact trace manifest")
        self.clear()

    def _core(self, events: list) -> dict[str, Any]:
        return {"schema": PAGE_TRACE_SCHEMA, "layer_count": self.layer_count, "page_bytes": self.page_bytes,
                "source": {}, "events": events}

    def clear(self) -> None:
        self._events: list[dict[str, Any]] = []
        self._event_bytes = 0  # sum of the events' JSON sizes
        self._requests = 0
        self._next_step: dict[tuple[str, int], int] = {}

    @property
    def manifest_bytes(self) -> int:
        # the events list adds one comma between consecutive events
        return self._base_bytes + self._event_bytes + max(0, len(self._events) - 1)

    def record(self, *, phase: str, layer: int, frequencies: Counter) -> None:
        if phase not in ("prefill", "decode"):
            raise ValueError(f"unsupported Qwen3 MoE page-trace phase {phase!r}")
        layer = int(layer)
        if not 0 <= layer < self.layer_count:
            raise ValueError(f"page-trace layer {layer} is outside {self.layer_count} layers")
        pages = [[int(e), int(frequencies[e])] for e in sorted(frequencies)]
        if not pages or any(e < 0 or c <= 0 for e, c in pages):
            raise ValueError("page trace requires unique non-negative pages with positive counts")
        event = {"phase": phase, "step": self._next_step.get((phase, layer), 0), "layer": layer, "pages": pages}
        size = len(_canonical_json(event))
        after = {"events": len(self._events) + 1, "page_requests": self._requests + len(pages),
                 "manifest_bytes": self.manifest_bytes + size + (1 if self._events else 0)}
        for cap, label in (("events", "event cap"), ("page_requests", "request cap"),
                           ("manifest_bytes", "manifest-byte cap")):
            if after[cap] > self.caps[cap]:
                raise PageTraceLimitError(f"page trace exceeded configured {label} {self.caps[cap]:,}")
        self._events.append(event)
        self._event_bytes += size
        self._requests += len(pages)
        self._next_step[(phase, layer)] = event["step"] + 1

    def export(self) -> dict[str, Any] | None:
        if not self._events:
            return None
        core = self._core([dict(e, pages=[list(p) for p in e["pages"]]) for e in self._events])
        manifest = {**core, "trace_sha256": hashlib.sha256(_canonical_json(core)).hexdigest()}
        if len(_canonical_json(manifest)) != self.manifest_bytes:
            raise RuntimeError("page trace manifest byte accounting drifted")
        return manifest

    @property
    def sha256(self) -> str | None:
        manifest = self.export()
        return None if manifest is None else manifest["trace_sha256"]

    def status(self) -> dict[str, Any]:
        return {"enabled": True, "schema": PAGE_TRACE_SCHEMA, "events": len(self._events),
                "page_requests": self._requests, "manifest_bytes": self.manifest_bytes,
                "trace_sha256": self.sha256, "caps": dict(self.caps),
                "retention": "phase/step/layer plus unique expert IDs and route counts only"}

    def drain(self) -> dict[str, Any] | None:
        manifest = self.export()
        self.clear()
        return manifest


# ---- slot policy (host logic) ---------------------------------------------------------------


@dataclass
class TransientPlan:
    """A transient prefill's page plan (``SlotPolicy.plan_transient_prefill``).

    ``slab_keys[i]`` runs from slab position ``i``; the first ``miss_count`` come from the
    host (admissions first), the rest are copies of resident pages read from
    ``resident_slots`` (same order).  ``admitted`` pairs each admitted page with its new
    cache slot; it holds the first admissions of ``to_admit`` that found a slot."""

    expert_ids: list[int]
    slab_keys: list[tuple[int, int]]
    miss_count: int
    resident_slots: list[int]
    stale: list[tuple[int, int]]
    to_admit: list[tuple[int, int]]
    preserved: int
    admitted: list[tuple[tuple[int, int], int]] = field(default_factory=list)

    def group_slots(self) -> list[int]:
        """Slab position of each routed expert, in ascending expert order."""
        pos = {key[1]: i for i, key in enumerate(self.slab_keys)}
        return [pos[e] for e in self.expert_ids]


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
    transient_prefill_acquires: int = 0
    transient_prefill_pages: int = 0
    transient_prefill_admitted_pages: int = 0
    transient_prefill_preserved_pages: int = 0
    transient_prefill_h2d_bytes: int = 0
    transient_prefill_resident_materialization_d2d_bytes: int = 0
    transient_prefill_admission_d2d_bytes: int = 0
    transient_prefill_replaced_pages: int = 0
    transient_prefill_skipped_protected_pages: int = 0
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

    def drop(self, key) -> int:
        """Take ``key`` out of the cache without counting an eviction (a page the caller
        replaces by choice); its slot becomes the next one handed out."""
        slot = self.entries.pop(key)
        self.layer_entry_counts[key[0]] -= 1
        self.free_slots.append(slot)
        if self.on_change is not None:
            self.on_change(key, -1)
        return slot

    def plan_transient_prefill(self, layer: int, frequencies: Counter) -> "TransientPlan":
        """Decide a transient prefill of ``layer`` (qwen3_moe_cuda.py:1615-1777) and apply its
        admissions to the cache state.

        Every routed page runs from the transient slab; only the layer's hottest routes
        become resident.  The layer may hold ``quota - (its decode-protected pages)`` seed
        pages: the unprotected routed pages ranked by (count descending, expert id).  Its
        unprotected pages outside that seed set are replaced (dropped without an eviction
        count); seed pages not yet resident are admitted in rank order through the normal
        slot reservation, which never evicts a decode-protected page or a page of this
        prefill (an admission that finds nothing evictable is skipped).  Slab order: pages
        to admit, the other non-resident pages, then the resident pages.  The resident
        pages' slots are read out (``resident_slots``) before any replacement, so the slab
        copies of those pages precede any reuse of their slots."""
        layer = int(layer)
        expert_ids = sorted(frequencies)
        keys = [(layer, e) for e in expert_ids]
        resident = [k for k in keys if k in self.entries]
        resident_set = set(resident)
        held_protected = sum(1 for k in self.decode_protected if k[0] == layer and k in self.entries)
        seats = max(0, self.layer_quotas[layer] - held_protected)
        ranked = sorted((k for k in keys if k not in self.decode_protected),
                        key=lambda k: (-frequencies[k[1]], k[1]))[:seats]
        seed = set(ranked)
        stale = [k for k in self.entries if k[0] == layer and k not in self.decode_protected and k not in seed]
        to_admit = [k for k in ranked if k not in self.entries]
        admit_set = set(to_admit)
        nonresident = to_admit + [k for k in keys if k not in resident_set and k not in admit_set]
        plan = TransientPlan(
            expert_ids=expert_ids, slab_keys=nonresident + resident, miss_count=len(nonresident),
            resident_slots=[self.entries[k] for k in resident], stale=stale, to_admit=to_admit,
            preserved=len(resident_set.difference(stale)),
        )
        for key in stale:
            self.drop(key)
        guard = self.decode_protected | set(keys)
        for key in to_admit:
            try:
                plan.admitted.append((key, self.reserve(key, guard)))
            except RuntimeError:
                break
        return plan

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


class PageBook:
    """Host side of the expert page cache: which slot holds which page (``SlotPolicy``),
    decode protection, the statistics and the page trace, and the decision of every
    acquire (qwen3_moe_cuda.py:1395-1777).  It does no device work, so the same decisions
    run in CPU tests against the reference's own cache.  ``ExpertPageCache`` owns one and
    moves the pages it decides on."""

    def __init__(self, *, capacity: int, layers: int, experts: int, page_bytes: int, max_active_pages: int,
                 cache_policy: str, trace: PageTrace | None = None, on_change=None):
        self.stats = PageCacheStats()
        self.policy = SlotPolicy(capacity, layers, cache_policy, self.stats, on_change=on_change)
        self.experts = int(experts)
        self.page_bytes = int(page_bytes)
        self.max_active_pages = int(max_active_pages)
        self.trace = trace

    @property
    def entries(self) -> OrderedDict:
        return self.policy.entries

    @property
    def decode_protected(self) -> set:
        return self.policy.decode_protected

    def reset(self, *, clear_pages: bool) -> None:
        """Statistics and trace start over; ``clear_pages`` also empties the cache (and the
        decode-protected set)."""
        self.stats.__init__()
        if self.trace is not None:
            self.trace.clear()
        if clear_pages:
            self.policy.reset()

    def _check_active(self, count: int) -> None:
        if count > self.max_active_pages:
            raise RuntimeError(f"active expert set {count} exceeds staging limit {self.max_active_pages}")

    def acquire(self, layer: int, routed: list[int], *, protect: bool, check_limit: bool = True):
        """A cache-fill acquire of the experts routed in ``layer``: ``(expert_ids, slots,
        misses)`` with ``slots[i]`` the slot of ``expert_ids[i]`` (ascending ids) and
        ``misses`` the ``(expert, slot)`` pages to transfer.

        Pages are touched or reserved in admission order (ascending id; under
        layer-frequency LRU ascending (route count, id), so the hottest pages end most
        recently used); the acquire's own pages are never evicted for each other.  With
        ``protect`` (decode) the pages join the decode-protected set.  The trace records
        the acquire before anything changes, so a trace cap error leaves the cache as it
        was."""
        layer = int(layer)
        frequencies = Counter(routed)
        expert_ids = sorted(frequencies)
        if check_limit:
            self._check_active(len(expert_ids))
        if self.trace is not None:
            self.trace.record(phase="decode" if protect else "prefill", layer=layer, frequencies=frequencies)
        keys = [(layer, e) for e in expert_ids]
        admission = keys
        if self.policy.policy == LAYER_FREQUENCY_CACHE_POLICY:
            admission = sorted(keys, key=lambda k: (frequencies[k[1]], k[1]))
        protected = set(keys)
        entries = self.policy.entries
        misses: list[tuple[int, int]] = []
        for key in admission:
            if key in entries:
                entries.move_to_end(key)
            else:
                misses.append((key[1], self.policy.reserve(key, protected)))
        st = self.stats
        st.page_requests += len(keys)
        st.page_misses += len(misses)
        st.page_hits += len(keys) - len(misses)
        st.host_to_device_bytes += len(misses) * self.page_bytes
        st.layer_acquires += 1
        st.active_experts_sum += len(keys)
        if protect:
            st.decode_protected_promotions += len(protected - self.policy.decode_protected)
            self.policy.decode_protected.update(keys)
        return expert_ids, [entries[k] for k in keys], misses

    def transient(self, layer: int, routed: list[int]) -> TransientPlan:
        """A transient prefill of ``layer`` (``SlotPolicy.plan_transient_prefill``), counted
        in the ``transient_prefill_*`` statistics."""
        layer = int(layer)
        frequencies = Counter(routed)
        count = len(frequencies)
        self._check_active(count)
        if self.trace is not None:
            self.trace.record(phase="prefill", layer=layer, frequencies=frequencies)
        plan = self.policy.plan_transient_prefill(layer, frequencies)
        n_res, b = count - plan.miss_count, self.page_bytes
        st = self.stats
        st.page_requests += count
        st.page_hits += n_res
        st.page_misses += plan.miss_count
        st.host_to_device_bytes += plan.miss_count * b
        st.layer_acquires += 1
        st.active_experts_sum += count
        st.transient_prefill_acquires += 1
        st.transient_prefill_pages += count
        st.transient_prefill_admitted_pages += len(plan.admitted)
        st.transient_prefill_preserved_pages += plan.preserved
        st.transient_prefill_h2d_bytes += plan.miss_count * b
        st.transient_prefill_resident_materialization_d2d_bytes += n_res * b
        st.transient_prefill_admission_d2d_bytes += len(plan.admitted) * b
        st.transient_prefill_replaced_pages += len(plan.stale)
        st.transient_prefill_skipped_protected_pages += len(plan.to_admit) - len(plan.admitted)
        return plan


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
        prefill_page_policy: str | None = None,
        page_trace: bool | None = None,
        page_trace_max_events: int = PAGE_TRACE_HARD_MAX_EVENTS,
        page_trace_max_requests: int = PAGE_TRACE_HARD_MAX_REQUESTS,
        page_trace_max_manifest_bytes: int = PAGE_TRACE_HARD_MAX_MANIFEST_BYTES,
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
        prefill = prefill_page_policy if prefill_page_policy is not None else \
            os.environ.get("MRUN_QWEN3_MOE_PREFILL_PAGE_POLICY", CACHE_FILL_PREFILL_PAGE_POLICY)
        self.prefill_page_policy = str(prefill).strip().lower()
        if self.prefill_page_policy not in SUPPORTED_PREFILL_PAGE_POLICIES:
            raise ValueError(f"unsupported expert prefill page policy {self.prefill_page_policy!r}; "
                             f"expected one of {sorted(SUPPORTED_PREFILL_PAGE_POLICIES)}")
        transient = self.prefill_page_policy == TRANSIENT_FREQUENCY_PREFILL_PAGE_POLICY
        # the transient policy's rules (qwen3_moe_cuda.py:1316-1330): admissions need a
        # per-layer quota, and speculative prefetch fills could displace decode pages
        if transient and str(policy).strip().lower() != LAYER_FREQUENCY_CACHE_POLICY:
            raise ValueError("transient-frequency-v1 prefill requires layer-frequency-lru-v1 "
                             "so every layer has a bounded admission quota")
        if transient and self.route_prefetch:
            raise ValueError("transient-frequency-v1 prefill is incompatible with route-history prefetch "
                             "because speculative pages can evict decode-protected residency")
        if page_trace is None:
            page_trace = os.environ.get("MRUN_QWEN3_MOE_PAGE_TRACE", "").strip().lower() not in \
                ("", "0", "false", "no", "off")
        self._page_trace = PageTrace(
            layer_count=store.layers, page_bytes=self.layout.page_stride, max_events=page_trace_max_events,
            max_requests=page_trace_max_requests, max_manifest_bytes=page_trace_max_manifest_bytes,
        ) if page_trace else None
        stride = self.layout.page_stride
        requested = int(float(cache_mb) * 1e6) // stride
        self.capacity = min(store.layers * store.experts, max(int(max_active_pages), requested))
        self.max_active_pages = int(max_active_pages)
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
        self.book = PageBook(capacity=self.capacity, layers=store.layers, experts=store.experts,
                             page_bytes=stride, max_active_pages=self.max_active_pages,
                             cache_policy=str(policy).strip().lower(), trace=self._page_trace,
                             on_change=self._slot_changed)
        self.policy = self.book.policy
        self.cache_policy = self.policy.policy
        # one pager arena: the policy's cache slots, then (transient prefill only) a slab of
        # max_active_pages slots that a prefill layer runs from; the pager orders every
        # transfer into either part against that slot's last readers
        self._slab_pages = self.max_active_pages if transient else 0
        self._arena = torch.empty((self.capacity + self._slab_pages, stride), dtype=torch.uint8, device=self.device)
        self.cache = self._arena[: self.capacity]
        self.slab = self._arena[self.capacity:] if transient else None
        # pinned staging for pages the host tier does not hold (read from the store file)
        self.stage = torch.empty((self.max_active_pages, stride), dtype=torch.uint8, pin_memory=True)
        self.compact = torch.empty((self.max_active_pages, stride), dtype=torch.uint8, device=self.device) \
            if self.page_binding_policy == COMPACT_PAGE_BINDING_POLICY else None
        handle = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            nat.call("qs_pager_create", nat.ptr(self._arena), stride, self.capacity + self._slab_pages,
                     TRANSFER_BYTES, ctypes.byref(handle))
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
        return self.book.stats

    @property
    def free_slots(self) -> list[int]:
        self._drain_deferred()
        return self.policy.free_slots

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
        n = self._arena.numel() + (self.compact.numel() if self.compact is not None else 0)
        return int(n)

    @property
    def layer_entry_counts(self) -> list[int]:
        self._drain_deferred()
        return self.policy.layer_entry_counts

    @property
    def page_trace_sha256(self) -> str | None:
        return None if self._page_trace is None else self._page_trace.sha256

    def page_trace_status(self) -> dict[str, Any]:
        return {"enabled": False} if self._page_trace is None else self._page_trace.status()

    def export_page_trace(self) -> dict[str, Any] | None:
        return None if self._page_trace is None else self._page_trace.export()

    def drain_page_trace(self) -> dict[str, Any] | None:
        return None if self._page_trace is None else self._page_trace.drain()

    def reset(self, *, clear_pages: bool) -> None:
        self.synchronize()
        self._drain_deferred()  # the deferred touches belong to the statistics being reset
        self.prefetch_stats = {"prefetched_pages": 0, "prefetch_rounds": 0, "wasted_prefetches": 0}
        self._prev_routes.clear()
        self._prefetched.clear()
        self.book.reset(clear_pages=clear_pages)

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
        Route prefetch and the page trace read the routes on the host, so they turn this
        binding off, and so does the compact-copy binding policy."""
        if (self.route_prefetch or self._page_trace is not None
                or self.page_binding_policy != SLOT_INDIRECT_PAGE_BINDING_POLICY
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
                    self.book.stats.host_to_device_bytes += len(fills) * self.layout.page_stride
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

    def _touch(self, layer: int, routed: list[int], protect: bool) -> None:
        """Bookkeeping of a device-table acquire (every page of the layer resident: no fills)."""
        routed = [e for e in routed if 0 <= e < self.store.experts]
        self._prefetched.difference_update((int(layer), e) for e in routed)
        _, _, misses = self.book.acquire(layer, routed, protect=protect, check_limit=False)
        assert not misses, "a device-table layer lost a page before its deferred bookkeeping"

    def _submit(self, slot: int, host_ptr: int) -> None:
        nat.call("qs_pager_submit", self._pager, slot, host_ptr, self.layout.page_stride, 0)
        nat.call("qs_pager_seal", self._pager, slot)

    def _submit_runs(self, pages: list[tuple[int, int]]) -> None:
        """H2D of ``(slot, host address)`` pages: pages whose slots and host rows both follow
        each other move as one run (``qs_pager_submit_run``, at most ``TRANSFER_BYTES``
        each), so a layer change's ~125 consecutive pages are a few large transfers."""
        stride = self.layout.page_stride
        cap = max(1, TRANSFER_BYTES // stride)
        pages = sorted(pages)
        i = 0
        while i < len(pages):
            j = i + 1
            while (j < len(pages) and j - i < cap and pages[j][0] == pages[j - 1][0] + 1
                   and pages[j][1] == pages[j - 1][1] + stride):
                j += 1
            if j - i == 1:
                self._submit(*pages[i])
            else:
                nat.call("qs_pager_submit_run", self._pager, pages[i][0], j - i, pages[i][1])
            i = j

    def _acquire_slots(self, slots: list[int]) -> None:
        """The compute stream waits for the pending transfers into ``slots``."""
        if slots:
            nat.call("qs_pager_acquire_many", self._pager, (ctypes.c_int * len(slots))(*slots), len(slots),
                     nat.stream_of(self.device))

    def _fill(self, layer: int, misses: list[tuple[int, int]]) -> None:
        """One H2D transfer per missing page into its pager slot, on the pager's copy
        stream: straight from the page's pinned tier row, else through the pinned staging
        buffer (pages only the store holds are read by one gather, in the given order)."""
        staged: list[tuple[int, int, torch.Tensor | None]] = []  # (expert, slot, pageable tier row)
        direct: list[tuple[int, int]] = []  # (slot, pinned tier row address)
        for expert, slot in misses:
            row = self.host_tier.host_page(layer, expert) if self.host_tier is not None else None
            if row is not None and self.host_tier.pinned:
                direct.append((slot, row.data_ptr()))
            else:
                staged.append((expert, slot, row))
        self._submit_runs(direct)
        if staged:
            if self._stage_in_flight:  # the previous staging copies must have landed
                self.synchronize()
            staged.sort(key=lambda item: item[2] is not None)  # store pages first (stable)
            n_store = sum(1 for item in staged if item[2] is None)
            if n_store:
                self.store.gather(layer, [expert for expert, _, _ in staged[:n_store]], self.stage)
            for i in range(n_store, len(staged)):
                self.stage[i].numpy()[:] = staged[i][2].numpy()
            self._submit_runs([(slot, self.stage[i].data_ptr()) for i, (_, slot, _) in enumerate(staged)])
            self._stage_in_flight = True

    def acquire_transient_prefill(self, layer: int, top_indices: torch.Tensor):
        """``(selected_experts, page views of the transient slab, group_slots)`` for a
        prefill layer under ``transient-frequency-v1`` (qwen3_moe_cuda.py:1615-1777).

        The layer runs from the slab, so a long prompt's scan over every expert cannot flush
        the decode working set; only its hottest routes are admitted into the cache, within
        the layer's quota and never over a decode-protected page
        (``SlotPolicy.plan_transient_prefill`` decides).  Device work, in stream order:
        resident pages are copied from their cache slots into the slab (before any of those
        slots is reused), the other pages travel once from the host into their slab slots
        (pager transfers), and the admitted pages are copied from the slab into their new
        cache slots.  ``group_slots[g]`` is the slab position of the g-th routed expert in
        ascending id order.  The slab's and the touched cache slots' free events are
        recorded by the next ``release()`` (after this layer's kernels), which every later
        transfer into them waits for."""
        if self.prefill_page_policy != TRANSIENT_FREQUENCY_PREFILL_PAGE_POLICY:
            raise RuntimeError("transient prefill acquisition requires transient-frequency-v1")
        if self.cache_policy != LAYER_FREQUENCY_CACHE_POLICY:
            raise RuntimeError("transient-frequency-v1 prefill requires layer-frequency-lru-v1")
        self.release()
        self._drain_deferred()
        layer = int(layer)
        plan = self.book.transient(layer, top_indices.detach().reshape(-1).cpu().tolist())
        count = len(plan.expert_ids)
        slab = self.capacity  # pager slot of slab position 0
        n_res = count - plan.miss_count
        touched: list[int] = []
        if n_res:
            dst = [slab + plan.miss_count + i for i in range(n_res)]
            self._acquire_slots(plan.resident_slots + dst)
            for src_slot, dst_slot in zip(plan.resident_slots, dst):
                self._arena[dst_slot].copy_(self._arena[src_slot], non_blocking=True)
            touched += plan.resident_slots + dst
        if plan.miss_count:
            misses = [(key[1], slab + i) for i, key in enumerate(plan.slab_keys[:plan.miss_count])]
            self._fill(layer, misses)
            self._acquire_slots([slot for _, slot in misses])
            touched += [slot for _, slot in misses]
        if plan.admitted:
            adm = [slot for _, slot in plan.admitted]
            self._acquire_slots(adm)
            for i, slot in enumerate(adm):
                self._arena[slot].copy_(self._arena[slab + i], non_blocking=True)
            touched += adm
        self._pending_release = list(dict.fromkeys(touched))
        selected = torch.tensor(plan.expert_ids, dtype=torch.long, device=self.device)
        group_slots = torch.tensor(plan.group_slots(), dtype=torch.long, device=self.device)
        return selected, self.store.view_pages(self.slab[:count]), group_slots

    def _acquire_resident(self, layer: int, top_indices: torch.Tensor, *, protect: bool):
        self.release()  # the previous acquire's kernels are queued: its slots may be refilled after them
        self._drain_deferred()  # earlier device-table layers' LRU touches precede any eviction here
        layer = int(layer)
        routed = top_indices.detach().reshape(-1).cpu().tolist()
        expert_ids, slot_list, misses = self.book.acquire(layer, routed, protect=protect)
        keys = [(layer, e) for e in expert_ids]
        self._prefetched.difference_update(keys)
        if misses:
            self._fill(layer, misses)
        self._acquire_slots(slot_list)
        self._pending_release = list(slot_list)
        if self.route_prefetch:
            self._prefetch_next_layer(layer, set(keys))
            self._prev_routes[layer] = expert_ids
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
        self.book.stats.host_to_device_bytes += len(fills) * self.layout.page_stride
        self.prefetch_stats["prefetched_pages"] += len(fills)
        self.prefetch_stats["prefetch_rounds"] += 1
