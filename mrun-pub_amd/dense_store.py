"""Device-resident int8 QStore with fused HIP projections (the ``DenseQStore`` surface).

Mirrors ``DenseQStore`` (src/mrun/engine/kernels/dense_qstore_cuda.py:1857-2362) and the
store-level calls of ``QStore`` (src/mrun/engine/kernels/qstore.py:1008-1185):

* ``compact_page(name)``       -- HBM page ``(codes, scales)``; byte-budgeted LRU, plus
  ``prepare_fully_resident()`` which pins every qrow block in one HBM arena;
* ``matmul(name, x)`` / ``matmul_row_stable`` / ``fused_swiglu`` / ``weight`` / ``fp32`` /
  ``row_blocks`` / ``has``;
* ``stats`` -- projection / page counters in the spirit of ``DenseQStoreStats``
  (dense_qstore_cuda.py:141-170).

The arena is one ``torch.uint8`` allocation holding every block's codes then scales at
256-byte aligned offsets, so a fully resident 28-layer stack is a single HBM region.
"""

from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np
import torch

from . import qrow as _qrow
from .qrow import CompactQRowPage
from .store import QStoreReader

_DTYPES = {None: torch.float32, "fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


@dataclass
class DenseQStoreStats:
    projection_calls: int = 0
    native_projection_calls: int = 0
    paired_swiglu_calls: int = 0
    page_loads: int = 0
    cache_hits: int = 0
    compact_h2d_bytes: int = 0
    compact_logical_bytes: int = 0
    expanded_compute_bytes_avoided: int = 0
    extra: dict = field(default_factory=dict)


def _align(n: int, a: int = 256) -> int:
    return (n + a - 1) // a * a


class DenseQStore:
    """int8 QStore whose qrow blocks live in HBM and run through the HIP kernels."""

    def __init__(
        self,
        store: QStoreReader | str | Path,
        *,
        device: str | torch.device = "cuda",
        compute_dtype: str | None = "bf16",
        compact_cache_mb: float = 0.0,
    ) -> None:
        self.reader = store if isinstance(store, QStoreReader) else QStoreReader(store)
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("DenseQStore requires a HIP (cuda) device")
        if compute_dtype not in _DTYPES:
            raise ValueError("compute_dtype must be fp32, bf16 or fp16")
        self.compute_dtype = _DTYPES[compute_dtype]
        self.compact_cache_budget = int(float(compact_cache_mb) * 1e6)
        self.compact_cache: OrderedDict[str, CompactQRowPage] = OrderedDict()
        self.compact_cache_bytes = 0
        self._resident: dict[str, CompactQRowPage] = {}
        self.arena: torch.Tensor | None = None
        self.stats = DenseQStoreStats()

    # ---- store surface --------------------------------------------------------------
    def _physical(self, name: str) -> str:
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
                return key
            key = str(blk["alias"])

    def has(self, name: str) -> bool:
        return self.reader.has(name)

    def fp32(self, name: str) -> torch.Tensor:
        return torch.from_numpy(self.reader.fp32(name)).to(self.device)

    def _load_page(self, key: str) -> CompactQRowPage:
        codes, scales = self.reader.qrow(key)
        c = torch.from_numpy(np.array(codes, copy=True)).to(self.device)
        s = torch.from_numpy(np.array(scales, copy=True)).to(self.device)
        page = CompactQRowPage(key, 0, int(codes.shape[0]), int(codes.shape[1]), c, s)
        self.stats.page_loads += 1
        self.stats.compact_h2d_bytes += page.compact_bytes
        return page

    def prepare_fully_resident(self) -> int:
        """Copy every qrow block into one HBM arena; returns the arena size in bytes."""
        names = self.reader.qrow_names()
        layout = []
        off = 0
        for name in names:
            blk = self.reader.blocks[name]
            out, inn = (int(v) for v in blk["shape"])
            c_off = off
            off = _align(off + out * inn)
            s_off = off
            off = _align(off + out * 4)
            layout.append((name, out, inn, c_off, s_off))
        arena = torch.empty(off, dtype=torch.uint8, device=self.device)
        for name, out, inn, c_off, s_off in layout:
            codes, scales = self.reader.qrow(name)
            arena[c_off : c_off + out * inn].copy_(
                torch.from_numpy(np.array(codes, copy=True).view(np.uint8).reshape(-1))
            )
            arena[s_off : s_off + out * 4].copy_(
                torch.from_numpy(np.array(scales, copy=True).view(np.uint8).reshape(-1))
            )
            c = arena[c_off : c_off + out * inn].view(torch.int8).view(out, inn)
            s = arena[s_off : s_off + out * 4].view(torch.float32)
            self._resident[name] = CompactQRowPage(name, 0, out, inn, c, s)
        self.arena = arena
        self.stats.compact_h2d_bytes += off
        return off

    def compact_page(self, name: str) -> CompactQRowPage:
        key = self._physical(name)
        page = self._resident.get(key)
        if page is not None:
            self.stats.cache_hits += 1
            return page
        page = self.compact_cache.get(key)
        if page is not None:
            self.compact_cache.move_to_end(key)
            self.stats.cache_hits += 1
            return page
        if self.reader.blocks[key].get("kind") != "qrow":
            raise ValueError(f"{name} is not a qrow block")
        page = self._load_page(key)
        if 0 < page.compact_bytes <= self.compact_cache_budget:
            self.compact_cache[key] = page
            self.compact_cache_bytes += page.compact_bytes
            while self.compact_cache_bytes > self.compact_cache_budget:
                _, ev = self.compact_cache.popitem(last=False)
                self.compact_cache_bytes -= ev.compact_bytes
        return page

    def block_kind(self, name: str) -> str | None:
        """``"qrow"`` / ``"fp32"`` of a block after alias resolution."""
        return self.reader.block_kind(name)

    def embed_rows(self, name: str, ids) -> torch.Tensor:
        """fp32 rows ``ids`` of a qrow block, shape ``[*ids.shape, in]``, on the store's device
        (qstore.py:1099-1128).  Reads only those rows from the host file unless the block is
        already on the device."""
        key = self._physical(name)
        page = self._resident.get(key) or self.compact_cache.get(key)
        if page is not None:
            return _qrow.qrow_embed_rows(page.codes, page.scales, ids)
        if self.reader.blocks[key].get("kind") != "qrow":
            raise ValueError(f"{name} is not a qrow block")
        out = int(self.reader.blocks[key]["shape"][0])
        flat, shape = _qrow.normalize_row_ids(ids, out)
        uniq, inverse = np.unique(flat.reshape(-1), return_inverse=True)
        codes, scales = self.reader.qrow_rows(key, uniq)
        c = torch.from_numpy(np.ascontiguousarray(codes)).to(self.device)
        s = torch.from_numpy(np.ascontiguousarray(scales)).to(self.device)
        return _qrow.qrow_embed_rows(c, s, inverse.reshape(shape))

    def weight(self, name: str) -> torch.Tensor:
        """Materialized ``[out, in]`` weight in the compute dtype (qstore.py:1026-1080)."""
        page = self.compact_page(name)
        return _qrow.qrow_dequant(page.codes, page.scales, self.compute_dtype)

    def _count(self, page: CompactQRowPage, n: int = 1) -> None:
        self.stats.projection_calls += n
        self.stats.native_projection_calls += n
        self.stats.compact_logical_bytes += page.compact_bytes * n
        self.stats.expanded_compute_bytes_avoided += page.expanded_compute_bytes(self.compute_dtype) * n

    def matmul(self, name: str, x: torch.Tensor) -> torch.Tensor:
        """``x @ W.T``; fp32 activations follow the store's compute dtype (qstore.py:1082-1092)."""
        page = self.compact_page(name)
        if x.dtype != self.compute_dtype:
            x = x.to(self.compute_dtype)
        y, _tag = _qrow.fused_qrow_matmul(page, x)
        self._count(page)
        return y

    def matmul_row_stable(self, name: str, x: torch.Tensor) -> torch.Tensor:
        """Batch-invariant projection (qstore.py:1094-1097)."""
        if x.ndim < 2 or int(x.shape[0]) <= 0:
            raise ValueError("row-stable matmul input must have a leading request axis")
        page = self.compact_page(name)
        if x.dtype != self.compute_dtype:
            x = x.to(self.compute_dtype)
        y = _qrow.qrow_matmul(page.codes, page.scales, x, row_stable=True)
        self._count(page)
        return y

    def matmul_multi(self, names: list[str], x: torch.Tensor) -> list[torch.Tensor]:
        """Projections sharing one activation (q/k/v) in a single launch."""
        pages = [self.compact_page(n) for n in names]
        if x.dtype != self.compute_dtype:
            x = x.to(self.compute_dtype)
        outs = _qrow.qrow_matmul_multi([(p.codes, p.scales) for p in pages], x)
        for p in pages:
            self._count(p)
        return outs

    def fused_swiglu(self, gate_name: str, up_name: str, x: torch.Tensor) -> tuple[torch.Tensor, str]:
        """Paired gate/up W8A16 + BF16 SwiGLU (dense_qstore_cuda.py:2346-2356)."""
        g, u = self.compact_page(gate_name), self.compact_page(up_name)
        y, tag = _qrow.fused_qrow_swiglu(g, u, x)
        self._count(g)
        self._count(u)
        self.stats.paired_swiglu_calls += 1
        return y, tag

    def row_blocks(self, name: str, bs: int = 8192):
        """Yield ``(start, end, W)`` row chunks of the materialized weight (qstore.py:1130-1185)."""
        page = self.compact_page(name)
        for start in range(0, page.out_features, bs):
            end = min(start + bs, page.out_features)
            yield start, end, _qrow.qrow_dequant(
                page.codes[start:end], page.scales[start:end], self.compute_dtype
            )

    def close(self) -> None:
        self.compact_cache.clear()
        self._resident.clear()
        self.arena = None
