"""Packed int3 / int2 QStore linears on gfx950 (device GEMV + dequant).

Mirrors the reference low-bit readers (src/mrun/engine/kernels/qstore.py:1283-1544:
``QStoreInt3`` / ``QStoreInt2`` with ``weight`` / ``matmul`` / ``matmul_row_stable`` /
``embed_rows`` / ``row_blocks``), which in the reference run on the CPU only.  Here the
packed codes and scales live in HBM and every product runs through ``csrc/qs_lowbit.hip``.
Both layouts are served: the reference's symmetric one (fixed offset, fp32 scales, G=128)
and the asymmetric G=64 fp16 scale + zero-point variant.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from . import _native as nat

IMPL_LOWBIT = "hip-gfx950-lowbit-mfma-v1"
OFFSET = {3: 4.0, 2: 1.0, 4: 8.0}


@dataclass(frozen=True)
class LowbitPage:
    """One packed block in HBM: ``packed [N, row_bytes] uint8``, ``scales [N, ng]``."""

    name: str
    bits: int
    group_size: int
    in_features: int
    packed: torch.Tensor
    scales: torch.Tensor
    zeros: torch.Tensor | None = None
    offset: float | None = None

    @property
    def out_features(self) -> int:
        return int(self.packed.shape[0])

    @property
    def row_bytes(self) -> int:
        return int(self.packed.shape[1])

    @property
    def compact_bytes(self) -> int:
        z = 0 if self.zeros is None else self.zeros.numel() * self.zeros.element_size()
        return self.packed.numel() + self.scales.numel() * self.scales.element_size() + z

    def _offset(self) -> float:
        return float(OFFSET[self.bits] if self.offset is None else self.offset)


def _check(page: LowbitPage) -> None:
    if page.packed.dtype != torch.uint8 or page.packed.ndim != 2 or not page.packed.is_contiguous():
        raise ValueError("packed codes must be contiguous uint8 [out, row_bytes]")
    if page.row_bytes < (page.in_features * page.bits + 7) // 8:
        raise ValueError("row_bytes too small for in_features")
    ng = (page.in_features + page.group_size - 1) // page.group_size
    if page.scales.shape != (page.out_features, ng) or page.scales.dtype not in (torch.float32, torch.float16):
        raise ValueError("scales must be float32/float16 [out, n_groups]")
    if page.zeros is not None and (page.zeros.shape != page.scales.shape or page.zeros.dtype not in (torch.float32, torch.float16)):
        raise ValueError("zeros must match scales in shape and be float32/float16")


@torch.inference_mode()
def lowbit_dequant(page: LowbitPage) -> torch.Tensor:
    """fp32 ``[out, in]`` weight ``(float(code) - zero) * scale`` (qstore.py:441-456)."""
    _check(page)
    device = nat.require_device(page.packed, page.scales, page.zeros)
    out = torch.empty((page.out_features, page.in_features), dtype=torch.float32, device=device)
    nat.call(
        "qs_lowbit_dequant", nat.ptr(page.packed), page.row_bytes, nat.ptr(page.scales),
        nat.dtype_code(page.scales.dtype), nat.ptr(page.zeros),
        nat.dtype_code(page.zeros.dtype) if page.zeros is not None else nat.QS_F32, page._offset(),
        page.bits, page.group_size, nat.ptr(out), page.out_features, page.in_features, nat.stream_of(device),
    )
    return out


@torch.inference_mode()
def lowbit_matmul(page: LowbitPage, x: torch.Tensor, *, row_stable: bool = False) -> torch.Tensor:
    """``x[..., in] @ W.T`` in fp32 (``QStoreInt3.matmul`` contract), fp32 ``[..., out]``.

    ``row_stable=True`` runs every activation row as its own M = 1 product, so row b of a
    batch equals the single-row result bit for bit (``matmul_row_stable``,
    qstore.py:1343-1380); otherwise rows share launches and the kernel choice depends on M.
    """
    _check(page)
    K = page.in_features
    if int(x.shape[-1]) != K:
        raise ValueError("activation width does not match the packed block")
    device = nat.require_device(page.packed, page.scales, page.zeros, x)
    x2 = x.reshape(-1, K)
    if x2.dtype not in (torch.bfloat16, torch.float32):
        x2 = x2.to(torch.float32)
    x2 = x2.contiguous()
    M, N = int(x2.shape[0]), page.out_features
    y = torch.empty((M, N), dtype=torch.float32, device=device)
    _gemv_into(page, x2, y, N, row_stable=row_stable)
    return y.reshape(*x.shape[:-1], N)


def _gemv_into(page: LowbitPage, x2: torch.Tensor, y: torch.Tensor, ldy: int, *, row_stable: bool) -> None:
    """``y[m, :N] = x2[m] @ W.T`` for every row of ``x2`` ([M, K], bf16/fp32, contiguous),
    into ``y`` with leading dimension ``ldy`` (fp32, on the device)."""
    M, K, N = int(x2.shape[0]), page.in_features, page.out_features
    if not M:
        return
    device = x2.device
    xdt = nat.dtype_code(x2.dtype)
    chunk = 1 if row_stable else M
    wsb = int(nat.load().qs_lowbit_workspace_bytes(xdt, chunk, N, K, page.group_size))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=device)
    for m0 in range(0, M, chunk):
        mm = min(chunk, M - m0)
        nat.call(
            "qs_lowbit_gemv", nat.ptr(x2[m0:]), xdt, K, nat.ptr(page.packed), page.row_bytes, nat.ptr(page.scales),
            nat.dtype_code(page.scales.dtype), nat.ptr(page.zeros),
            nat.dtype_code(page.zeros.dtype) if page.zeros is not None else nat.QS_F32, page._offset(),
            page.bits, page.group_size, y.data_ptr() + 4 * m0 * ldy, ldy, mm, N, K, nat.ptr(ws), wsb,
            nat.stream_of(device),
        )


_LOWBIT_FILES = {3: "weights.i3", 2: "weights.i2"}


def _regular_file_stats(d: Path, names) -> tuple:
    """(name, device, inode, mode, size, mtime, ctime) of each runtime file; a missing file,
    a symlink or another non-regular file is refused (qstore.py:859-880)."""
    import stat as _stat

    out = []
    for name in names:
        try:
            st = (d / name).lstat()
        except OSError as exc:
            raise RuntimeError(f"QStore runtime file is unavailable: {name}") from exc
        if not _stat.S_ISREG(st.st_mode):
            kind = "symlink" if _stat.S_ISLNK(st.st_mode) else "non-regular file"
            raise RuntimeError(f"QStore runtime file must be regular, not a {kind}: {name}")
        out.append((name, st.st_dev, st.st_ino, st.st_mode, st.st_size, st.st_mtime_ns, st.st_ctime_ns))
    return tuple(out)


class _ChunkStage:
    """Double-buffered pinned host + device chunks of one row geometry for streamed blocks."""

    def __init__(self, rows: int, row_bytes: int, n_groups: int, device: torch.device):
        self.rows, self.row_bytes, self.n_groups = rows, row_bytes, n_groups
        self.host = [(torch.empty((rows, row_bytes), dtype=torch.uint8, pin_memory=True),
                      torch.empty((rows, n_groups), dtype=torch.float32, pin_memory=True)) for _ in range(2)]
        self.dev = [(torch.empty((rows, row_bytes), dtype=torch.uint8, device=device),
                     torch.empty((rows, n_groups), dtype=torch.float32, device=device)) for _ in range(2)]
        self.copied: list[torch.cuda.Event | None] = [None, None]

    def nbytes(self) -> int:
        return 2 * self.rows * (self.row_bytes + 4 * self.n_groups)


class DeviceLowbitQStore:
    """``QStoreInt3`` / ``QStoreInt2`` on the device (qstore.py:1283-1544).

    Reads a reference-format low-bit store directory: ``manifest.json`` (blocks of kind
    ``qrow3`` / ``qrow2`` with ``shape``, ``w_off``, ``row_bytes``, ``s_off``, ``n_groups``,
    ``group_size``; ``fp32`` blocks with ``e_off``; aliases), ``weights.i3`` / ``weights.i2``,
    ``scales.f32`` and ``extras.f32``.

    Opening follows the reference's rules for these stores (qstore.py:326-346, 774-797,
    859-880, 1286-1301): the manifest is a JSON object that does not claim the int8 v3
    schema, ``dtype`` / ``group_size`` / ``config`` are present, and the three runtime files
    are regular files that do not change while the store opens.  Beyond the reference,
    every block's geometry (``row_bytes`` = ceil(in * bits / 8), ``n_groups`` = ceil(in / G))
    and byte range are checked against the files, so a corrupt store fails at open
    (``RuntimeError``) rather than in a kernel.

    Device residency: ``cache_mb=None`` keeps every packed block in HBM after its first use.
    With a budget, blocks are admitted while they fit and never evicted (the reference's
    default resident policy, qstore.py:946-1006); a block outside the budget streams
    through double-buffered pinned and device chunks of ``matmul_chunk_rows`` rows (the
    manifest's value, 1024 by default, qstore_int3.py:27) for every call.
    """

    _KIND_BITS = {"qrow3": 3, "qrow2": 2}

    def __init__(self, directory: str | Path, *, device: str | torch.device = "cuda", dtype: str | None = None,
                 cache_mb: float | None = None):
        from .store import QSTORE_SCHEMA

        d = Path(directory)
        man = json.loads((d / "manifest.json").read_text(encoding="utf-8"))
        if not isinstance(man, dict):
            raise RuntimeError("QStore manifest must be a JSON object")
        declared = man.get("dtype")
        if declared not in ("int3", "int2") or (dtype is not None and declared != dtype):
            raise RuntimeError(f"low-bit QStore must declare dtype {dtype or 'int3/int2'}, got {declared!r}")
        if man.get("schema_version") == QSTORE_SCHEMA:
            raise RuntimeError(f"unsupported semantic QStore dtype {declared!r}")
        self.man = man
        self.bits = 3 if declared == "int3" else 2
        self.blocks = man["blocks"]
        self.cfg = man["config"]
        self.G = int(man["group_size"])
        self.matmul_chunk_rows = max(1, int(man.get("matmul_chunk_rows", 1024)))
        self.directory = d
        names = ("manifest.json", _LOWBIT_FILES[self.bits], "scales.f32", "extras.f32")
        opened = _regular_file_stats(d, names)
        self.w = np.memmap(d / names[1], dtype=np.uint8, mode="r")
        self.s = np.memmap(d / "scales.f32", dtype=np.float32, mode="r")
        self.e = np.memmap(d / "extras.f32", dtype=np.float32, mode="r")
        self._check_blocks()
        if _regular_file_stats(d, names) != opened:
            self.close()
            raise RuntimeError("QStore files changed while the store was being opened")
        self.device = torch.device(device)
        self.cache_budget = None if cache_mb is None else int(float(cache_mb) * 1e6)
        self.cache_bytes = 0
        self._pages: dict[str, LowbitPage] = {}
        self._streamed: set[str] = set()
        self._stages: dict[tuple[int, int], _ChunkStage] = {}
        self.stats = {"resident_blocks": 0, "streamed_calls": 0, "streamed_chunks": 0, "h2d_bytes": 0}

    # -- validation --------------------------------------------------------------------
    def _geometry(self, key: str, b: dict) -> tuple[int, int, int, int, int]:
        """``(out, in, row_bytes, n_groups, G)`` of a packed block, checked."""
        if b.get("kind") not in self._KIND_BITS:
            raise ValueError(f"{key} is not a packed low-bit block")
        if self._KIND_BITS[b["kind"]] != self.bits:
            raise RuntimeError(f"QStore block {key!r} of kind {b['kind']} in a {self.bits}-bit store")
        out, inn = (int(v) for v in b["shape"])
        rb, ng = int(b["row_bytes"]), int(b["n_groups"])
        G = int(b.get("group_size", self.G))
        if out < 1 or inn < 1 or G < 1 or rb != (inn * self.bits + 7) // 8 or ng != (inn + G - 1) // G:
            raise RuntimeError(f"QStore block {key!r} geometry is inconsistent")
        return out, inn, rb, ng, G

    def _check_blocks(self) -> None:
        for key, b in self.blocks.items():
            if not isinstance(b, dict):
                raise RuntimeError(f"QStore block {key!r} must be an object")
            if "alias" in b:
                self._resolve(key)  # the chain ends in a block
                continue
            kind = b.get("kind")
            if kind == "fp32":
                n = int(np.prod(b["shape"]))
                if int(b["e_off"]) % 4 or int(b["e_off"]) // 4 + n > self.e.size:
                    raise RuntimeError(f"QStore block {key!r} exceeds extras.f32")
                continue
            out, inn, rb, ng, G = self._geometry(key, b)
            if int(b["w_off"]) < 0 or int(b["w_off"]) + out * rb > self.w.size:
                raise RuntimeError(f"QStore block {key!r} exceeds {_LOWBIT_FILES[self.bits]}")
            if int(b["s_off"]) % 4 or int(b["s_off"]) < 0 or int(b["s_off"]) // 4 + out * ng > self.s.size:
                raise RuntimeError(f"QStore block {key!r} exceeds scales.f32")

    def _resolve(self, name: str) -> tuple[str, dict]:
        key, seen = str(name), set()
        while True:
            if key in seen:
                raise RuntimeError(f"cyclic QStore alias at {name!r}")
            seen.add(key)
            if key not in self.blocks:
                raise KeyError(f"QStore has no block {key!r}")
            b = self.blocks[key]
            if "alias" not in b:
                return key, b
            key = b["alias"]

    # -- host views --------------------------------------------------------------------
    def _host_rows(self, b: dict, rb: int, ng: int, start: int, end: int) -> tuple[np.ndarray, np.ndarray]:
        w0, s0 = int(b["w_off"]), int(b["s_off"]) // 4
        packed = np.asarray(self.w[w0 + start * rb:w0 + end * rb], dtype=np.uint8).reshape(end - start, rb)
        scales = np.asarray(self.s[s0 + start * ng:s0 + end * ng], dtype=np.float32).reshape(end - start, ng)
        return packed, scales

    # -- device pages --------------------------------------------------------------------
    def page(self, name: str) -> LowbitPage | None:
        """The block's HBM-resident page, uploading it while the budget allows; ``None``
        when the block streams instead."""
        key, b = self._resolve(name)
        if key in self._pages:
            return self._pages[key]
        out, inn, rb, ng, G = self._geometry(key, b)
        size = out * (rb + 4 * ng)
        if key in self._streamed or (self.cache_budget is not None and size > self.cache_budget - self.cache_bytes):
            self._streamed.add(key)
            return None
        packed, scales = self._host_rows(b, rb, ng, 0, out)
        pg = LowbitPage(key, self.bits, G, inn, torch.from_numpy(np.array(packed)).to(self.device),
                        torch.from_numpy(np.array(scales)).to(self.device))
        self._pages[key] = pg
        self.cache_bytes += size
        self.stats["resident_blocks"] += 1
        self.stats["h2d_bytes"] += size
        return pg

    def _chunks(self, key: str, b: dict):
        """``(start, end, LowbitPage)`` over a streamed block, ``matmul_chunk_rows`` rows at a
        time: each chunk is copied host -> pinned -> device on the current stream, through
        two alternating buffers (a pinned buffer is refilled only after its previous copy
        has completed; a device buffer only after the kernels queued on it, by stream
        order)."""
        out, inn, rb, ng, G = self._geometry(key, b)
        rows = min(self.matmul_chunk_rows, out)
        stage = self._stages.get((rb, ng))
        if stage is None or stage.rows < rows:
            stage = self._stages[(rb, ng)] = _ChunkStage(rows, rb, ng, self.device)
        self.stats["streamed_calls"] += 1
        for i, start in enumerate(range(0, out, rows)):
            end = min(start + rows, out)
            n, j = end - start, i % 2
            if stage.copied[j] is not None:
                stage.copied[j].synchronize()
            (hp, hs), (dp, ds) = stage.host[j], stage.dev[j]
            packed, scales = self._host_rows(b, rb, ng, start, end)
            np.copyto(hp[:n].numpy(), packed)
            np.copyto(hs[:n].numpy(), scales)
            dp[:n].copy_(hp[:n], non_blocking=True)
            ds[:n].copy_(hs[:n], non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
            stage.copied[j] = ev
            self.stats["streamed_chunks"] += 1
            self.stats["h2d_bytes"] += n * (rb + 4 * ng)
            yield start, end, LowbitPage(key, self.bits, G, inn, dp[:n], ds[:n])

    # -- store surface ---------------------------------------------------------------------
    def has(self, name: str) -> bool:
        return str(name) in self.blocks

    def block_kind(self, name: str) -> str | None:
        return self._resolve(name)[1].get("kind")

    def fp32(self, name: str) -> torch.Tensor:
        """An ``fp32`` block of ``extras.f32`` (norms, biases) on the store's device
        (qstore.py:1008-1024)."""
        key, b = self._resolve(name)
        if b.get("kind") != "fp32":
            raise ValueError(f"{name} is not an fp32 block")
        n = int(np.prod(b["shape"]))
        off = int(b["e_off"]) // 4
        vals = np.array(self.e[off:off + n], dtype=np.float32, copy=True).reshape(b["shape"])
        return torch.from_numpy(vals).to(self.device)

    def weight(self, name: str) -> torch.Tensor:
        key, b = self._resolve(name)
        pg = self.page(key)
        if pg is not None:
            return lowbit_dequant(pg)
        out, inn = (int(v) for v in b["shape"])
        W = torch.empty((out, inn), dtype=torch.float32, device=self.device)
        for start, end, chunk in self._chunks(key, b):
            W[start:end] = lowbit_dequant(chunk)
        return W

    def embed_rows(self, name: str, ids) -> torch.Tensor:
        """fp32 rows ``ids`` of a packed block, ``[*ids.shape, in]`` (qstore.py:1382-1395,
        1513-1526).  Only the selected rows are read from the host file."""
        from .qrow import normalize_row_ids

        key, b = self._resolve(name)
        out, inn, rb, ng, G = self._geometry(key, b)
        flat, shape = normalize_row_ids(ids, out)
        flat = flat.reshape(-1)
        if flat.size == 0:
            return torch.empty((*shape, inn), dtype=torch.float32, device=self.device)
        packed, scales = self._host_rows(b, rb, ng, 0, out)
        sel = LowbitPage(key, self.bits, G, inn,
                         torch.from_numpy(np.ascontiguousarray(packed[flat])).to(self.device),
                         torch.from_numpy(np.ascontiguousarray(scales[flat])).to(self.device))
        return lowbit_dequant(sel).reshape(*shape, inn)

    def _matmul(self, name: str, x: torch.Tensor, *, row_stable: bool) -> torch.Tensor:
        key, b = self._resolve(name)
        pg = self.page(key)
        if pg is not None:
            return lowbit_matmul(pg, x, row_stable=row_stable)
        out, inn = (int(v) for v in b["shape"])
        if int(x.shape[-1]) != inn:
            raise ValueError("activation width does not match the packed block")
        nat.require_device(x)
        x2 = x.reshape(-1, inn)
        if x2.dtype not in (torch.bfloat16, torch.float32):
            x2 = x2.to(torch.float32)
        x2 = x2.contiguous()
        y = torch.empty((int(x2.shape[0]), out), dtype=torch.float32, device=x2.device)
        for start, end, chunk in self._chunks(key, b):
            _gemv_into(chunk, x2, y[:, start:], out, row_stable=row_stable)
        return y.reshape(*x.shape[:-1], out)

    def matmul(self, name: str, x: torch.Tensor) -> torch.Tensor:
        return self._matmul(name, x, row_stable=False)

    def matmul_row_stable(self, name: str, x: torch.Tensor) -> torch.Tensor:
        """Each row runs as its own product: batched rows equal B=1 rows bit for bit."""
        if x.ndim < 2 or int(x.shape[0]) <= 0:
            raise ValueError("row-stable matmul input must have shape [B, ..., in]")
        return self._matmul(name, x, row_stable=True)

    def row_blocks(self, name: str, bs: int = 8192):
        """``(start, end, W[start:end])`` fp32 row blocks (qstore.py:1396-1416)."""
        key, b = self._resolve(name)
        out, inn, rb, ng, G = self._geometry(key, b)
        pg = self.page(key)
        for start in range(0, out, bs):
            end = min(start + bs, out)
            if pg is not None:
                rows = LowbitPage(key, self.bits, G, inn, pg.packed[start:end], pg.scales[start:end])
            else:
                packed, scales = self._host_rows(b, rb, ng, start, end)
                rows = LowbitPage(key, self.bits, G, inn, torch.from_numpy(np.array(packed)).to(self.device),
                                  torch.from_numpy(np.array(scales)).to(self.device))
            yield start, end, lowbit_dequant(rows)

    def device_bytes(self) -> int:
        return self.cache_bytes + sum(st.nbytes() for st in self._stages.values())

    def close(self) -> None:
        """Release the device pages, staging buffers and file mappings (idempotent)."""
        if getattr(self, "_stages", None):
            for st in self._stages.values():
                for ev in st.copied:
                    if ev is not None:
                        ev.synchronize()
        self._pages = {}
        self._stages = {}
        self.cache_bytes = 0
        for attr in ("w", "s", "e"):
            arr = getattr(self, attr, None)
            mm = getattr(arr, "_mmap", None)
            if mm is not None:
                mm.close()
            setattr(self, attr, None)
