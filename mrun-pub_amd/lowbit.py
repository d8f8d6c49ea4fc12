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
    if M:
        xdt = nat.dtype_code(x2.dtype)
        chunk = 1 if row_stable else M
        wsb = int(nat.load().qs_lowbit_workspace_bytes(xdt, chunk, N, K, page.group_size))
        ws = torch.empty(wsb, dtype=torch.uint8, device=device)
        for m0 in range(0, M, chunk):
            mm = min(chunk, M - m0)
            nat.call(
                "qs_lowbit_gemv", nat.ptr(x2[m0:]), xdt, K, nat.ptr(page.packed), page.row_bytes, nat.ptr(page.scales),
                nat.dtype_code(page.scales.dtype), nat.ptr(page.zeros),
                nat.dtype_code(page.zeros.dtype) if page.zeros is not None else nat.QS_F32, page._offset(),
                page.bits, page.group_size, nat.ptr(y[m0:]), N, mm, N, K, nat.ptr(ws), wsb, nat.stream_of(device),
            )
    return y.reshape(*x.shape[:-1], N)


class DeviceLowbitQStore:
    """``QStoreInt3`` / ``QStoreInt2`` reader with HBM-resident blocks (qstore.py:1283-1544).

    Reads a reference-format low-bit store directory: ``manifest.json`` (blocks of kind
    ``qrow3`` / ``qrow2`` with ``shape``, ``w_off``, ``row_bytes``, ``s_off``,
    ``n_groups``, ``group_size``), ``weights.i3`` / ``weights.i2`` and ``scales.f32``.
    """

    _KIND_BITS = {"qrow3": 3, "qrow2": 2}

    def __init__(self, directory: str | Path, *, device: str | torch.device = "cuda"):
        d = Path(directory)
        self.man = json.loads((d / "manifest.json").read_text())
        dtype = self.man.get("dtype")
        if dtype not in ("int3", "int2"):
            raise RuntimeError(f"low-bit QStore must declare dtype int3/int2, got {dtype!r}")
        self.bits = 3 if dtype == "int3" else 2
        self.blocks = self.man["blocks"]
        self.G = int(self.man.get("group_size", 128))
        self.w = np.memmap(d / f"weights.i{self.bits}", dtype=np.uint8, mode="r")
        self.s = np.memmap(d / "scales.f32", dtype=np.float32, mode="r")
        self.device = torch.device(device)
        self._pages: dict[str, LowbitPage] = {}

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

    def page(self, name: str) -> LowbitPage:
        key, b = self._resolve(name)
        if key in self._pages:
            return self._pages[key]
        if b.get("kind") not in self._KIND_BITS:
            raise ValueError(f"{name} is not a packed low-bit block")
        out, inn = (int(v) for v in b["shape"])
        rb, ng = int(b["row_bytes"]), int(b["n_groups"])
        G = int(b.get("group_size", self.G))
        packed = np.array(self.w[b["w_off"] : b["w_off"] + out * rb], dtype=np.uint8).reshape(out, rb)
        so = int(b["s_off"]) // 4
        scales = np.array(self.s[so : so + out * ng], dtype=np.float32).reshape(out, ng)
        pg = LowbitPage(
            key, self._KIND_BITS[b["kind"]], G, inn,
            torch.from_numpy(packed).to(self.device), torch.from_numpy(scales).to(self.device),
        )
        self._pages[key] = pg
        return pg

    def weight(self, name: str) -> torch.Tensor:
        return lowbit_dequant(self.page(name))

    def has(self, name: str) -> bool:
        return str(name) in self.blocks

    def block_kind(self, name: str) -> str | None:
        return self._resolve(name)[1].get("kind")

    def embed_rows(self, name: str, ids) -> torch.Tensor:
        """fp32 rows ``ids`` of a packed block, ``[*ids.shape, in]`` (qstore.py:1382-1395,
        1513-1526).  Only the selected rows are read from the host file."""
        from .qrow import normalize_row_ids

        key, b = self._resolve(name)
        if b.get("kind") not in self._KIND_BITS:
            raise ValueError(f"{name} is not a packed low-bit block")
        out, inn = (int(v) for v in b["shape"])
        rb, ng = int(b["row_bytes"]), int(b["n_groups"])
        G = int(b.get("group_size", self.G))
        flat, shape = normalize_row_ids(ids, out)
        flat = flat.reshape(-1)
        if flat.size == 0:
            return torch.empty((*shape, inn), dtype=torch.float32, device=self.device)
        packed = np.asarray(self.w[b["w_off"] : b["w_off"] + out * rb], dtype=np.uint8).reshape(out, rb)
        so = int(b["s_off"]) // 4
        scales = np.asarray(self.s[so : so + out * ng], dtype=np.float32).reshape(out, ng)
        sel = LowbitPage(key, self._KIND_BITS[b["kind"]], G, inn,
                         torch.from_numpy(np.ascontiguousarray(packed[flat])).to(self.device),
                         torch.from_numpy(np.ascontiguousarray(scales[flat])).to(self.device))
        return lowbit_dequant(sel).reshape(*shape, inn)

    def matmul(self, name: str, x: torch.Tensor) -> torch.Tensor:
        return lowbit_matmul(self.page(name), x)

    def matmul_row_stable(self, name: str, x: torch.Tensor) -> torch.Tensor:
        """Each row runs as its own product: batched rows equal B=1 rows bit for bit."""
        if x.ndim < 2 or int(x.shape[0]) <= 0:
            raise ValueError("row-stable matmul input must have shape [B, ..., in]")
        return lowbit_matmul(self.page(name), x, row_stable=True)

    def row_blocks(self, name: str, bs: int = 8192):
        W = self.weight(name)
        for start in range(0, W.shape[0], bs):
            end = min(start + bs, W.shape[0])
            yield start, end, W[start:end]
