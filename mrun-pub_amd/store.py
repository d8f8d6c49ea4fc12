"""QStore int8 on-disk format: manifest reader/validator and a writer.

Format (reference src/mrun/engine/kernels/qstore_build.py:1-25, 556-713; reader
src/mrun/engine/kernels/qstore.py:124-219, 326-373, 677-741):

* ``manifest.json`` -- ``{"schema_version", "dtype": "int8", "config": {...}, "blocks":
  {name: desc}, "source", "builder", "derived", ...}`` where ``desc`` is ``{"kind": "qrow",
  "shape": [out, in], "w_off", "w_len", "s_off", "s_len"}``, ``{"kind": "fp32", "shape":
  [...], "e_off", "e_len"}`` or ``{"alias": other}``;
* ``weights.i8`` -- int8 row-major codes of every qrow block, back to back;
* ``scales.f32`` -- one fp32 scale per output row of every qrow block;
* ``extras.f32`` -- fp32 tensors (norms, biases).

Opening follows ``_load_qstore_manifest`` (qstore.py:326-373):

* ``schema_version == "mrun-qstore-int8-v3"``: the manifest's own digests are checked
  (``provenance.check_semantic_identity``), every block mapping is validated as
  ``_validate_int8_layout`` does (qstore.py:124-219: ranges contiguous, gap-free, in
  bounds, covering each file; qrow and fp32 blocks present; aliases acyclic), and the
  files are re-hashed against the ``derived`` record.  Any violation is a ``RuntimeError``.
* any other manifest (legacy and v2 stores, e.g. the reference's own test stores with no
  ``dtype``): opened without layout validation, identity ``legacy-unverified``; a block
  whose range falls outside its file raises ``RuntimeError`` when it is read.

Unknown blocks raise ``KeyError``.
"""

from __future__ import annotations

import json
import math
from collections.abc import Mapping
from pathlib import Path
from typing import Any

import numpy as np

from . import provenance

QSTORE_SCHEMA = "mrun-qstore-int8-v3"
QSTORE_FILES = ("weights.i8", "scales.f32", "extras.f32")
QSTORE_QUANTIZATION = {
    "codec": "symmetric-int8",
    "granularity": "per-output-channel",
    "scale_dtype": "float32",
    "full_precision_blocks": "float32",
    "zero_point": 0,
}


def _req_int(block: Mapping[str, Any], key: str, *, positive: bool = False) -> int:
    value = block.get(key)
    if isinstance(value, bool) or not isinstance(value, int):
        raise RuntimeError(f"QStore block field {key!r} must be an integer")
    if value < (1 if positive else 0):
        raise RuntimeError(f"QStore block field {key!r} must be {'positive' if positive else 'non-negative'}")
    return value


def _req_shape(block: Mapping[str, Any], dims: int | None = None) -> tuple[int, ...]:
    raw = block.get("shape")
    if not isinstance(raw, list) or not raw:
        raise RuntimeError("QStore block shape must be a non-empty list")
    if any(isinstance(v, bool) or not isinstance(v, int) or v <= 0 for v in raw):
        raise RuntimeError("QStore block shape dimensions must be positive integers")
    if dims is not None and len(raw) != dims:
        raise RuntimeError(f"QStore block shape must have {dims} dimensions")
    return tuple(raw)


def validate_int8_layout(directory: Path, manifest: Mapping[str, Any]) -> None:
    """Check every block mapping of a v3 store before any memory map is opened
    (qstore.py:124-219)."""
    if manifest.get("dtype") != "int8":
        raise RuntimeError("semantic QStore v3 must declare dtype='int8'")
    blocks = manifest.get("blocks")
    if not isinstance(manifest.get("config"), Mapping) or not isinstance(blocks, Mapping) or not blocks:
        raise RuntimeError("semantic QStore v3 requires config and a non-empty block table")
    intervals: dict[str, list[tuple[int, int, str]]] = {f: [] for f in QSTORE_FILES}
    n_qrow = n_fp32 = 0
    for name, blk in blocks.items():
        if not isinstance(name, str) or not name or not isinstance(blk, Mapping):
            raise RuntimeError("QStore block names and descriptors must be non-empty mappings")
        if "alias" in blk:
            if not isinstance(blk.get("alias"), str) or not blk["alias"]:
                raise RuntimeError(f"QStore alias {name!r} has an invalid target")
            continue
        kind = blk.get("kind")
        if kind == "qrow":
            out, inn = _req_shape(blk, 2)
            w_off, w_len = _req_int(blk, "w_off"), _req_int(blk, "w_len", positive=True)
            s_off, s_len = _req_int(blk, "s_off"), _req_int(blk, "s_len", positive=True)
            if w_len != out * inn:
                raise RuntimeError(f"QStore qrow {name!r} weight length does not match its shape")
            if s_len != out * 4 or s_off % 4:
                raise RuntimeError(f"QStore qrow {name!r} scale range does not match its shape")
            intervals["weights.i8"].append((w_off, w_off + w_len, name))
            intervals["scales.f32"].append((s_off, s_off + s_len, name))
            n_qrow += 1
        elif kind == "fp32":
            shape = _req_shape(blk)
            e_off, e_len = _req_int(blk, "e_off"), _req_int(blk, "e_len", positive=True)
            if e_len != math.prod(shape) * 4 or e_off % 4:
                raise RuntimeError(f"QStore fp32 {name!r} range does not match its shape")
            intervals["extras.f32"].append((e_off, e_off + e_len, name))
            n_fp32 += 1
        else:
            raise RuntimeError(f"QStore block {name!r} has unsupported kind {kind!r}")
    if not n_qrow or not n_fp32:
        raise RuntimeError("semantic QStore v3 requires qrow and fp32 blocks")
    for name, blk in blocks.items():
        if isinstance(blk, Mapping) and "alias" in blk:
            seen = {name}
            target = blk["alias"]
            while True:
                if target not in blocks:
                    raise RuntimeError(f"QStore alias {name!r} targets missing block {target!r}")
                if target in seen:
                    raise RuntimeError(f"QStore alias cycle contains {target!r}")
                seen.add(target)
                nxt = blocks[target].get("alias") if isinstance(blocks[target], Mapping) else None
                if nxt is None:
                    break
                target = nxt
    for filename, ranges in intervals.items():
        path = directory / filename
        if not path.is_file():
            raise RuntimeError(f"QStore derived file is missing: {filename}")
        size = path.stat().st_size
        if not ranges:
            raise RuntimeError(f"QStore block table does not reference {filename}")
        prev = 0
        for start, end, bname in sorted(ranges):
            if end > size:
                raise RuntimeError(f"QStore {filename} range for block {bname!r} exceeds file bounds")
            if start < prev:
                raise RuntimeError(f"QStore {filename} ranges overlap at block {bname!r}")
            if start != prev:
                raise RuntimeError(f"QStore {filename} has an unreferenced gap before block {bname!r}")
            prev = end
        if prev != size:
            raise RuntimeError(f"QStore {filename} block ranges do not cover the complete file")


class QStoreReader:
    """Memory-mapped read-only view of an int8 QStore directory.

    ``identity`` reports what was verified: ``content_identity_verified`` is True only for
    a v3 store whose manifest digests and file hashes all matched on open.
    """

    def __init__(self, directory: str | Path):
        d = Path(directory).resolve()
        manifest = json.loads((d / "manifest.json").read_text(encoding="utf-8"))
        if not isinstance(manifest, dict):
            raise RuntimeError("QStore manifest must be a JSON object")
        if manifest.get("schema_version") == QSTORE_SCHEMA:
            ids = provenance.check_semantic_identity(manifest)
            validate_int8_layout(d, manifest)
            provenance.verify_store_files(d, manifest, QSTORE_FILES)
            self.identity = {
                "content_identity_verified": True,
                "semantic_identity_verified": True,
                "blob_identity_verified": True,
                "identity_status": "content-addressed-semantic-v2-files-verified",
                **ids,
            }
        else:
            blocks = manifest.get("blocks")
            if not isinstance(blocks, Mapping):
                raise RuntimeError("QStore manifest has no block table")
            self.identity = provenance.legacy_identity(manifest)
        self.directory = d
        self.man = manifest
        self.schema_version = manifest.get("schema_version")
        self.blocks: dict[str, dict] = manifest["blocks"]
        self.cfg = manifest.get("config", {})
        self.w = self._map("weights.i8", np.int8)
        self.s = self._map("scales.f32", np.float32)
        self.e = self._map("extras.f32", np.float32)

    @property
    def content_identity_verified(self) -> bool:
        return bool(self.identity["content_identity_verified"])

    @property
    def identity_status(self) -> str:
        return str(self.identity["identity_status"])

    def _map(self, filename: str, dtype) -> np.ndarray:
        path = self.directory / filename
        if not path.is_file():
            raise RuntimeError(f"QStore file is missing: {filename}")
        if path.stat().st_size < np.dtype(dtype).itemsize:
            return np.zeros(0, dtype)
        return np.memmap(path, dtype=dtype, mode="r")

    @staticmethod
    def _span(arr: np.ndarray, start: int, count: int, what: str) -> np.ndarray:
        """``arr[start:start+count]``, or RuntimeError when the range leaves the file
        (legacy stores are not validated on open)."""
        if start < 0 or count < 0 or start + count > arr.shape[0]:
            raise RuntimeError(f"QStore {what} range exceeds its file")
        return np.asarray(arr[start : start + count])

    def _resolve(self, name: str) -> dict:
        """Follow aliases (qstore.py:928-942)."""
        key = str(name)
        seen: set[str] = set()
        while True:
            if key in seen:
                raise RuntimeError(f"cyclic QStore alias at {name!r}")
            seen.add(key)
            try:
                block = self.blocks[key]
            except KeyError as exc:
                raise KeyError(f"QStore has no block {key!r}") from exc
            alias = block.get("alias")
            if alias is None:
                return block
            key = str(alias)

    def has(self, name: str) -> bool:
        return name in self.blocks

    def qrow(self, name: str, start_row: int = 0, end_row: int | None = None) -> tuple[np.ndarray, np.ndarray]:
        """``(codes int8[rows, in], scales f32[rows])`` views of a qrow block row range."""
        b = self._resolve(name)
        if b.get("kind") != "qrow":
            raise ValueError(f"{name} is not a qrow block")
        out, inn = (int(v) for v in b["shape"])
        stop = out if end_row is None else int(end_row)
        if start_row < 0 or stop <= start_row or stop > out:
            raise ValueError(f"invalid row range [{start_row}, {stop}) for {name}")
        w0 = int(b["w_off"]) + start_row * inn
        codes = self._span(self.w, w0, (stop - start_row) * inn, f"weights of {name!r}")
        s0 = int(b["s_off"]) // 4 + start_row
        scales = self._span(self.s, s0, stop - start_row, f"scales of {name!r}")
        return codes.reshape(stop - start_row, inn), scales

    def qrow_rows(self, name: str, ids: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
        """``(codes int8[n, in], scales f32[n])`` of the rows ``ids`` (flattened) of a qrow
        block; indices follow numpy rules (negative counts from the end)."""
        b = self._resolve(name)
        if b.get("kind") != "qrow":
            raise ValueError(f"{name} is not a qrow block")
        out, inn = (int(v) for v in b["shape"])
        codes = self._span(self.w, int(b["w_off"]), out * inn, f"weights of {name!r}").reshape(out, inn)
        scales = self._span(self.s, int(b["s_off"]) // 4, out, f"scales of {name!r}")
        flat = np.asarray(ids, dtype=np.int64).reshape(-1)
        return codes[flat], scales[flat]

    def block_kind(self, name: str) -> str | None:
        return self._resolve(name).get("kind")

    def fp32(self, name: str) -> np.ndarray:
        b = self._resolve(name)
        if b.get("kind") != "fp32":
            raise ValueError(f"{name} is not an fp32 block")
        n = math.prod(b["shape"])
        off = int(b["e_off"]) // 4
        return np.array(self._span(self.e, off, n, f"extras of {name!r}"), dtype=np.float32).reshape(b["shape"])

    def qrow_names(self) -> list[str]:
        return [n for n, b in self.blocks.items() if isinstance(b, Mapping) and b.get("kind") == "qrow"]


def write_qstore(
    directory: str | Path,
    qrow: Mapping[str, tuple[np.ndarray, np.ndarray]],
    fp32: Mapping[str, np.ndarray] | None = None,
    *,
    aliases: Mapping[str, str] | None = None,
    config: Mapping[str, Any] | None = None,
    model_name: str = "synthetic",
    legacy: bool = False,
) -> Path:
    """Write an int8 QStore with the reference builder's layout (qstore_build.py:556-713).

    By default the store is v3: ``schema_version``, ``dtype``, and content-addressed
    ``source`` / ``builder`` / ``derived`` records.  The source records hash the arrays
    handed in (one record per block, config as JSON), since no checkpoint file exists
    here.  A v3 store needs at least one fp32 block.  ``legacy=True`` writes the older
    manifest without a schema version or provenance, as the reference's own tests do.
    """
    d = Path(directory)
    d.mkdir(parents=True, exist_ok=True)
    blocks: dict[str, dict] = {}
    source_files: list[dict] = []
    w_off = s_off = e_off = 0
    with open(d / "weights.i8", "wb") as wf, open(d / "scales.f32", "wb") as sf, open(d / "extras.f32", "wb") as ef:
        for name, (codes, scales) in qrow.items():
            codes = np.ascontiguousarray(codes, dtype=np.int8)
            scales = np.ascontiguousarray(scales, dtype=np.float32)
            if codes.ndim != 2 or scales.shape != (codes.shape[0],):
                raise ValueError(f"{name}: codes [out,in] and scales [out] required")
            wf.write(codes.tobytes())
            sf.write(scales.tobytes())
            source_files.append(provenance.bytes_record(f"{name}.qrow", codes.tobytes() + scales.tobytes()))
            blocks[name] = {"kind": "qrow", "shape": list(codes.shape), "w_off": w_off,
                            "w_len": codes.nbytes, "s_off": s_off, "s_len": scales.nbytes}
            w_off += codes.nbytes
            s_off += scales.nbytes
        for name, arr in (fp32 or {}).items():
            arr = np.ascontiguousarray(arr, dtype=np.float32)
            ef.write(arr.tobytes())
            source_files.append(provenance.bytes_record(f"{name}.fp32", arr.tobytes()))
            blocks[name] = {"kind": "fp32", "shape": list(arr.shape), "e_off": e_off, "e_len": arr.nbytes}
            e_off += arr.nbytes
    for name, target in (aliases or {}).items():
        blocks[name] = {"alias": target}
    cfg = dict(config or {})
    if legacy:
        manifest: dict[str, Any] = {"dtype": "int8", "config": cfg, "blocks": blocks}
    else:
        if not fp32:
            raise ValueError("a v3 QStore needs at least one fp32 block")
        source = provenance.source_record(
            model_name=model_name, hf_id=model_name,
            config=provenance.bytes_record("config.json", json.dumps(cfg, sort_keys=True).encode()),
            index=None, safetensors=sorted(source_files, key=lambda r: r["name"]))
        builder = provenance.builder_record(
            name="mrun_pub_amd.store.write_qstore", build_schema_version=QSTORE_SCHEMA,
            source_files=[provenance.file_record(Path(__file__), "mrun_pub_amd/store.py")],
            quantization=QSTORE_QUANTIZATION)
        manifest = {"schema_version": QSTORE_SCHEMA, "model_name": model_name, "dtype": "int8",
                    "config": cfg, "source": source, "builder": builder, "blocks": blocks}
        manifest["derived"] = provenance.derived_record(d, QSTORE_FILES, manifest)
    (d / "manifest.json").write_text(json.dumps(manifest, indent=1, sort_keys=True) + "\n")
    return d


def reseal_qstore(directory: str | Path) -> None:
    """Recompute the ``derived`` record of a v3 store after its manifest or files were edited
    (for writers that patch a store in place; tests use it to reach the layout checks)."""
    d = Path(directory)
    manifest = json.loads((d / "manifest.json").read_text(encoding="utf-8"))
    manifest.pop("derived", None)
    manifest["derived"] = provenance.derived_record(d, QSTORE_FILES, manifest)
    (d / "manifest.json").write_text(json.dumps(manifest, indent=1, sort_keys=True) + "\n")
