"""Content addresses of QStore v3 stores (the reference's provenance format).

A v3 manifest carries three provenance records (reference
src/mrun/store_provenance.py:150-175 source, :231-275 derived, :390-412 builder):

* ``source``  -- file records of the checkpoint the store was built from, bound by
  ``source_checkpoint_sha256`` = canonical hash of ``{schema_version, config, index,
  safetensors}``;
* ``builder`` -- file records of the code that built it, bound by
  ``source_bundle_sha256`` = canonical hash of ``{schema_version, files}``;
* ``derived`` -- one record per store file plus ``manifest_semantic_sha256`` (the manifest
  without ``derived``, with the machine-local ``source_dir`` and ``revision`` left out),
  bound by ``derived_store_sha256``.

A record is ``{"name", "bytes", "sha256"}``; a canonical hash is SHA-256 of the compact
sorted-key JSON text.  The schema names and the hashing rules are a compatibility
contract: a store the reference wrote verifies here and the other way round.  Errors are
``RuntimeError`` (store corruption), as in the reference.
"""

from __future__ import annotations

import hashlib
import json
from collections.abc import Iterable, Mapping
from pathlib import Path
from typing import Any

SOURCE_SCHEMA = "mrun-source-checkpoint-v1"
DERIVED_SCHEMA_SEMANTIC = "mrun-derived-store-v2"
SEMANTIC_MANIFEST_SCHEMA = "mrun-store-semantic-manifest-v1"
BUILDER_SCHEMA = "mrun-store-builder-v1"

_HEX = frozenset("0123456789abcdef")


def canonical_sha256(payload: object) -> str:
    text = json.dumps(payload, sort_keys=True, separators=(",", ":"))
    return hashlib.sha256(text.encode("utf-8")).hexdigest()


def sha256_file(path: Path) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as fh:
        while True:
            chunk = fh.read(1 << 23)
            if not chunk:
                return h.hexdigest()
            h.update(chunk)


def is_digest(value: object) -> bool:
    return isinstance(value, str) and len(value) == 64 and set(value) <= _HEX


def file_record(path: Path, name: str | None = None) -> dict[str, Any]:
    """``{"name", "bytes", "sha256"}`` of one non-empty file."""
    path = Path(path)
    if not path.is_file():
        raise RuntimeError(f"provenance input is missing: {path}")
    size = path.stat().st_size
    if size <= 0:
        raise RuntimeError(f"provenance input is empty: {path}")
    return {"name": name or path.name, "bytes": size, "sha256": sha256_file(path)}


def bytes_record(name: str, data: bytes) -> dict[str, Any]:
    """The record of a file whose content is ``data`` (for writers that hold it in memory)."""
    if not data:
        raise RuntimeError(f"provenance input is empty: {name}")
    return {"name": name, "bytes": len(data), "sha256": hashlib.sha256(data).hexdigest()}


def semantic_manifest_sha256(manifest: Mapping[str, Any]) -> str:
    body = {str(k): v for k, v in manifest.items() if k != "derived"}
    src = body.get("source")
    if isinstance(src, Mapping):
        body["source"] = {k: v for k, v in src.items() if k not in ("source_dir", "revision")}
    return canonical_sha256({"schema_version": SEMANTIC_MANIFEST_SCHEMA, "manifest": body})


def derived_record(directory: Path, filenames: Iterable[str], manifest: Mapping[str, Any]) -> dict[str, Any]:
    """The ``derived`` record of a store directory (hashes every listed file)."""
    files = [file_record(Path(directory) / n, n) for n in sorted(set(filenames))]
    content = {
        "schema_version": DERIVED_SCHEMA_SEMANTIC,
        "files": files,
        "manifest_semantic_sha256": semantic_manifest_sha256(manifest),
    }
    return {**content, "derived_store_sha256": canonical_sha256(content)}


def source_record(*, model_name: str, hf_id: str, config: Mapping[str, Any],
                  index: Mapping[str, Any] | None, safetensors: list[Mapping[str, Any]],
                  revision: Mapping[str, Any] | None = None) -> dict[str, Any]:
    """A ``source`` record over already-computed file records."""
    content = {"schema_version": SOURCE_SCHEMA, "config": dict(config),
               "index": None if index is None else dict(index),
               "safetensors": [dict(r) for r in safetensors]}
    return {**content, "model_name": model_name, "hf_id": hf_id,
            "revision": dict(revision or {"kind": "unknown", "commits": []}),
            "source_checkpoint_sha256": canonical_sha256(content)}


def builder_record(*, name: str, build_schema_version: str, source_files: list[Mapping[str, Any]],
                   quantization: Mapping[str, Any]) -> dict[str, Any]:
    files = [dict(r) for r in source_files]
    return {"schema_version": BUILDER_SCHEMA, "name": name, "build_schema_version": build_schema_version,
            "source_files": files,
            "source_bundle_sha256": canonical_sha256({"schema_version": BUILDER_SCHEMA, "files": files}),
            "quantization": dict(quantization)}


def _check_source(source: object) -> Mapping[str, Any]:
    if not isinstance(source, Mapping):
        raise RuntimeError("store has no publication-grade source provenance")
    need = ("schema_version", "model_name", "hf_id", "revision", "config", "index", "safetensors",
            "source_checkpoint_sha256")
    absent = [k for k in need if k not in source]
    if absent:
        raise RuntimeError(f"store source provenance is incomplete: {absent}")
    if source["schema_version"] != SOURCE_SCHEMA:
        raise RuntimeError("store source provenance schema mismatch")
    digest = source["source_checkpoint_sha256"]
    if not is_digest(digest):
        raise RuntimeError("store source checkpoint digest is invalid")
    bound = {k: source.get(k) for k in ("schema_version", "config", "index", "safetensors")}
    if digest != canonical_sha256(bound):
        raise RuntimeError("store source checkpoint digest does not match its file records")
    return source


def _check_builder(builder: object) -> None:
    if not isinstance(builder, Mapping):
        raise RuntimeError("store has no publication-grade builder provenance")
    if builder.get("schema_version") != BUILDER_SCHEMA:
        raise RuntimeError("store builder provenance schema mismatch")
    files = builder.get("source_files")
    if not isinstance(files, list) or not files:
        raise RuntimeError("store builder provenance has no source files")
    digest = builder.get("source_bundle_sha256")
    if not is_digest(digest) or digest != canonical_sha256({"schema_version": BUILDER_SCHEMA, "files": files}):
        raise RuntimeError("store builder source digest does not match its file records")


def _check_derived_semantics(manifest: Mapping[str, Any]) -> Mapping[str, Any]:
    derived = manifest.get("derived")
    if not isinstance(derived, Mapping):
        raise RuntimeError("store has no semantic derived provenance")
    if derived.get("schema_version") != DERIVED_SCHEMA_SEMANTIC:
        raise RuntimeError("store semantic derived provenance schema mismatch")
    files = derived.get("files")
    if not isinstance(files, list) or not files:
        raise RuntimeError("store semantic derived provenance has no files")
    names = [r.get("name") for r in files if isinstance(r, Mapping)]
    if len(names) != len(files) or names != sorted(set(names)):
        raise RuntimeError("store semantic derived file records are invalid")
    for r in files:
        size = r.get("bytes")
        if isinstance(size, bool) or not isinstance(size, int) or size <= 0 or not is_digest(r.get("sha256")):
            raise RuntimeError("store semantic derived file record is invalid")
    sem = derived.get("manifest_semantic_sha256")
    if not is_digest(sem) or sem != semantic_manifest_sha256(manifest):
        raise RuntimeError("store semantic manifest digest mismatch")
    content = {"schema_version": DERIVED_SCHEMA_SEMANTIC, "files": files, "manifest_semantic_sha256": sem}
    store_digest = derived.get("derived_store_sha256")
    if not is_digest(store_digest) or store_digest != canonical_sha256(content):
        raise RuntimeError("store derived digest does not match its semantic/file records")
    return derived


def check_semantic_identity(manifest: Mapping[str, Any]) -> dict[str, Any]:
    """Strict check of the internal digests of a v3 manifest, without reading any blob
    (reference inspect_semantic_store_identity(strict=True), store_provenance.py:278-378)."""
    source = _check_source(manifest.get("source"))
    _check_builder(manifest.get("builder"))
    derived = _check_derived_semantics(manifest)
    return {
        "source_checkpoint_sha256": source["source_checkpoint_sha256"],
        "derived_store_sha256": derived["derived_store_sha256"],
        "manifest_semantic_sha256": derived["manifest_semantic_sha256"],
    }


def verify_store_files(directory: Path, manifest: Mapping[str, Any], filenames: Iterable[str]) -> None:
    """Re-hash the store files and compare with the ``derived`` record
    (reference verify_derived_provenance, store_provenance.py:254-275)."""
    derived = manifest.get("derived")
    if not isinstance(derived, Mapping):
        raise RuntimeError("existing store has no publication-grade derived-file provenance")
    names = sorted(set(filenames))
    files = derived.get("files")
    if derived.get("schema_version") != DERIVED_SCHEMA_SEMANTIC or not isinstance(files, list):
        raise RuntimeError("existing store derived-file provenance schema mismatch")
    if [r.get("name") if isinstance(r, Mapping) else None for r in files] != names:
        raise RuntimeError("existing store derived-file set mismatch")
    semantic = {k: v for k, v in manifest.items() if k != "derived"}
    try:
        fresh = derived_record(directory, names, semantic)
    except RuntimeError as exc:
        raise RuntimeError(f"existing store derived-file hash mismatch ({exc})") from exc
    if dict(derived) != fresh:
        raise RuntimeError("existing store derived-file hash mismatch")


def legacy_identity(manifest: object) -> dict[str, Any]:
    """Identity of a manifest that is not v3: declared digests are reported, never trusted
    (reference store_provenance.py:295-318)."""
    src = drv = None
    if isinstance(manifest, Mapping):
        s, d = manifest.get("source"), manifest.get("derived")
        if isinstance(s, Mapping) and is_digest(s.get("source_checkpoint_sha256")):
            src = s["source_checkpoint_sha256"]
        if isinstance(d, Mapping) and is_digest(d.get("derived_store_sha256")):
            drv = d["derived_store_sha256"]
    return {
        "content_identity_verified": False,
        "semantic_identity_verified": False,
        "blob_identity_verified": False,
        "identity_status": "declared-content-only-unverified" if src and drv else "legacy-unverified",
        "source_checkpoint_sha256": src,
        "derived_store_sha256": drv,
        "manifest_semantic_sha256": None,
    }
