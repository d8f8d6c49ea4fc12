"""QStore int8 format: writer -> validated memory-mapped reader (CPU), v3 and legacy
manifests, and the store fixtures written with the reference's own code."""

from __future__ import annotations

import hashlib
import json
import shutil
from pathlib import Path

import numpy as np
import pytest

from mrun_pub_amd.store import QStoreReader, reseal_qstore, write_qstore

GOLD = Path(__file__).resolve().parent / "golden"


def _blocks(seed=0):
    rng = np.random.default_rng(seed)
    out = {}
    for name, (n, k) in {"l0.q": (32, 64), "l0.k": (8, 64), "l0.down": (64, 96)}.items():
        out[name] = (rng.integers(-127, 128, size=(n, k), dtype=np.int8),
                     (rng.uniform(0.5, 1.5, n) / 127).astype(np.float32))
    return out


def test_round_trip_and_aliases(tmp_path):
    blocks = _blocks()
    norm = np.arange(64, dtype=np.float32)
    write_qstore(tmp_path, blocks, {"l0.norm": norm}, aliases={"lm_head": "l0.q", "tied": "lm_head"})
    r = QStoreReader(tmp_path)
    assert r.content_identity_verified
    for name, (codes, scales) in blocks.items():
        c, s = r.qrow(name)
        np.testing.assert_array_equal(c, codes)
        np.testing.assert_array_equal(s, scales)
    np.testing.assert_array_equal(r.qrow("tied")[0], blocks["l0.q"][0])
    np.testing.assert_array_equal(r.fp32("l0.norm"), norm)
    c, s = r.qrow("l0.down", 10, 20)
    np.testing.assert_array_equal(c, blocks["l0.down"][0][10:20])
    assert sorted(r.qrow_names()) == sorted(blocks)
    with pytest.raises(KeyError):
        r.qrow("missing")
    with pytest.raises(ValueError):
        r.qrow("l0.norm")
    with pytest.raises(ValueError):
        r.qrow("l0.q", 5, 5)


_NORM = {"l0.norm": np.arange(64, dtype=np.float32)}


def _corrupt(tmp_path, edit):
    """Edit a v3 manifest and re-seal its provenance, so that the layout rules (not the
    digests) are what the reader trips over."""
    write_qstore(tmp_path, _blocks(), _NORM)
    man = json.loads((tmp_path / "manifest.json").read_text())
    edit(man)
    (tmp_path / "manifest.json").write_text(json.dumps(man))
    reseal_qstore(tmp_path)


@pytest.mark.parametrize(
    "edit",
    [
        lambda m: m["blocks"]["l0.k"].update(w_off=m["blocks"]["l0.k"]["w_off"] + 1),  # gap/overlap
        lambda m: m["blocks"]["l0.q"].update(w_len=7),  # length != shape
        lambda m: m["blocks"]["l0.q"].update(s_off=2),  # misaligned scales
        lambda m: m["blocks"].update(x={"alias": "nowhere"}),  # dangling alias
        lambda m: m["blocks"].update(a={"alias": "b"}, b={"alias": "a"}),  # alias cycle
        lambda m: m.update(dtype="int4"),
        lambda m: m["blocks"]["l0.q"].update(kind="qrow9"),
        lambda m: m["blocks"]["l0.q"].update(shape=[32, True]),
        lambda m: m["blocks"].pop("l0.norm"),  # v3 needs an fp32 block (and extras covered)
    ],
)
def test_layout_violations_are_rejected(tmp_path, edit):
    # reference _validate_int8_layout, src/mrun/engine/kernels/qstore.py:124-219
    _corrupt(tmp_path, edit)
    with pytest.raises(RuntimeError):
        QStoreReader(tmp_path)


def test_truncated_file_is_rejected(tmp_path):
    write_qstore(tmp_path, _blocks(), _NORM)
    data = (tmp_path / "weights.i8").read_bytes()
    (tmp_path / "weights.i8").write_bytes(data[:-1])
    # the layout check runs before the files are hashed (qstore.py:345-358)
    with pytest.raises(RuntimeError, match="exceeds|cover"):
        QStoreReader(tmp_path)


def test_written_v3_store_is_content_verified(tmp_path):
    write_qstore(tmp_path, _blocks(), _NORM)
    r = QStoreReader(tmp_path)
    assert r.content_identity_verified
    assert r.identity_status == "content-addressed-semantic-v2-files-verified"
    # a flipped weight byte, an edited block table, an edited source record: all refused
    for edit in ("blob", "manifest", "source"):
        d = tmp_path.parent / f"{tmp_path.name}_{edit}"
        shutil.copytree(tmp_path, d)
        if edit == "blob":
            b = bytearray((d / "weights.i8").read_bytes())
            b[5] ^= 1
            (d / "weights.i8").write_bytes(bytes(b))
        else:
            man = json.loads((d / "manifest.json").read_text())
            if edit == "manifest":
                man["blocks"]["l0.q"]["shape"] = [32, 64]
                man["config"]["x"] = 1
            else:
                man["source"]["model_name"] = "other"
                man["source"]["safetensors"][0]["bytes"] += 1
            (d / "manifest.json").write_text(json.dumps(man))
        with pytest.raises(RuntimeError, match="mismatch|does not match"):
            QStoreReader(d)


def test_legacy_store_opens_unvalidated(tmp_path):
    """Non-v3 manifests open without layout validation (qstore.py:334-343); a block that
    leaves its file fails when read, not on open."""
    blocks = _blocks()
    write_qstore(tmp_path, blocks, legacy=True)
    r = QStoreReader(tmp_path)
    assert not r.content_identity_verified and r.identity_status == "legacy-unverified"
    np.testing.assert_array_equal(r.qrow("l0.k")[0], blocks["l0.k"][0])
    man = json.loads((tmp_path / "manifest.json").read_text())
    man["blocks"]["l0.k"]["w_off"] = 10**9
    (tmp_path / "manifest.json").write_text(json.dumps(man))
    r = QStoreReader(tmp_path)
    with pytest.raises(RuntimeError, match="exceeds"):
        r.qrow("l0.k")


def _golden():
    manifest = json.loads((GOLD / "golden_manifest.json").read_text())
    path = GOLD / "refstore.npz"
    assert hashlib.sha256(path.read_bytes()).hexdigest() == manifest["refstore.npz"]
    return np.load(path, allow_pickle=False), json.loads((GOLD / "refstore.json").read_text())


def test_reference_test_layout_store(tmp_path):
    """The reference's own test store layout (tests/test_qstore_cache.py:19-46: no dtype,
    an unreferenced 4-byte extras file) opens, and its rows dequantize to what the
    reference's QStore.weight / embed_rows returned (refstore.npz, written by the
    reference)."""
    g, info = _golden()
    shutil.copytree(GOLD / "refstore" / "legacy", tmp_path / "s")
    r = QStoreReader(tmp_path / "s")
    assert r.identity_status == info["legacy"]["identity_status"]
    assert r.content_identity_verified == info["legacy"]["content_identity_verified"]
    for name in ("L0.q", "L0.up"):
        codes, scales = r.qrow(name)
        w = codes.astype(np.float32) * scales[:, None]
        assert np.array_equal(w.view(np.uint32), g[f"legacy_weight_{name}"].view(np.uint32))
        ids = g["legacy_ids"]
        c, s = r.qrow_rows(name, ids)
        e = (c.astype(np.float32) * s[:, None]).reshape(*ids.shape, -1)
        assert np.array_equal(e.view(np.uint32), g[f"legacy_embed_{name}"].view(np.uint32))


def test_reference_sealed_v3_store(tmp_path):
    """A v3 store whose provenance the reference's own functions built verifies here with
    the same digests the reference's QStore reported."""
    g, info = _golden()
    shutil.copytree(GOLD / "refstore" / "v3", tmp_path / "s")
    r = QStoreReader(tmp_path / "s")
    assert r.content_identity_verified
    for key in ("identity_status", "source_checkpoint_sha256", "derived_store_sha256",
                "manifest_semantic_sha256"):
        assert r.identity[key] == info["v3"][key], key
    codes, scales = r.qrow("lm_head")
    assert np.array_equal(codes.astype(np.float32) * scales[:, None], g["v3_weight_lm_head"])
    assert np.array_equal(r.fp32("L0.norm"), g["v3_fp32_L0.norm"])
    b = bytearray((tmp_path / "s" / "scales.f32").read_bytes())
    b[0] ^= 0x40
    (tmp_path / "s" / "scales.f32").write_bytes(bytes(b))
    with pytest.raises(RuntimeError, match="hash mismatch"):
        QStoreReader(tmp_path / "s")
