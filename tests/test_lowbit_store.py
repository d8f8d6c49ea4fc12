"""Opening low-bit (int3 / int2) stores: the reference's rules and this reader's range
checks, on the host (no device work happens before a block is used)."""

from __future__ import annotations

import json
import shutil
from pathlib import Path

import numpy as np
import pytest

GOLD = Path(__file__).resolve().parent / "golden" / "lowbit_store"


def _lb():
    from mrun_pub_amd import lowbit

    return lowbit


def _copy(tmp_path, bits):
    d = tmp_path / f"toy-int{bits}"
    shutil.copytree(GOLD / f"toy-int{bits}", d)
    return d


def _edit(d, fn):
    man = json.loads((d / "manifest.json").read_text())
    fn(man)
    (d / "manifest.json").write_text(json.dumps(man))


@pytest.mark.parametrize("bits", [3, 2])
def test_reference_layout_stores_open(bits):
    store = _lb().DeviceLowbitQStore(GOLD / f"toy-int{bits}", dtype=f"int{bits}")
    assert store.bits == bits and store.G == 128 and store.matmul_chunk_rows == 24
    assert store.has("A2") and store.block_kind("A2") == f"qrow{bits}" and store.block_kind("norm") == "fp32"
    store.close()
    store.close()  # idempotent


def test_manifest_rules(tmp_path):
    lb = _lb()
    d = _copy(tmp_path, 3)
    with pytest.raises(RuntimeError, match="dtype"):
        lb.DeviceLowbitQStore(d, dtype="int2")
    (d / "manifest.json").write_text("[1, 2]")
    with pytest.raises(RuntimeError, match="JSON object"):
        lb.DeviceLowbitQStore(d)
    d = _copy(tmp_path / "a", 3)
    _edit(d, lambda m: m.update(schema_version="mrun-qstore-int8-v3"))
    with pytest.raises(RuntimeError, match="unsupported semantic QStore dtype"):
        lb.DeviceLowbitQStore(d)
    d = _copy(tmp_path / "b", 3)
    _edit(d, lambda m: m.pop("group_size"))
    with pytest.raises(KeyError):
        lb.DeviceLowbitQStore(d)
    d = _copy(tmp_path / "c", 3)
    _edit(d, lambda m: m.pop("config"))
    with pytest.raises(KeyError):
        lb.DeviceLowbitQStore(d)


def test_runtime_files_must_be_regular(tmp_path):
    lb = _lb()
    d = _copy(tmp_path, 2)
    (d / "extras.f32").unlink()
    with pytest.raises(RuntimeError, match="unavailable: extras.f32"):
        lb.DeviceLowbitQStore(d)
    (d / "extras.f32").symlink_to(GOLD / "toy-int2" / "extras.f32")
    with pytest.raises(RuntimeError, match="not a symlink"):
        lb.DeviceLowbitQStore(d)


@pytest.mark.parametrize("edit,match", [
    (lambda m: m["blocks"]["B"].update(w_off=10**6), "exceeds weights"),
    (lambda m: m["blocks"]["B"].update(s_off=10**6), "exceeds scales"),
    (lambda m: m["blocks"]["B"].update(s_off=2), "exceeds scales"),
    (lambda m: m["blocks"]["A"].update(row_bytes=7), "geometry"),
    (lambda m: m["blocks"]["A"].update(n_groups=1), "geometry"),
    (lambda m: m["blocks"]["norm"].update(e_off=4), "exceeds extras"),
    (lambda m: m["blocks"]["A"].update(kind="qrow2"), "kind qrow2"),
    (lambda m: m["blocks"].update(C={"alias": "missing"}), "no block"),
    (lambda m: m["blocks"].update(C={"alias": "D"}, D={"alias": "C"}), "cyclic"),
])
def test_block_table_is_checked_at_open(tmp_path, edit, match):
    d = _copy(tmp_path, 3)
    _edit(d, edit)
    with pytest.raises((RuntimeError, KeyError), match=match):
        _lb().DeviceLowbitQStore(d)
