"""QStore v3 int8 format: writer -> validated memory-mapped reader (CPU)."""

from __future__ import annotations

import json

import numpy as np
import pytest

from mrun_pub_amd.store import QStoreReader, write_qstore


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


def _corrupt(tmp_path, edit):
    write_qstore(tmp_path, _blocks())
    man = json.loads((tmp_path / "manifest.json").read_text())
    edit(man)
    (tmp_path / "manifest.json").write_text(json.dumps(man))


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
    ],
)
def test_layout_violations_are_rejected(tmp_path, edit):
    # reference _validate_int8_layout, src/mrun/engine/kernels/qstore.py:124-219
    _corrupt(tmp_path, edit)
    with pytest.raises(RuntimeError):
        QStoreReader(tmp_path)


def test_truncated_file_is_rejected(tmp_path):
    write_qstore(tmp_path, _blocks())
    data = (tmp_path / "weights.i8").read_bytes()
    (tmp_path / "weights.i8").write_bytes(data[:-1])
    with pytest.raises(RuntimeError, match="exceeds|cover"):
        QStoreReader(tmp_path)
