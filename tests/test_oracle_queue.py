"""Expert-queue oracle against the reference's KATs (tests/test_expert_queue.py:16-139) and
the golden vectors written from the reference's CPU functions (tests/golden/queue.npz)."""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np

from oracle import expert_queue as oe
from oracle.qrow import round_bf16

GOLD = Path(__file__).resolve().parent / "golden"
FIELDS = ("token_ids", "expert_ids", "route_slots", "coefficients", "epochs", "deadlines", "starts", "counts")


def _gold():
    manifest = json.loads((GOLD / "golden_manifest.json").read_text())
    path = GOLD / "queue.npz"
    assert hashlib.sha256(path.read_bytes()).hexdigest() == manifest["queue.npz"]
    return np.load(path, allow_pickle=False)


def test_reference_kats():
    p = oe.build_dense([[2, 0], [2, 1], [3, 2]], [[0.6, 0.3], [0.5, 0.4], [0.2, 0.5]], 4, [7, 8, 9], [30, 10, 20])
    assert p["counts"].tolist() == [1, 1, 3, 1] and p["starts"].tolist() == [0, 1, 2, 5]
    assert p["token_ids"].tolist() == [0, 1, 0, 1, 2, 2]
    assert p["route_slots"].tolist() == [1, 1, 0, 0, 1, 0]
    assert p["epochs"].tolist() == [7, 8, 7, 8, 9, 9]
    red, valid = oe.scatter(p, np.ones((6, 2), np.float32), [7, 99, 9], 3)
    assert int(valid.sum()) == 4
    np.testing.assert_allclose(red[:, 0], [0.9, 0.0, 0.7], rtol=1e-6)
    f = oe.build_flat([0, 1, 2, 2], [2, 1, 3, 0], [0, 0, 0, 1], [0.7, 0.9, 0.8, 0.2], 4, [5, 6, 7], [50, 60, 70])
    assert f["counts"].tolist() == [1, 1, 1, 1] and f["starts"].tolist() == [0, 1, 2, 3]
    assert f["token_ids"].tolist() == [2, 1, 0, 2] and f["route_slots"].tolist() == [1, 0, 0, 0]
    red, valid = oe.scatter(f, np.ones((4, 2), np.float32), [5, 6, 7], 3)
    assert valid.all()
    np.testing.assert_allclose(red[:, 1], [0.7, 0.9, 1.0], rtol=1e-6)


def test_golden_dense_and_flat_bit_exact():
    g = _gold()
    for tag, wt in (("f32", g["d_w"]), ("bf16", round_bf16(g["d_w"]))):
        p = oe.build_dense(g["d_top"], wt, 24, g["d_ep"], g["d_dl"])
        for f in FIELDS:
            assert np.array_equal(p[f], g[f"d_{tag}_{f}"]), (tag, f)
        red, valid = oe.scatter(p, g[f"d_{tag}_out"], g[f"d_{tag}_active"], 40)
        assert np.array_equal(valid, g[f"d_{tag}_valid"])
        assert np.array_equal(red.view(np.uint32), g[f"d_{tag}_reduced"].view(np.uint32))
    p = oe.build_flat(g["f_tok"], g["f_exp"], g["f_slot"], g["f_cf"], 24, g["d_ep"], g["d_dl"])
    for f in FIELDS:
        assert np.array_equal(p[f], g[f"f_{f}"]), f
    red, valid = oe.scatter(p, g["f_out"], g["f_active"], 40)
    assert np.array_equal(valid, g["f_valid"])
    assert np.array_equal(red.view(np.uint32), g["f_reduced"].view(np.uint32))


def test_scatter_order_matters():
    """A planted reversal of the packet order changes the reduced bits on the golden case, so
    the bit-exact check above pins the order, not just the set of packets."""
    g = _gold()
    p = oe.build_flat(g["f_tok"], g["f_exp"], g["f_slot"], g["f_cf"], 24, g["d_ep"], g["d_dl"])
    rev = {k: (v[::-1].copy() if v.shape == p["token_ids"].shape else v) for k, v in p.items()}
    red, _ = oe.scatter(rev, g["f_out"][::-1].copy(), g["f_active"], 40)
    assert not np.array_equal(red.view(np.uint32), g["f_reduced"].view(np.uint32))
