"""Expert-queue kernels (qs_expert_queue_build / qs_expert_queue_scatter) against the
reference's KATs and the golden vectors written from its CPU functions, bit for bit."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import expert_queue as oe

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"
FIELDS = ("token_ids", "expert_ids", "route_slots", "coefficients", "epochs", "deadlines", "starts", "counts")


def _q():
    from mrun_pub_amd import expert_queue

    return expert_queue


def _t(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def _check_plan(plan, ref, prefix=""):
    for f in FIELDS:
        got = getattr(plan, f).cpu().numpy()
        assert np.array_equal(got, ref[f"{prefix}{f}"]), f


def test_reference_kats(dev):
    q = _q()
    plan = q.build_expert_queue(
        _t(np.array([[2, 0], [2, 1], [3, 2]]), dev), _t(np.array([[0.6, 0.3], [0.5, 0.4], [0.2, 0.5]], np.float32), dev),
        num_experts=4, epochs=_t(np.array([7, 8, 9]), dev), deadlines=_t(np.array([30, 10, 20]), dev))
    assert plan.assignments == 6
    assert plan.counts.tolist() == [1, 1, 3, 1] and plan.starts.tolist() == [0, 1, 2, 5]
    assert plan.token_ids.tolist() == [0, 1, 0, 1, 2, 2] and plan.route_slots.tolist() == [1, 1, 0, 0, 1, 0]
    assert plan.epochs.tolist() == [7, 8, 7, 8, 9, 9]
    reduced, valid = q.scatter_committed(plan, torch.ones((6, 2), device=dev), active_epochs=_t(np.array([7, 99, 9]), dev))
    assert int(valid.sum()) == 4 and valid.dtype == torch.bool
    torch.testing.assert_close(reduced[:, 0].cpu(), torch.tensor([0.9, 0.0, 0.7]))
    flat = q.build_expert_queue_flat(
        _t(np.array([0, 1, 2, 2]), dev), _t(np.array([2, 1, 3, 0]), dev), _t(np.array([0, 0, 0, 1]), dev),
        _t(np.array([0.7, 0.9, 0.8, 0.2], np.float32), dev), num_rows=3, num_experts=4, top_k=2,
        epochs=_t(np.array([5, 6, 7]), dev), deadlines=_t(np.array([50, 60, 70]), dev))
    assert flat.counts.tolist() == [1, 1, 1, 1] and flat.token_ids.tolist() == [2, 1, 0, 2]
    assert flat.route_slots.tolist() == [1, 0, 0, 0] and flat.counts.dtype == torch.int32
    reduced, valid = q.scatter_committed(flat, torch.ones((4, 2), device=dev), active_epochs=_t(np.array([5, 6, 7]), dev))
    assert bool(valid.all())
    torch.testing.assert_close(reduced[:, 1].cpu(), torch.tensor([0.7, 0.9, 1.0]))


def test_validation_errors(dev):
    q = _q()
    common = dict(num_rows=1, num_experts=4, top_k=2, epochs=_t(np.array([1]), dev), deadlines=_t(np.array([2]), dev))
    with pytest.raises(ValueError, match="same route slot twice"):
        q.build_expert_queue_flat(_t(np.array([0, 0]), dev), _t(np.array([1, 2]), dev), _t(np.array([0, 0]), dev),
                                  _t(np.array([0.6, 0.4], np.float32), dev), **common)
    with pytest.raises(ValueError, match="same expert twice"):
        q.build_expert_queue_flat(_t(np.array([0, 0]), dev), _t(np.array([1, 1]), dev), _t(np.array([0, 1]), dev),
                                  _t(np.array([0.6, 0.4], np.float32), dev), **common)
    dense = dict(top_weights=_t(np.array([[0.5, 0.5]], np.float32), dev), num_experts=4,
                 epochs=_t(np.array([1]), dev), deadlines=_t(np.array([10]), dev))
    with pytest.raises(ValueError, match="same expert twice"):
        q.build_expert_queue(_t(np.array([[2, 2]]), dev), **dense)
    with pytest.raises(ValueError, match="out-of-range"):
        q.build_expert_queue(_t(np.array([[2, 4]]), dev), **dense)


@pytest.mark.parametrize("tag", ["f32", "bf16"])
def test_dense_golden(dev, tag):
    q = _q()
    g = np.load(GOLD / "queue.npz", allow_pickle=False)
    w = _t(g["d_w"], dev) if tag == "f32" else _t(g["d_w"], dev, torch.bfloat16)
    args = (_t(g["d_top"], dev), w)
    kw = dict(num_experts=24, epochs=_t(g["d_ep"], dev), deadlines=_t(g["d_dl"], dev))
    plan = q.build_expert_queue(*args, **kw)
    _check_plan(plan, g, f"d_{tag}_")
    dplan = q.build_expert_queue_device(*args, **kw)  # stable too: the same plan, int32 ranges
    for f in FIELDS:
        assert torch.equal(getattr(dplan, f).to(getattr(plan, f).dtype), getattr(plan, f)), f
    assert dplan.counts.dtype == torch.int32
    out = _t(g[f"d_{tag}_out"], dev)
    act = _t(g[f"d_{tag}_active"], dev)
    for fn in (q.scatter_committed, q.scatter_committed_device):
        red, valid = fn(plan, out, active_epochs=act)
        assert np.array_equal(valid.cpu().numpy(), g[f"d_{tag}_valid"])
        assert np.array_equal(red.cpu().numpy().view(np.uint32), g[f"d_{tag}_reduced"].view(np.uint32))


def test_flat_golden(dev):
    q = _q()
    g = np.load(GOLD / "queue.npz", allow_pickle=False)
    plan = q.build_expert_queue_flat(_t(g["f_tok"], dev), _t(g["f_exp"], dev), _t(g["f_slot"], dev), _t(g["f_cf"], dev),
                                     num_rows=40, num_experts=24, top_k=6, epochs=_t(g["d_ep"], dev),
                                     deadlines=_t(g["d_dl"], dev))
    _check_plan(plan, g, "f_")
    red, valid = q.scatter_committed(plan, _t(g["f_out"], dev), active_epochs=_t(g["f_active"], dev))
    assert np.array_equal(valid.cpu().numpy(), g["f_valid"])
    assert np.array_equal(red.cpu().numpy().view(np.uint32), g["f_reduced"].view(np.uint32))


@pytest.mark.parametrize("rows,E,k,H", [(512, 128, 8, 2048), (64, 128, 8, 2048), (3000, 64, 4, 64), (1, 8, 8, 5)])
def test_config_sizes_against_oracle(dev, rows, E, k, H):
    """Config-4 shapes (128 experts, top-8, H 2048) and larger queues, bf16 expert outputs."""
    q = _q()
    rng = np.random.default_rng(rows + E)
    top = np.stack([rng.permutation(E)[:k] for _ in range(rows)]).astype(np.int64)
    w = rng.random((rows, k)).astype(np.float32)
    ep = rng.integers(0, 3, size=rows)
    dl = rng.integers(0, 1000, size=rows)
    plan = q.build_expert_queue_device(_t(top, dev), _t(w, dev), num_experts=E, epochs=_t(ep, dev),
                                       deadlines=_t(dl, dev))
    ref = oe.build_dense(top, w, E, ep, dl)
    for f in FIELDS:
        assert np.array_equal(getattr(plan, f).cpu().numpy(), ref[f].astype(getattr(plan, f).cpu().numpy().dtype)), f
    out = torch.randn(rows * k, H, device=dev).to(torch.bfloat16)
    act = np.where(rng.random(rows) < 0.8, ep, ep + 7)
    red, valid = q.scatter_committed_device(plan, out, active_epochs=_t(act, dev))
    r_red, r_valid = oe.scatter(ref, out.float().cpu().numpy(), act, rows)
    assert np.array_equal(valid.cpu().numpy(), r_valid)
    assert np.array_equal(red.cpu().numpy().view(np.uint32), r_red.view(np.uint32))


def test_device_builder_drops_out_of_range_experts(dev):
    """The unvalidated builder never writes out of bounds: a bad expert id leaves the queue,
    and the freed tail rows carry sentinels that assert_valid reports."""
    q = _q()
    top = np.array([[0, 3], [9, 1]], dtype=np.int64)
    plan = q.build_expert_queue_device(_t(top, dev), torch.ones(2, 2, device=dev), num_experts=4,
                                       epochs=_t(np.array([1, 2]), dev), deadlines=_t(np.array([3, 4]), dev))
    assert plan.counts.tolist() == [1, 1, 0, 1]
    assert plan.token_ids.tolist()[:3] == [0, 1, 0] and plan.expert_ids.tolist()[3] == -1
    with pytest.raises(AssertionError):
        plan.assert_valid()


def test_scatter_matches_rows_by_token_alone(dev):
    """An unvalidated flat plan may carry two packets with the same (token, route slot) or a
    slot outside [0, top_k): the reference's index_add_ counts every packet whose epoch
    matches, by token alone (expert_queue.py:487-514), and so does the device scatter,
    with the same bits on every call."""
    q = _q()
    tok = np.array([0, 1, 0, 2, 0, 1], np.int64)
    exp = np.array([3, 1, 2, 0, 1, 2], np.int64)
    slot = np.array([1, 0, 1, 9, 0, -4], np.int64)  # (0, 1) twice; slots 9 and -4 out of range
    cf = np.array([0.5, 0.25, 0.75, 1.5, 2.0, 3.0], np.float32)
    ep = np.array([4, 5, 6], np.int64)
    plan = q.build_expert_queue_flat(_t(tok, dev), _t(exp, dev), _t(slot, dev), _t(cf, dev), num_rows=3,
                                     num_experts=4, top_k=2, epochs=_t(ep, dev), deadlines=_t(ep, dev),
                                     validate=False)
    rng = np.random.default_rng(8)
    out = rng.standard_normal((6, 33)).astype(np.float32)
    act = np.array([4, 5, 6], np.int64)
    ref = {f: getattr(plan, f).cpu().numpy() for f in FIELDS}
    r_red, r_valid = oe.scatter(ref, out, act, 3)
    assert r_valid.all()
    first = None
    for _ in range(3):
        red, valid = q.scatter_committed(plan, _t(out, dev), active_epochs=_t(act, dev))
        assert np.array_equal(valid.cpu().numpy(), r_valid)
        assert np.array_equal(red.cpu().numpy().view(np.uint32), r_red.view(np.uint32))
        first = red if first is None else first
        assert torch.equal(red, first)


def test_scatter_more_rows_than_one_grid_dimension(dev):
    """A prefill queue of 70,000 token rows (more than 65,535, the limit of one grid
    dimension): every row reduced, against the oracle."""
    q = _q()
    rows, E, k, H = 70000, 16, 2, 8
    rng = np.random.default_rng(70)
    top = np.stack([rng.permutation(E)[:k] for _ in range(rows)]).astype(np.int64)
    w = rng.random((rows, k)).astype(np.float32)
    ep = rng.integers(0, 3, size=rows)
    plan = q.build_expert_queue_device(_t(top, dev), _t(w, dev), num_experts=E, epochs=_t(ep, dev),
                                       deadlines=_t(ep, dev))
    out = rng.standard_normal((rows * k, H)).astype(np.float32)
    act = np.where(rng.random(rows) < 0.9, ep, ep + 1)
    red, valid = q.scatter_committed_device(plan, _t(out, dev), active_epochs=_t(act, dev))
    ref = {f: getattr(plan, f).cpu().numpy() for f in FIELDS}
    r_red, r_valid = oe.scatter(ref, out, act, rows)
    assert np.array_equal(valid.cpu().numpy(), r_valid)
    assert np.array_equal(red.cpu().numpy().view(np.uint32), r_red.view(np.uint32))
