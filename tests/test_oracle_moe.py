"""Pins the MoE oracle (CPU) against the reference's own KATs and closed forms."""

from __future__ import annotations

import numpy as np
import torch

from oracle import moe as om
from oracle import qrow as oq


def test_reference_kat_grouped_route_tensors():
    # reference tests/test_olmoe_cuda.py:73-91
    indices = np.array([[3, 1], [1, 2], [3, 2]], dtype=np.int64)
    weights = np.array([[0.7, 0.3], [0.6, 0.4], [0.8, 0.2]], dtype=np.float32)
    token_ids, coef, starts, counts, inverse = om.route_stable(indices, weights, 5)
    assert counts.tolist() == [0, 2, 2, 2, 0]
    assert starts.tolist() == [0, 0, 2, 4, 6]
    assert token_ids.tolist() == [0, 1, 1, 2, 0, 2]
    np.testing.assert_array_equal(coef, np.array([0.3, 0.6, 0.4, 0.2, 0.7, 0.8], np.float32))


def test_reference_kat_inverse_bijection():
    # reference tests/test_olmoe_cuda.py:94-112
    indices = np.array([[3, 1], [1, 2], [3, 2]], dtype=np.int64)
    weights = np.array([[0.7, 0.3], [0.6, 0.4], [0.8, 0.2]], dtype=np.float32)
    token_ids, coef, starts, counts, inverse = om.route_stable(indices, weights, 5)
    assert sorted(inverse.tolist()) == list(range(indices.size))
    for original, dest in enumerate(inverse.tolist()):
        token, rank = divmod(original, indices.shape[1])
        expert = int(indices[token, rank])
        assert token_ids[dest] == token
        assert starts[expert] <= dest < starts[expert] + counts[expert]
        assert coef[dest] == weights[token, rank]


def test_reference_kat_compact_route():
    # reference tests/test_qwen3_moe_cuda.py:1140-1153
    top = np.array([[7, 2], [9, 7]])
    sel = np.array([2, 7, 9])
    compact = np.searchsorted(sel, top)
    token_ids, coef, starts, counts, _ = om.route_stable(compact, np.array([[0.7, 0.3], [0.6, 0.4]], np.float32), 3)
    assert counts.tolist() == [1, 2, 1] and starts.tolist() == [0, 1, 3]
    assert sorted(token_ids.tolist()) == [0, 0, 1, 1]


def test_reference_kat_stable_reduce_equals_index_add_and_is_order_invariant():
    # reference tests/test_qwen3_moe_cuda.py:1155-1241
    top = np.array([[2, 0], [1, 2]])
    w = np.array([[0.7, 0.3], [0.6, 0.4]], np.float32)
    token_ids, coef, starts, counts, inverse = om.route_stable(top, w, 3)
    eo = np.array([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0], [7.0, 8.0]], np.float32)
    expected = torch.zeros((2, 2), dtype=torch.float32)
    expected.index_add_(0, torch.from_numpy(token_ids), torch.from_numpy(eo * coef[:, None]))
    got = om.stable_route_reduce(eo, coef, inverse, 2, 2)
    np.testing.assert_allclose(got, expected.numpy(), rtol=1e-6, atol=0)
    # reverse the two rows of expert group 2, carrying the inverse along
    perm = np.array([0, 1, 3, 2])
    old_to_new = np.empty_like(perm)
    old_to_new[perm] = np.arange(4)
    again = om.stable_route_reduce(eo[perm], coef[perm], old_to_new[inverse], 2, 2)
    assert np.array_equal(again, got)


def test_stable_route_is_a_stable_sort_on_random_routes():
    rng = np.random.default_rng(0)
    top = np.stack([rng.permutation(16)[:4] for _ in range(50)])
    w = rng.random(top.shape).astype(np.float32)
    token_ids, coef, starts, counts, inverse = om.route_stable(top, w, 16)
    flat = top.reshape(-1)
    # queue rows of one expert keep ascending original assignment order
    for e in range(16):
        rows = np.nonzero(flat == e)[0]
        assert inverse[rows].tolist() == list(range(starts[e], starts[e] + counts[e]))


def test_router_matches_torch_library_routines():
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((64, 128)).astype(np.float32)
    w, idx = om.router(logits, 8)
    p = torch.softmax(torch.from_numpy(logits), dim=-1)
    tw, ti = p.topk(8, dim=-1)
    tw = (tw / tw.sum(-1, keepdim=True)).to(torch.bfloat16).float().numpy()
    assert np.array_equal(idx, ti.numpy())
    np.testing.assert_allclose(w, tw, rtol=1e-2, atol=1e-3)  # bf16 rounding of ulp-level differences


def test_grouped_int8_mm_brute_force_and_slots():
    rng = np.random.default_rng(2)
    E, N, K = 3, 8, 64
    w = rng.integers(-127, 128, size=(E, N, K), dtype=np.int8)
    ws = rng.uniform(0.5, 1.5, size=(E, N)).astype(np.float32) / 127
    counts = np.array([2, 0, 3], np.int32)
    starts = np.array([0, 2, 2], np.int32)
    a = rng.integers(-127, 128, size=(5, K), dtype=np.int8)
    asc = rng.uniform(0.1, 1.0, size=5).astype(np.float32)
    out = om.grouped_int8_mm(a, asc, w, ws, starts, counts, out_bf16=False)
    for g, (s0, c) in enumerate(zip(starts, counts)):
        for m in range(c):
            for n in range(N):
                acc = int(np.dot(a[s0 + m].astype(np.int64), w[g, n].astype(np.int64)))
                assert out[s0 + m, n] == np.float32(np.float32(np.float32(acc) * asc[s0 + m]) * ws[g, n])
    # slot indirection == compact weights
    slots = np.array([2, 0, 1])
    w_phys = w[[1, 2, 0]]
    ws_phys = ws[[1, 2, 0]]
    assert np.array_equal(
        om.grouped_int8_mm(a, asc, w_phys, ws_phys, starts, counts, slots=slots, out_bf16=False), out
    )


def test_moe_forward_close_to_dense_float_reference():
    rng = np.random.default_rng(3)
    T, E, k, H, I = 16, 8, 2, 128, 64
    logits = rng.standard_normal((T, E)).astype(np.float32)
    w, idx = om.router(logits, k)
    gu = rng.integers(-127, 128, size=(E, 2 * I, H), dtype=np.int8)
    gus = (rng.uniform(0.5, 1.5, size=(E, 2 * I)) / 127 / np.sqrt(H)).astype(np.float32)
    dn = rng.integers(-127, 128, size=(E, H, I), dtype=np.int8)
    dns = (rng.uniform(0.5, 1.5, size=(E, H)) / 127 / np.sqrt(I)).astype(np.float32)
    x = oq.round_bf16(rng.standard_normal((T, H)).astype(np.float32))
    got = om.moe_forward(x, idx, w, gu, gus, dn, dns)
    ref = om.moe_dense_reference(x, idx, w, gu, gus, dn, dns)
    # per-token int8 quantisation of both GEMMs' activations plus bf16 boundaries: measured
    # 1.5% on this case
    assert oq.rel_l2(got, ref) < 0.025
    # the W8A8 flow is closer to the bf16 restatement of the reference's eager math than to
    # a version of it with wrong routing weights (a planted transposition of the ranks)
    b16 = om.moe_streamed_reference(x, idx, w, gu, gus, dn, dns)
    bad = om.moe_streamed_reference(x, idx, w[:, ::-1], gu, gus, dn, dns)
    assert oq.rel_l2(got, b16) < 0.025 < oq.rel_l2(got, bad)


def _golden_forward():
    import hashlib
    import json
    from pathlib import Path

    gold = Path(__file__).resolve().parent / "golden"
    manifest = json.loads((gold / "golden_manifest.json").read_text())
    path = gold / "moe_forward.npz"
    assert hashlib.sha256(path.read_bytes()).hexdigest() == manifest["moe_forward.npz"]
    return np.load(path, allow_pickle=False)


def test_dense_reference_against_streamed_forward_golden():
    """moe_dense_reference against the reference's own streamed_moe_forward (fp32 run): the
    residual after the MoE layer, h0 + moe, within fp32 summation-order noise."""
    g = _golden_forward()
    moe = om.moe_dense_reference(g["f32_y"], g["f32_top_idx"], g["f32_top_w"], g["gu_q"], g["gu_s"], g["dn_q"], g["dn_s"])
    h1 = (g["f32_h0"].astype(np.float64) + moe).astype(np.float32)
    assert oq.rel_l2(h1, g["f32_h1"]) < 1e-6
    f32 = om.moe_streamed_reference(g["f32_y"], g["f32_top_idx"], g["f32_top_w"], g["gu_q"], g["gu_s"],
                                    g["dn_q"], g["dn_s"], dtype="fp32")
    assert oq.rel_l2((g["f32_h0"] + f32).astype(np.float32), g["f32_h1"]) < 1e-6
    # a dropped expert (the routing weight of rank 2 set to zero) is far outside that bound
    w = g["f32_top_w"].copy()
    w[:, 2] = 0
    bad = om.moe_dense_reference(g["f32_y"], g["f32_top_idx"], w, g["gu_q"], g["gu_s"], g["dn_q"], g["dn_s"])
    assert oq.rel_l2((g["f32_h0"] + bad).astype(np.float32), g["f32_h1"]) > 1e-3
    # the router restatement picks the reference's experts from the same normalised input
    _, idx = om.router(g["f32_y"] @ g["router"].T, 3, bf16=False)
    assert np.array_equal(np.sort(idx, -1), np.sort(g["f32_top_idx"], -1))


def test_streamed_reference_bf16_reproduces_golden():
    """The bf16 restatement gives the reference's bf16 residual bit for bit; dropping one bf16
    boundary (the rounding of silu(g) * u) no longer does."""
    g = _golden_forward()
    args = (g["bf16_y"], g["bf16_top_idx"], g["bf16_top_w"], g["gu_q"], g["gu_s"], g["dn_q"], g["dn_s"])
    h1 = oq.round_bf16(g["bf16_h0"] + om.moe_streamed_reference(*args))
    assert np.mean(h1 == g["bf16_h1"]) >= 0.999 and oq.rel_l2(h1, g["bf16_h1"]) < 1e-3
    bad = oq.round_bf16(g["bf16_h0"] + om.moe_streamed_reference(*args, round_act=False))
    assert np.mean(bad == g["bf16_h1"]) < 0.99


def _expert_order_accumulate(ye, top_idx, top_w, inverse):
    """moe[tok] += bf16(w_e * ye) in ascending expert order, each step rounded to bf16: the
    accumulation of streamed_moe_forward (moe_safetensors.py:603-627)."""
    T, k = top_idx.shape
    out = np.zeros((T, ye.shape[1]), dtype=np.float32)
    w_all = oq.round_bf16(np.asarray(top_w, dtype=np.float32))
    for e in np.unique(top_idx):
        for t in range(T):
            ranks = np.nonzero(top_idx[t] == e)[0]
            if ranks.size:
                r = int(ranks[0])
                contrib = oq.round_bf16(w_all[t, r] * ye[inverse[t * k + r]])
                out[t] = oq.round_bf16(out[t] + contrib)
    return out


def test_grouped_w8a16_reproduces_streamed_forward_golden():
    """The weight-only grouped GEMMs over the stable queue, accumulated in the reference's
    expert order, give the reference's bf16 residual (streamed_moe_forward on the same
    bf16(code * scale) weights) bit for bit; swapping the gate and up halves does not."""
    g = _golden_forward()
    idx, w = g["bf16_top_idx"], g["bf16_top_w"]
    gu, gus, dn, dns = g["gu_q"], g["gu_s"], g["dn_q"], g["dn_s"]
    token_ids, coef, starts, counts, inverse = om.route_stable(idx, w, gu.shape[0])
    rows = oq.round_bf16(g["bf16_y"])[token_ids]

    def layer(gate_up):
        act = om.grouped_w8a16_mm(rows, gate_up, gus, starts, counts, swiglu=True)
        ye = om.grouped_w8a16_mm(act, dn, dns, starts, counts)
        return oq.round_bf16(g["bf16_h0"] + _expert_order_accumulate(ye, idx, w, inverse))

    h1 = layer(gu)
    assert np.mean(h1 == g["bf16_h1"]) >= 0.999 and oq.rel_l2(h1, g["bf16_h1"]) < 1e-3
    I = gu.shape[1] // 2
    swapped = np.concatenate([gu[:, I:], gu[:, :I]], axis=1)
    assert np.mean(layer(swapped) == g["bf16_h1"]) < 0.9


def test_grouped_w8a16_slots_and_flow_against_dense_reference():
    rng = np.random.default_rng(5)
    E, N, K = 3, 8, 64
    w = rng.integers(-127, 128, size=(E, N, K), dtype=np.int8)
    ws = rng.uniform(0.5, 1.5, size=(E, N)).astype(np.float32) / 127
    counts = np.array([2, 0, 3], np.int32)
    starts = np.array([0, 2, 2], np.int32)
    rows = oq.round_bf16(rng.standard_normal((5, K)).astype(np.float32))
    out = om.grouped_w8a16_mm(rows, w, ws, starts, counts, out_bf16=False)
    slots = np.array([2, 0, 1])
    assert np.array_equal(
        om.grouped_w8a16_mm(rows, w[[1, 2, 0]], ws[[1, 2, 0]], starts, counts, slots=slots, out_bf16=False), out
    )
    # whole layer: no activation quantization, so within bf16-boundary noise of the float
    # formulation (the W8A8 flow is held to 2.5% on the same kind of case)
    T, E, k, H, I = 16, 8, 2, 128, 64
    logits = rng.standard_normal((T, E)).astype(np.float32)
    wt, idx = om.router(logits, k)
    gu = rng.integers(-127, 128, size=(E, 2 * I, H), dtype=np.int8)
    gus = (rng.uniform(0.5, 1.5, size=(E, 2 * I)) / 127 / np.sqrt(H)).astype(np.float32)
    dn = rng.integers(-127, 128, size=(E, H, I), dtype=np.int8)
    dns = (rng.uniform(0.5, 1.5, size=(E, H)) / 127 / np.sqrt(I)).astype(np.float32)
    x = oq.round_bf16(rng.standard_normal((T, H)).astype(np.float32))
    got = om.moe_forward_w8a16(x, idx, wt, gu, gus, dn, dns)
    ref = om.moe_dense_reference(x, idx, wt, gu, gus, dn, dns)
    assert oq.rel_l2(got, ref) < 0.01
    assert oq.rel_l2(got, ref) < oq.rel_l2(om.moe_forward(x, idx, wt, gu, gus, dn, dns), ref)
