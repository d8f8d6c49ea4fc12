"""GPU parity of the routed-MoE kernels against the CPU oracle (through the C ABI)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle import qrow as oq

pytestmark = pytest.mark.gpu


def _moe():
    from mrun_pub_amd import moe

    return moe


def _t(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def test_route_reference_kat(dev):
    # reference tests/test_olmoe_cuda.py:73-112
    idx = torch.tensor([[3, 1], [1, 2], [3, 2]], dtype=torch.long, device=dev)
    w = torch.tensor([[0.7, 0.3], [0.6, 0.4], [0.8, 0.2]], dtype=torch.float32, device=dev)
    tok, coef, starts, counts, inv, _ = _moe().grouped_route_tensors_with_inverse(idx, w, num_experts=5)
    assert counts.tolist() == [0, 2, 2, 2, 0]
    assert starts.tolist() == [0, 0, 2, 4, 6]
    assert tok.tolist() == [0, 1, 1, 2, 0, 2]
    assert np.array_equal(coef.cpu().numpy(), np.array([0.3, 0.6, 0.4, 0.2, 0.7, 0.8], np.float32))
    assert sorted(inv.tolist()) == list(range(6))


# A * E <= 2^22: one workgroup per expert; (16384, 64, 4) and (9000, 512, 1): one workgroup
@pytest.mark.parametrize("T,E,k", [(64, 128, 8), (512, 128, 8), (7, 5, 3), (1, 128, 8), (3000, 64, 4),
                                   (200, 512, 8), (100, 300, 6), (16384, 64, 4), (9000, 512, 1)])
@pytest.mark.parametrize("wdt", [torch.float32, torch.bfloat16])
def test_route_equals_stable_argsort(dev, T, E, k, wdt):
    rng = np.random.default_rng(T + E + k)
    top = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int64)
    w = rng.random((T, k)).astype(np.float32)
    tw = torch.from_numpy(w).to(wdt)
    tok, coef, starts, counts, inv, _ = _moe().grouped_route_tensors_with_inverse(_t(top, dev), tw.to(dev), num_experts=E)
    r_tok, r_coef, r_starts, r_counts, r_inv = om.route_stable(top, tw.float().numpy(), E)
    assert np.array_equal(tok.cpu().numpy(), r_tok)
    assert np.array_equal(coef.float().cpu().numpy(), r_coef)
    assert np.array_equal(starts.cpu().numpy(), r_starts)
    assert np.array_equal(counts.cpu().numpy(), r_counts)
    assert np.array_equal(inv.cpu().numpy(), r_inv)
    assert coef.dtype == wdt


def test_route_drops_out_of_range_experts(dev):
    """Device indices outside [0, E) leave the queue (no host sync): the valid assignments
    keep the stable order, inverse is -1 for the dropped ones, the spare queue rows hold
    token 0 / coefficient 0, and the reduce adds nothing for a dropped rank."""
    E, k = 6, 3
    top = np.array([[0, 5, 2], [-1, 1, 6], [2, 3, 99]], dtype=np.int64)
    w = np.arange(1, 10, dtype=np.float32).reshape(3, 3) / 10
    tok, coef, starts, counts, inv, _ = _moe().grouped_route_tensors_with_inverse(
        _t(top, dev), _t(w, dev), num_experts=E)
    keep = (top >= 0) & (top < E)
    r_tok, r_coef, r_starts, r_counts, r_inv = om.route_stable(np.where(keep, top, 0)[keep][None, :], w[keep][None, :], E)
    n = int(keep.sum())
    assert counts.cpu().numpy().tolist() == np.bincount(top[keep], minlength=E).tolist()
    assert starts.cpu().numpy().tolist() == r_starts.tolist()
    flat_tok = (np.arange(9) // 3)[keep.reshape(-1)]
    assert tok.cpu().numpy()[:n].tolist() == flat_tok[np.argsort(top[keep], kind="stable")].tolist()
    assert tok.cpu().numpy()[n:].tolist() == [0] * (9 - n)
    assert coef.cpu().numpy()[n:].tolist() == [0.0] * (9 - n)
    inv_h = inv.cpu().numpy()
    assert (inv_h[~keep.reshape(-1)] == -1).all() and sorted(inv_h[keep.reshape(-1)].tolist()) == list(range(n))
    H = 8
    eo = np.random.default_rng(0).standard_normal((9, H)).astype(np.float32)
    red = _moe().stable_route_reduce(_t(eo, dev), coef, tok, counts, _t(top, dev), torch.arange(E, device=dev),
                                     inverse_assignments=inv)
    ref = np.zeros((3, H), np.float32)
    for t in range(3):
        acc = None
        for r in range(3):
            q = inv_h[t * 3 + r]
            c = np.float32(0) * eo[0] if q < 0 else (eo[q] * coef.cpu().numpy()[q]).astype(np.float32)
            acc = c if acc is None else (acc + c).astype(np.float32)
        ref[t] = acc
    assert np.array_equal(red.float().cpu().numpy(), ref)


@pytest.mark.parametrize("T,E,k", [(300, 64, 4), (16384, 64, 4)])  # per-expert / one workgroup
def test_route_drops_out_of_range_both_kernels(dev, T, E, k):
    rng = np.random.default_rng(T)
    top = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int64)
    bad = rng.random((T, k)) < 0.01
    # int64 ids are range-checked before any narrowing: 2**32 + 3 is not expert 3
    top[bad] = rng.choice([-3, -1, E, E + 7, 2**32 + 3, -(2**32) + 1], size=int(bad.sum()))
    w = rng.random((T, k)).astype(np.float32)
    tok, coef, starts, counts, inv, _ = _moe().grouped_route_tensors_with_inverse(_t(top, dev), _t(w, dev), num_experts=E)
    keep = ~bad
    flat = top.reshape(-1)
    fk = keep.reshape(-1)
    order = np.argsort(np.where(fk, flat, E), kind="stable")[: int(fk.sum())]
    n = int(fk.sum())
    assert counts.cpu().numpy().tolist() == np.bincount(flat[fk], minlength=E).tolist()
    assert tok.cpu().numpy()[:n].tolist() == (order // k).tolist()
    assert np.array_equal(coef.cpu().numpy()[:n], w.reshape(-1)[order])
    assert not tok.cpu().numpy()[n:].any() and not coef.cpu().numpy()[n:].any()
    exp_inv = np.full(T * k, -1, np.int64)
    exp_inv[order] = np.arange(n)
    assert np.array_equal(inv.cpu().numpy(), exp_inv)


def test_router_against_oracle(dev):
    rng = np.random.default_rng(4)
    logits = rng.standard_normal((512, 128)).astype(np.float32)
    w, idx = _moe().route_topk(_t(logits, dev), 8)
    rw, ridx = om.router(logits, 8)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert oq.rel_l2(w.float().cpu().numpy(), rw) < 2e-3


# expert counts for each logits-per-lane width (1, 2, 4, 8, 16 per lane), k up to 16
@pytest.mark.parametrize("T,E,k", [(33, 5, 3), (64, 64, 16), (70, 200, 8), (40, 300, 6), (20, 1024, 16), (9, 700, 1)])
@pytest.mark.parametrize("norm", [True, False])
def test_router_widths_fp32(dev, T, E, k, norm):
    rng = np.random.default_rng(E + k)
    logits = (rng.standard_normal((T, E)) * 3).astype(np.float32)
    w, idx = _moe().route_topk(_t(logits, dev), k, norm_topk=norm, out_dtype=torch.float32)
    rw, ridx = om.router(logits, k, norm_topk=norm, bf16=False)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    # expf and numpy's exp may differ in the last place
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=2e-6, atol=0)


def test_stable_reduce_reference_kat(dev):
    # reference tests/test_qwen3_moe_cuda.py:1155-1241 (reconstructed and compiled inverse)
    top = torch.tensor([[2, 0], [1, 2]], dtype=torch.long, device=dev)
    w = torch.tensor([[0.7, 0.3], [0.6, 0.4]], device=dev)
    sel = torch.tensor([0, 1, 2], dtype=torch.long, device=dev)
    tok, coef, starts, counts, inv = _moe()._compact_route_with_inverse(top, w, sel)
    eo = torch.tensor([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0], [7.0, 8.0]], device=dev)
    expected = torch.zeros((2, 2), dtype=torch.float32, device=dev)
    expected.index_add_(0, tok, eo * coef[:, None])
    rec = _moe().stable_route_reduce(eo, coef, tok, counts, top, sel)
    com = _moe().stable_route_reduce(eo, coef, tok, counts, top, sel, inverse_assignments=inv)
    torch.testing.assert_close(rec, expected)
    assert torch.equal(rec, com)


@pytest.mark.parametrize("T,k,H", [(64, 8, 2048), (5, 3, 100)])
def test_stable_reduce_bit_exact(dev, T, k, H):
    rng = np.random.default_rng(T)
    A = T * k
    eo = oq.round_bf16(rng.standard_normal((A, H)).astype(np.float32))
    coef = rng.random(A).astype(np.float32)
    inv = rng.permutation(A).astype(np.int64)
    tok = (np.argsort(inv) // k).astype(np.int64)
    got = _moe().stable_route_reduce(
        _t(eo, dev, torch.bfloat16), _t(coef, dev), _t(tok, dev), torch.tensor([A], dtype=torch.int32, device=dev),
        torch.zeros((T, k), dtype=torch.long, device=dev), torch.zeros(1, dtype=torch.long, device=dev),
        inverse_assignments=_t(inv, dev),
    )
    assert np.array_equal(got.cpu().numpy(), om.stable_route_reduce(eo, coef, inv, T, k))


@pytest.mark.parametrize("T,k,H", [(64, 8, 2048), (5, 3, 100)])  # 8-wide kernel, scalar kernel
def test_stable_reduce_bf16_out_is_cast_of_fp32(dev, T, k, H):
    rng = np.random.default_rng(T + 1)
    A = T * k
    eo = _t(oq.round_bf16(rng.standard_normal((A, H)).astype(np.float32)), dev, torch.bfloat16)
    coef = _t(rng.random(A).astype(np.float32), dev)
    inv = rng.permutation(A).astype(np.int64)
    tok = _t((np.argsort(inv) // k).astype(np.int64), dev)
    args = (eo, coef, tok, torch.tensor([A], dtype=torch.int32, device=dev),
            torch.zeros((T, k), dtype=torch.long, device=dev), torch.zeros(1, dtype=torch.long, device=dev))
    f32 = _moe().stable_route_reduce(*args, inverse_assignments=_t(inv, dev))
    b16 = _moe().stable_route_reduce(*args, inverse_assignments=_t(inv, dev), out_dtype=torch.bfloat16)
    assert b16.dtype == torch.bfloat16
    assert torch.equal(b16, f32.to(torch.bfloat16))


# H = 2048 / 768: one wave per row, row kept in registers; 8192: row read twice;
# 100: scalar kernel (H % 8 != 0)
@pytest.mark.parametrize("H", [2048, 768, 8192, 100])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_quantize_rows_matches_oracle(dev, H, dtype):
    rng = np.random.default_rng(H)
    T, A = 37, 150
    x = rng.standard_normal((T, H)).astype(np.float32) * rng.uniform(0.1, 10, size=(T, 1)).astype(np.float32)
    x[3] = 0.0  # all-zero row: scale 1, codes 0
    x[5, 7] = 40.0  # an outlier sets the scale
    x[6] *= np.float32(1e-37)  # scale below 2^-120: the division path
    x[7] *= np.float32(1e-30)  # denormal elements in a row with a normal scale
    if dtype == torch.bfloat16:
        x = oq.round_bf16(x)
    rows = rng.integers(0, T, size=A).astype(np.int64)
    rows[:6] = [3, 5, 3, 0, 6, 7]
    q, s = _moe().quantize_rows(_t(x, dev, dtype), _t(rows, dev))
    q_r, s_r = om.quantize_rows(x[rows])
    assert np.array_equal(s.cpu().numpy(), s_r)
    assert np.array_equal(q.cpu().numpy(), q_r)
    q2, s2 = _moe().quantize_rows(_t(x, dev, dtype))  # no gather: row a is source row a
    q2_r, s2_r = om.quantize_rows(x)
    assert np.array_equal(s2.cpu().numpy(), s2_r) and np.array_equal(q2.cpu().numpy(), q2_r)


def _layer(rng, E, H, I):
    gu = rng.integers(-127, 128, size=(E, 2 * I, H), dtype=np.int8)
    gus = (rng.uniform(0.5, 1.5, size=(E, 2 * I)) / 127).astype(np.float32)
    dn = rng.integers(-127, 128, size=(E, H, I), dtype=np.int8)
    dns = (rng.uniform(0.5, 1.5, size=(E, H)) / 127).astype(np.float32)
    return gu, gus, dn, dns


@pytest.mark.parametrize("swiglu", [False, True])
# K = H: streamed with 128-byte chunks (256, 4096) or 64-byte chunks (320), K-split (12288)
@pytest.mark.parametrize("H", [256, 320, 4096, 12288])
def test_grouped_gemm_matches_oracle(dev, swiglu, H):
    if swiglu and H > 8192:
        pytest.skip("the SwiGLU kernel takes K <= 8192 (its K splits stop at 8 waves)")
    rng = np.random.default_rng(7)
    E, I, T, k = 16, 128, 40, 4
    gu, gus, dn, dns = _layer(rng, E, H, I)
    top = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int64)
    tok, coef, starts, counts, inv = om.route_stable(top, np.ones((T, k), np.float32), E)
    a = rng.integers(-127, 128, size=(T * k, H), dtype=np.int8)
    asc = rng.uniform(0.01, 0.1, size=T * k).astype(np.float32)
    layer = _moe().Int8ExpertLayer.from_arrays(*(torch.from_numpy(v) for v in (gu, gus, dn, dns)), dev)
    out, tag = _moe().grouped_int8_mm(
        _t(a, dev), _t(asc, dev), layer.gate_up, layer.gate_up_scales, _t(starts, dev), _t(counts, dev), swiglu=swiglu
    )
    ref = om.grouped_int8_mm(a, asc, gu, gus, starts, counts, swiglu=swiglu)
    if swiglu:
        assert oq.rel_l2(out.float().cpu().numpy(), ref) <= 1e-3
    else:
        # int32 accumulators exact + closed-form epilogue: bit-exact bf16
        assert np.array_equal(out.float().cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("swiglu", [False, True])
@pytest.mark.parametrize("max_rows", [0, 16, 400, 4000])  # row tiles of 32, 16, 64, 64 rows
@pytest.mark.parametrize("H", [256, 2048])
def test_grouped_gemm_row_tiles(dev, swiglu, max_rows, H):
    """Skewed routing (expert 0 takes every token): groups longer than one row tile take
    several passes; max_rows only changes the tiling, never the result."""
    rng = np.random.default_rng(11)
    E, I, T, k = 8, 96, 200, 2
    gu, gus, dn, dns = _layer(rng, E, H, I)
    top = np.stack([np.concatenate([[0], 1 + rng.permutation(E - 1)[: k - 1]]) for _ in range(T)]).astype(np.int64)
    tok, coef, starts, counts, inv = om.route_stable(top, np.ones((T, k), np.float32), E)
    assert counts.max() == T
    a = rng.integers(-127, 128, size=(T * k, H), dtype=np.int8)
    asc = rng.uniform(0.01, 0.1, size=T * k).astype(np.float32)
    layer = _moe().Int8ExpertLayer.from_arrays(*(torch.from_numpy(v) for v in (gu, gus, dn, dns)), dev)
    out, _ = _moe().grouped_int8_mm(
        _t(a, dev), _t(asc, dev), layer.gate_up, layer.gate_up_scales, _t(starts, dev), _t(counts, dev),
        max_rows=max_rows, swiglu=swiglu,
    )
    ref = om.grouped_int8_mm(a, asc, gu, gus, starts, counts, swiglu=swiglu)
    if swiglu:
        assert oq.rel_l2(out.float().cpu().numpy(), ref) <= 1e-3
    else:
        assert np.array_equal(out.float().cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_grouped_gemm_slot_indirection(dev):
    rng = np.random.default_rng(8)
    E, H, I, T, k = 8, 128, 64, 16, 2
    gu, gus, dn, dns = _layer(rng, E, H, I)
    top = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int64)
    tok, coef, starts, counts, inv = om.route_stable(top, np.ones((T, k), np.float32), E)
    a = rng.integers(-127, 128, size=(T * k, H), dtype=np.int8)
    asc = rng.uniform(0.01, 0.1, size=T * k).astype(np.float32)
    perm = rng.permutation(E)
    slots = np.argsort(perm).astype(np.int32)  # logical g lives in physical slot slots[g]
    phys = _moe().Int8ExpertLayer.from_arrays(*(torch.from_numpy(v[perm]) for v in (gu, gus, dn, dns)), dev)
    comp = _moe().Int8ExpertLayer.from_arrays(*(torch.from_numpy(v) for v in (gu, gus, dn, dns)), dev)
    o1, _ = _moe().grouped_int8_mm(_t(a[:, :I].copy(), dev), _t(asc, dev), phys.down, phys.down_scales, _t(starts, dev), _t(counts, dev), group_slots=_t(slots, dev))
    o2, _ = _moe().grouped_int8_mm(_t(a[:, :I].copy(), dev), _t(asc, dev), comp.down, comp.down_scales, _t(starts, dev), _t(counts, dev))
    assert torch.equal(o1, o2)


@pytest.mark.parametrize("T", [64, 512])
def test_moe_layer_config4(dev, T):
    """128 experts, top-8, H 2048, I 768, router N(0,1) over T tokens."""
    rng = np.random.default_rng(T)
    E, k, H, I = 128, 8, 2048, 768
    gu, gus, dn, dns = _layer(rng, E, H, I)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    x = oq.round_bf16(rng.standard_normal((T, H)).astype(np.float32))
    layer = _moe().Int8ExpertLayer.from_arrays(*(torch.from_numpy(v) for v in (gu, gus, dn, dns)), dev)
    backend = _moe().Int8ExpertBackend([layer])
    tw, ti = _moe().route_topk(_t(logits, dev), k)
    y = backend.moe(0, _t(x, dev, torch.bfloat16), ti, tw)
    assert y.dtype == torch.bfloat16 and y.shape == (T, H)
    ref = om.moe_forward(x, ti.cpu().numpy(), tw.float().cpu().numpy(), gu, gus, dn, dns)
    assert oq.rel_l2(y.float().cpu().numpy(), ref) <= 1e-3


# ---- weight-only (W8A16) grouped GEMM over the same int8 pages --------------------------


def _w16_rows(rng, n, H):
    return oq.round_bf16(rng.standard_normal((n, H)).astype(np.float32))


@pytest.mark.parametrize("swiglu", [False, True])
# K = H: one staged phase (256, 2048), 64-code chunks (320), several K phases (4096 at
# 64 rows, 12288)
@pytest.mark.parametrize("H,max_rows", [(256, None), (320, None), (2048, None), (4096, 4000), (12288, None)])
def test_grouped_w8a16_matches_oracle(dev, swiglu, H, max_rows):
    rng = np.random.default_rng(17)
    E, I, T, k = 16, 128, 40, 4
    gu, gus, dn, dns = _layer(rng, E, H, I)
    top = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int64)
    tok, coef, starts, counts, inv = om.route_stable(top, np.ones((T, k), np.float32), E)
    rows = _w16_rows(rng, T * k, H)
    layer = _moe().Int8ExpertLayer.from_arrays(*(torch.from_numpy(v) for v in (gu, gus, dn, dns)), dev)
    args = (_t(rows, dev, torch.bfloat16), layer.gate_up, layer.gate_up_scales, _t(starts, dev), _t(counts, dev))
    if swiglu:
        out, tag = _moe().grouped_w8a16_mm(*args, swiglu=True, max_rows=max_rows)
        assert tag.startswith("hip-gfx950-")
        ref = om.grouped_w8a16_mm(rows, gu, gus, starts, counts, swiglu=True)
        assert oq.rel_l2(out.float().cpu().numpy(), ref) <= 1e-3
    else:
        out, _ = _moe().grouped_w8a16_mm(*args, out_dtype=torch.float32, max_rows=max_rows)
        ref = om.grouped_w8a16_mm(rows, gu, gus, starts, counts, out_bf16=False)
        # exact bf16 products, fp32 sums in another order than the oracle's float64 sum
        assert oq.rel_l2(out.cpu().numpy(), ref) <= 1e-5
        o16, _ = _moe().grouped_w8a16_mm(*args, max_rows=max_rows)
        assert torch.equal(o16, out.to(torch.bfloat16))


@pytest.mark.parametrize("max_rows", [0, 16, 400, 4000])  # row tiles of 32, 16, 64, 64 rows
def test_grouped_w8a16_row_tiles_gather_and_slots(dev, max_rows):
    """Skewed routing (expert 0 takes every token) over several row passes; the in-kernel
    gather (row_ids) equals gathering first; slot indirection equals compact weights; an
    id outside the source reads zeros."""
    rng = np.random.default_rng(19)
    E, H, I, T, k = 8, 2048, 128, 200, 2
    gu, gus, dn, dns = _layer(rng, E, H, I)
    top = np.stack([np.concatenate([[0], 1 + rng.permutation(E - 1)[: k - 1]]) for _ in range(T)]).astype(np.int64)
    tok, coef, starts, counts, inv = om.route_stable(top, np.ones((T, k), np.float32), E)
    assert counts.max() == T
    src = _w16_rows(rng, T, H)
    layer = _moe().Int8ExpertLayer.from_arrays(*(torch.from_numpy(v) for v in (gu, gus, dn, dns)), dev)
    st, ct = _t(starts, dev), _t(counts, dev)
    got, _ = _moe().grouped_w8a16_mm(_t(src, dev, torch.bfloat16), layer.gate_up, layer.gate_up_scales, st, ct,
                                     row_ids=_t(tok, dev), max_rows=max_rows, swiglu=True)
    ref = om.grouped_w8a16_mm(src[tok], gu, gus, starts, counts, swiglu=True)
    assert oq.rel_l2(got.float().cpu().numpy(), ref) <= 1e-3
    pre, _ = _moe().grouped_w8a16_mm(_t(src[tok], dev, torch.bfloat16), layer.gate_up, layer.gate_up_scales, st, ct,
                                     max_rows=max_rows, swiglu=True)
    assert torch.equal(got, pre)
    perm = rng.permutation(E)
    slots = np.argsort(perm).astype(np.int32)
    phys = _moe().Int8ExpertLayer.from_arrays(*(torch.from_numpy(v[perm]) for v in (gu, gus, dn, dns)), dev)
    act = _t(_w16_rows(rng, T * k, I), dev, torch.bfloat16)
    o1, _ = _moe().grouped_w8a16_mm(act, phys.down, phys.down_scales, st, ct, group_slots=_t(slots, dev),
                                    max_rows=max_rows)
    o2, _ = _moe().grouped_w8a16_mm(act, layer.down, layer.down_scales, st, ct, max_rows=max_rows)
    assert torch.equal(o1, o2)
    bad = tok.copy()
    bad[3] = T  # outside the source
    ob, _ = _moe().grouped_w8a16_mm(_t(src, dev, torch.bfloat16), layer.gate_up, layer.gate_up_scales, st, ct,
                                    row_ids=_t(bad, dev), max_rows=max_rows, swiglu=True)
    assert torch.all(ob[3] == 0) and torch.equal(ob[:3], got[:3]) and torch.equal(ob[4:], got[4:])


@pytest.mark.parametrize("T", [64, 512])
def test_moe_layer_config4_w8a16(dev, T):
    """BASELINE config 4 through the weight-only flow: bf16 activations, no per-token
    quantization; closer to the float formulation than the W8A8 flow."""
    rng = np.random.default_rng(T + 1)
    E, k, H, I = 128, 8, 2048, 768
    gu, gus, dn, dns = _layer(rng, E, H, I)
    gus /= np.sqrt(H)
    dns /= np.sqrt(I)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    x = oq.round_bf16(rng.standard_normal((T, H)).astype(np.float32))
    layer = _moe().Int8ExpertLayer.from_arrays(*(torch.from_numpy(v) for v in (gu, gus, dn, dns)), dev)
    tw, ti = _moe().route_topk(_t(logits, dev), k)
    y = _moe().Int8ExpertBackend([layer], w8a16=True).moe(0, _t(x, dev, torch.bfloat16), ti, tw)
    assert y.dtype == torch.bfloat16 and y.shape == (T, H)
    idx, w = ti.cpu().numpy(), tw.float().cpu().numpy()
    ref = om.moe_forward_w8a16(x, idx, w, gu, gus, dn, dns)
    assert oq.rel_l2(y.float().cpu().numpy(), ref) <= 1e-3
    y8 = _moe().Int8ExpertBackend([layer]).moe(0, _t(x, dev, torch.bfloat16), ti, tw)
    dense = om.moe_dense_reference(x, idx, w, gu, gus, dn, dns)
    assert oq.rel_l2(y.float().cpu().numpy(), dense) < oq.rel_l2(y8.float().cpu().numpy(), dense)


# ---- route + source quantization in one launch, gathered in the gate/up kernel ---------


@pytest.mark.parametrize("T,E,k,H,dtype", [(64, 128, 8, 2048, torch.bfloat16), (512, 128, 8, 2048, torch.bfloat16),
                                           (7, 5, 3, 256, torch.float32), (33, 16, 4, 196, torch.bfloat16),
                                           (16385, 64, 4, 64, torch.bfloat16)])
def test_route_quant_equals_route_then_quantize(dev, T, E, k, H, dtype):
    """qs_moe_route_quant (one launch; the last two cases take its two-launch fallback:
    H % 8 != 0, and A * E > 2^22) gives qs_moe_route's plan and quantize_rows' codes and
    scales of the unpermuted source rows, bit for bit."""
    rng = np.random.default_rng(T + E + H)
    top = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int64)
    w = _t(rng.random((T, k)).astype(np.float32), dev)
    src = _t(rng.standard_normal((T, H)).astype(np.float32) * 3, dev, dtype)
    src[min(3, T - 1)] = 0  # a zero row: scale 1
    ti = _t(top, dev)
    got = _moe()._route_impl(ti, w, E, True, coef_f32=True, quant_source=src)
    want = _moe()._route_impl(ti, w, E, True, coef_f32=True)
    for a, b in zip(got[:5], want[:5]):
        assert torch.equal(a, b)
    q, s = _moe().quantize_rows(src)
    assert torch.equal(got[6], q) and torch.equal(got[7], s)


@pytest.mark.parametrize("swiglu", [False, True])
@pytest.mark.parametrize("max_rows", [0, 16, 4000])
def test_grouped_int8_rows_equals_gathered(dev, swiglu, max_rows):
    """grouped_int8_mm over the T quantized source rows through row_ids equals it over the
    gathered rows, bit for bit (skewed groups take several passes); an id outside the
    source reads a zero row."""
    rng = np.random.default_rng(23)
    E, H, I, T, k = 8, 2048, 128, 200, 2
    gu, gus, dn, dns = _layer(rng, E, H, I)
    top = np.stack([np.concatenate([[0], 1 + rng.permutation(E - 1)[: k - 1]]) for _ in range(T)]).astype(np.int64)
    tok, coef, starts, counts, inv = om.route_stable(top, np.ones((T, k), np.float32), E)
    layer = _moe().Int8ExpertLayer.from_arrays(*(torch.from_numpy(v) for v in (gu, gus, dn, dns)), dev)
    q = _t(rng.integers(-127, 128, size=(T, H), dtype=np.int8), dev)
    s = _t(rng.uniform(0.01, 0.1, size=T).astype(np.float32), dev)
    st, ct, td = _t(starts, dev), _t(counts, dev), _t(tok, dev)
    got, _ = _moe().grouped_int8_mm(q, s, layer.gate_up, layer.gate_up_scales, st, ct, swiglu=swiglu,
                                    max_rows=max_rows, row_ids=td)
    want, _ = _moe().grouped_int8_mm(q[td], s[td], layer.gate_up, layer.gate_up_scales, st, ct, swiglu=swiglu,
                                     max_rows=max_rows)
    assert torch.equal(got, want)
    bad = tok.copy()
    bad[5] = T
    ob, _ = _moe().grouped_int8_mm(q, s, layer.gate_up, layer.gate_up_scales, st, ct, swiglu=swiglu,
                                   max_rows=max_rows, row_ids=_t(bad, dev))
    assert torch.all(ob[5] == 0) and torch.equal(ob[:5], got[:5]) and torch.equal(ob[6:], got[6:])


@pytest.mark.parametrize("w8a16", [False, True])
def test_moe_layer_graph_replays_equal_eager(dev, w8a16):
    """The whole layer (route + quantization launch, gathered gate/up, requantization,
    down, reduce; or the weight-only flow) captured in a HIP graph: three replays with
    eager work and synchronizations between them each equal the eager result bit for bit."""
    rng = np.random.default_rng(29)
    E, k, H, I, T = 32, 4, 512, 256, 48
    gu, gus, dn, dns = _layer(rng, E, H, I)
    layer = _moe().Int8ExpertLayer.from_arrays(*(torch.from_numpy(v) for v in (gu, gus, dn, dns)), dev)
    backend = _moe().Int8ExpertBackend([layer], w8a16=w8a16)
    x = _t(rng.standard_normal((T, H)).astype(np.float32), dev, torch.bfloat16)
    tw, ti = _moe().route_topk(_t(rng.standard_normal((T, E)).astype(np.float32), dev), k)
    eager = backend.moe(0, x, ti, tw)
    torch.cuda.synchronize()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        backend.moe(0, x, ti, tw)
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = backend.moe(0, x, ti, tw)
    for rep in range(3):
        backend.moe(0, x, ti, tw)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep}"
