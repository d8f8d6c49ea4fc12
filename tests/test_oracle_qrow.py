"""Pins the qrow oracle (CPU) against the reference's own KATs, library routines and brute force."""

from __future__ import annotations

import numpy as np
import torch

from oracle import qrow as oq


def test_reference_compact_qrow_kat_exact():
    # reference tests/test_dense_qstore_cuda.py:72-96: fp32 path must equal x @ (codes*scales).T
    codes = np.array([[1, -2, 3, 4], [-1, 2, 0, 3], [4, 1, -3, 2]], dtype=np.int8)
    scales = np.array([0.5, 0.25, 0.125], dtype=np.float32)
    x = np.array([[1.0, 2.0, -1.0, 0.5], [0.5, -1.0, 2.0, 3.0]], dtype=np.float32)
    got = oq.qrow_matmul_f32(codes, scales, x)
    # hand expansion of the KAT (all values are exact binary fractions)
    W = np.array(
        [[0.5, -1.0, 1.5, 2.0], [-0.25, 0.5, 0.0, 0.75], [0.5, 0.125, -0.375, 0.25]],
        dtype=np.float32,
    )
    np.testing.assert_array_equal(oq.dequant_qrow(codes, scales), W)
    expected = np.array(
        [[0.5 - 2.0 - 1.5 + 1.0, -0.25 + 1.0 + 0.0 + 0.375, 0.5 + 0.25 + 0.375 + 0.125],
         [0.25 + 1.0 + 3.0 + 6.0, -0.125 - 0.5 + 0.0 + 2.25, 0.25 - 0.125 - 0.75 + 0.75]],
        dtype=np.float32,
    )
    np.testing.assert_array_equal(got, expected)


def test_round_bf16_matches_torch_cast_including_ties_and_specials():
    rng = np.random.default_rng(1)
    vals = rng.standard_normal(20000).astype(np.float32) * np.float32(3.0)
    # exact ties: bf16 grid point + half an ulp (both parities), subnormals, extremes
    grid = np.array([1.0, 1.0078125, 2.0, 3.0, -1.0078125], dtype=np.float32)
    ties = (grid.view(np.uint32) + np.uint32(0x8000)).view(np.float32)
    specials = np.array(
        [0.0, -0.0, 1e-40, -1e-40, 3.4e38, -3.4e38, np.inf, -np.inf, np.nan], dtype=np.float32
    )
    a = np.concatenate([vals, ties, specials])
    ours = oq.round_bf16(a)
    ref = torch.from_numpy(a).to(torch.bfloat16).float().numpy()
    same = (ours.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(ours) & np.isnan(ref))
    assert same.all()


def test_round_f16_matches_torch_cast():
    rng = np.random.default_rng(2)
    a = (rng.standard_normal(5000) * 100).astype(np.float32)
    np.testing.assert_array_equal(
        oq.round_f16(a), torch.from_numpy(a).to(torch.float16).float().numpy()
    )


def test_quant_row_int8_brute_force():
    rng = np.random.default_rng(3)
    W = rng.standard_normal((6, 33)).astype(np.float32)
    W[2] = 0.0  # zero row -> scale 1, codes 0
    W[3, 5] = W[3].max() * 2  # dominant element -> code 127
    q, s = oq.quant_row_int8(W)
    for n in range(W.shape[0]):
        amax = np.float32(np.abs(W[n]).max())
        scale = np.float32(amax / np.float32(127.0)) if amax != 0 else np.float32(1.0)
        assert s[n] == scale
        for k in range(W.shape[1]):
            r = np.float32(W[n, k] / scale)
            lo = np.floor(r)
            frac = r - lo
            if frac > 0.5 or (frac == 0.5 and lo % 2 == 1):
                lo += 1
            assert q[n, k] == int(np.clip(lo, -127, 127))
    assert (q[2] == 0).all() and s[2] == 1.0
    assert q[3, 5] == 127


def test_w8a16_matmul_matches_float64_brute_force():
    rng = np.random.default_rng(4)
    q = rng.integers(-127, 128, size=(5, 7), dtype=np.int8)
    s = (rng.uniform(0.5, 1.5, size=5) / 127).astype(np.float32)
    x = oq.round_bf16(rng.standard_normal((3, 7)).astype(np.float32))
    got = oq.qrow_matmul_w8a16(q, s, x)
    for m in range(3):
        for n in range(5):
            acc = 0.0
            for k in range(7):
                w = float(oq.round_bf16(np.array([np.float32(q[n, k]) * s[n]], np.float32))[0])
                acc += float(x[m, k]) * w
            exp = oq.round_bf16(np.array([acc], dtype=np.float32))[0]
            assert got[m, n] == exp


def test_w8a16_weight_rounding_matters():
    # a plausible mistake (skipping the per-element bf16 weight rounding) must be visible
    rng = np.random.default_rng(5)
    q = rng.integers(-127, 128, size=(256, 1536), dtype=np.int8)
    s = (rng.uniform(0.5, 1.5, size=256) / 127).astype(np.float32)
    x = oq.round_bf16(rng.standard_normal((4, 1536)).astype(np.float32))
    good = oq.qrow_matmul_w8a16(q, s, x)
    unrounded = oq.round_bf16((x.astype(np.float64) @ oq.dequant_qrow(q, s).T.astype(np.float64)).astype(np.float32))
    assert oq.rel_l2(unrounded, good) > 1e-3


def test_swiglu_matches_torch_reference_composition():
    # operands of reference tests/test_dense_qstore_cuda.py:99-124, composed with torch CPU ops
    gc = np.array([[1, -2, 3, 4], [-1, 2, 0, 3], [4, 1, -3, 2]], dtype=np.int8)
    gs = np.array([0.5, 0.25, 0.125], dtype=np.float32)
    uc = np.array([[2, 1, -1, 3], [4, -2, 1, 0], [-3, 2, 2, 1]], dtype=np.int8)
    us = np.array([0.25, 0.125, 0.5], dtype=np.float32)
    x = np.array([[1.0, 2.0, -1.0, 0.5], [0.5, -1.0, 2.0, 3.0]], dtype=np.float32)
    xt = torch.from_numpy(x).to(torch.bfloat16)
    wg = (torch.from_numpy(gc).float() * torch.from_numpy(gs)[:, None]).to(torch.bfloat16)
    wu = (torch.from_numpy(uc).float() * torch.from_numpy(us)[:, None]).to(torch.bfloat16)
    g = (xt @ wg.t()).to(torch.bfloat16)
    u = (xt @ wu.t()).to(torch.bfloat16)
    silu = (g.float() * torch.sigmoid(g.float())).to(torch.bfloat16)
    ref = (silu.float() * u.float()).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(oq.qrow_swiglu(gc, gs, uc, us, x), ref)


def test_row_stable_equals_batched_in_oracle():
    rng = np.random.default_rng(6)
    q = rng.integers(-127, 128, size=(64, 128), dtype=np.int8)
    s = (rng.uniform(0.5, 1.5, size=64) / 127).astype(np.float32)
    x = oq.round_bf16(rng.standard_normal((5, 128)).astype(np.float32))
    full = oq.qrow_matmul_w8a16(q, s, x)
    for m in range(5):
        np.testing.assert_array_equal(oq.qrow_matmul_w8a16(q, s, x[m : m + 1])[0], full[m])


# ---- head top-2 and fp32 rerank ------------------------------------------------------------


def _kat_head():
    # reference tests/test_dense_qstore_cuda.py:246-266 (page rows 11..17, unit scales)
    codes = np.array(
        [[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 0], [0, 0, 0, 1], [1, 1, 0, 0], [-1, 0, 1, 0], [1, 1, 0, 0]],
        dtype=np.int8,
    )
    x = np.array([[2.0, 3.0, -1.0, 0.5], [-2.0, 0.0, 4.0, 1.0]], dtype=np.float32)
    return codes, np.ones(7, np.float32), x


def test_top2_and_rerank_reference_kat():
    codes, scales, x = _kat_head()
    idx, val = oq.qrow_top2(oq.head_logits(codes, scales, x, "fp32"), start_row=11)
    assert idx.tolist() == [[15, 17], [16, 13]]  # test_dense_qstore_cuda.py:281
    assert val.tolist() == [[5.0, 5.0], [6.0, 4.0]]
    best, best_v = oq.rerank_fp32(codes, scales, x, idx, start_row=11)
    assert best.tolist() == [15, 16] and best_v.tolist() == [5.0, 6.0]  # :283-284


def test_top2_semantic_row_count_masks_padding_kat():
    # reference tests/test_dense_qstore_cuda.py:289-311
    codes = np.array([[2, 0], [0, 2], [1, 1], [100, 100]], dtype=np.int8)
    scales = np.ones(4, np.float32)
    x = np.ones((1, 2), np.float32)
    logits = oq.head_logits(codes, scales, x, "fp32")
    for rows, want in ((None, 3), (3, 0)):
        cand, _ = oq.qrow_top2(logits, row_count=rows)
        best, _ = oq.rerank_fp32(codes, scales, x, cand)
        assert int(best[0]) == want


def test_top2_matches_a_stable_sort():
    # discrete logits with many ties: the first two of a (value desc, index asc) sort
    rng = np.random.default_rng(5)
    for _ in range(50):
        L = rng.integers(-4, 5, size=(3, 37)).astype(np.float32)
        idx, val = oq.qrow_top2(L, start_row=100)
        for m in range(3):
            order = np.lexsort((np.arange(37), -L[m]))
            assert idx[m].tolist() == [100 + int(order[0]), 100 + int(order[1])]
            assert val[m].tolist() == [float(L[m, order[0]]), float(L[m, order[1]])]
