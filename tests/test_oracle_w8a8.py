"""Pins the W8A8 oracle (CPU): brute force, torch's own ops in the reference composition,
and the reference's published test properties (tests/test_w8a8.py:14-64)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import w8a8 as ow


def _setup(out=64, inn=128, T=5, n_outlier=3, seed=0):
    # same construction as the reference's _setup (test_w8a8.py:14-22), numpy RNG
    rng = np.random.default_rng(seed)
    q_w = rng.integers(-127, 128, size=(out, inn), dtype=np.int8)
    sc_w = (rng.random(out) * 0.02 + 1e-3).astype(np.float32)
    W = q_w.astype(np.float32) * sc_w[:, None]
    x = rng.standard_normal((T, inn)).astype(np.float32)
    x[:, rng.permutation(inn)[:n_outlier]] *= 300.0
    ref = x @ W.T
    return q_w, sc_w, x, ref


def test_int8_gemm_brute_force():
    rng = np.random.default_rng(1)
    qx = rng.integers(-128, 128, size=(3, 37), dtype=np.int8)
    qw = rng.integers(-128, 128, size=(4, 37), dtype=np.int8)
    acc = ow.int8_gemm(qx, qw)
    for t in range(3):
        for n in range(4):
            assert acc[t, n] == sum(int(qx[t, k]) * int(qw[n, k]) for k in range(37))
    # extreme magnitudes: K * 127^2 stays within int32 for K = 4096
    big = np.full((1, 4096), 127, np.int8)
    assert ow.int8_gemm(big, -big)[0, 0] == -4096 * 127 * 127
    # the float64 evaluation equals numpy's integer matmul on full-width random operands,
    # -128 included (a lossy float32 evaluation would fail here)
    qx = rng.integers(-128, 128, size=(33, 14336), dtype=np.int8)
    qw = rng.integers(-128, 128, size=(50, 14336), dtype=np.int8)
    qx[0] = -128
    qw[0] = -128
    qx[1] = 127
    qw[1] = 127
    qw[1, 0] = 126  # an odd sum above 2^24: not representable in float32
    exact = qx.astype(np.int64) @ qw.astype(np.int64).T
    assert np.array_equal(ow.int8_gemm(qx, qw), exact)
    assert not np.array_equal((qx.astype(np.float32) @ qw.astype(np.float32).T).astype(np.int64), exact)


def test_act_quant_matches_reference_torch_composition():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((9, 300)).astype(np.float32)
    x[0] = 0.0  # zero row -> scale 1, codes 0
    x[1, :4] = [1.5, 2.5, -0.5, 127.0]  # half-way points after scaling: ties to even
    x[2] *= 1e-20
    keep = np.ones(300, np.float32)
    keep[[3, 17]] = 0.0
    for kp in (None, keep):
        q, s = ow.act_quant(x, kp)
        xt = torch.from_numpy(x)
        src = xt if kp is None else xt * torch.from_numpy(kp)
        sc = src.abs().amax(dim=1, keepdim=True) / 127.0
        sc = torch.where(sc == 0, torch.ones_like(sc), sc)
        qt = torch.round(src / sc).clamp_(-127, 127).to(torch.int8)
        assert np.array_equal(q, qt.numpy())
        assert np.array_equal(s, sc[:, 0].numpy())
    assert (ow.act_quant(x)[0][0] == 0).all() and ow.act_quant(x)[1][0] == 1.0


def test_round_half_even_is_used():
    # a mistaken round-half-away would turn 2.5 into 3
    x = np.array([[2.5, -2.5, 0.5, 127.0]], np.float32)  # scale = 1
    q, s = ow.act_quant(x)
    assert s[0] == 1.0 and q.tolist() == [[2, -2, 0, 127]]


def test_reference_properties_outlier_protection():
    q_w, sc_w, x, ref = _setup(n_outlier=3)
    d0 = np.abs(ow.w8a8_matmul(q_w, sc_w, x, protect_k=0) - ref).max()
    d = np.abs(ow.w8a8_matmul(q_w, sc_w, x, protect_k=4) - ref).max()
    assert d0 > 20.0 and d < 0.5 and d < d0 / 20


def test_reference_properties_argmax_and_static_list():
    q_w, sc_w, x, ref = _setup(out=128, inn=256, T=8, n_outlier=4)
    y = ow.w8a8_matmul(q_w, sc_w, x, protect_k=8)
    assert np.array_equal(y.argmax(-1), ref.argmax(-1))
    q_w, sc_w, x, _ = _setup(n_outlier=3)
    idx = ow.protect_topk(x, 4)
    assert np.array_equal(ow.w8a8_matmul(q_w, sc_w, x, protect_idx=idx), ow.w8a8_matmul(q_w, sc_w, x, protect_k=4))


def test_no_side_path_epilogue_is_closed_form():
    q_w, sc_w, x, _ = _setup(out=16, inn=64, T=3, n_outlier=0)
    q, s = ow.act_quant(x)
    acc = ow.int8_gemm(q, q_w)
    exp = (acc.astype(np.float32) * s[:, None]).astype(np.float32) * sc_w[None, :]
    assert np.array_equal(ow.w8a8_matmul(q_w, sc_w, x), exp)


def test_protect_topk_matches_torch_topk():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((7, 500)).astype(np.float32)
    idx = ow.protect_topk(x, 8)
    ref = torch.topk(torch.from_numpy(np.abs(x).max(axis=0)), 8).indices.numpy()
    assert np.array_equal(idx, ref)
