"""GPU parity of the int8 qrow kernels against the CPU oracle (through the C ABI)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import qrow as oq

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-3  # rel-L2, bf16 outputs
F32_TOL = 1e-5  # rel-L2, fp32 outputs


def _qrow():
    from mrun_pub_amd import qrow

    return qrow


def _case(n, k, seed=0):
    rng = np.random.default_rng(seed)
    codes = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    scales = (rng.uniform(0.5, 1.5, size=n) / 127).astype(np.float32)
    return rng, codes, scales


def _dev(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


@pytest.mark.parametrize("n,k", [(64, 128), (300, 1024), (17, 48), (5, 7), (33, 1040), (1030, 4096)])
@pytest.mark.parametrize("dtype", ["fp32", "bf16", "fp16"])
def test_dequant_bit_exact(dev, n, k, dtype):
    _, codes, scales = _case(n, k, seed=n + k)
    tdt = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}[dtype]
    got = _qrow().qrow_dequant(_dev(codes, dev), _dev(scales, dev), tdt).float().cpu().numpy()
    ref = oq.qrow_weight(codes, scales, dtype)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_reference_kat_fp32_exact(dev):
    # reference tests/test_dense_qstore_cuda.py:72-96 (generic kernel: K=4)
    codes = np.array([[1, -2, 3, 4], [-1, 2, 0, 3], [4, 1, -3, 2]], dtype=np.int8)
    scales = np.array([0.5, 0.25, 0.125], dtype=np.float32)
    x = np.array([[1.0, 2.0, -1.0, 0.5], [0.5, -1.0, 2.0, 3.0]], dtype=np.float32)
    from mrun_pub_amd.qrow import CompactQRowPage, fused_qrow_matmul

    page = CompactQRowPage("toy", 0, 3, 4, _dev(codes, dev), _dev(scales, dev))
    y, tag = fused_qrow_matmul(page, _dev(x, dev))
    assert tag.startswith("hip-gfx950")
    np.testing.assert_array_equal(y.cpu().numpy(), oq.qrow_matmul_f32(codes, scales, x))


@pytest.mark.parametrize("m", [1, 2, 5])
@pytest.mark.parametrize("n,k", [(4096, 1024), (256, 1536), (33, 80), (7, 13)])
def test_matmul_fp32(dev, m, n, k):
    rng, codes, scales = _case(n, k, seed=m * 7 + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = _qrow().qrow_matmul(_dev(codes, dev), _dev(scales, dev), _dev(x, dev))
    assert y.dtype == torch.float32 and y.shape == (m, n)
    err = oq.rel_l2(y.cpu().numpy(), oq.qrow_matmul_f32(codes, scales, x))
    assert err <= F32_TOL, err


@pytest.mark.parametrize("m", [1, 2, 3, 4, 16, 32, 37])
@pytest.mark.parametrize(
    "n,k", [(1536, 1536), (256, 1536), (8960, 1536), (1536, 8960), (1000, 4096), (100, 192), (24, 40)]
)
def test_matmul_bf16_w8a16(dev, m, n, k):
    rng, codes, scales = _case(n, k, seed=m * 31 + n + k)
    x = oq.round_bf16(rng.standard_normal((m, k)).astype(np.float32))
    y = _qrow().qrow_matmul(_dev(codes, dev), _dev(scales, dev), _dev(x, dev, torch.bfloat16))
    assert y.dtype == torch.bfloat16 and y.shape == (m, n)
    err = oq.rel_l2(y.float().cpu().numpy(), oq.qrow_matmul_w8a16(codes, scales, x))
    assert err <= BF16_TOL, err


@pytest.mark.parametrize("m,n", [(1, 512), (16, 512), (23, 512), (32, 512), (32, 200)])
def test_matmul_fp16(dev, m, n):
    """f16 rows; at M > 16 the 512-row case takes the activation-row split (32 units of 16
    rows), the 200-row case (13 units) the unsplit launch."""
    rng, codes, scales = _case(n, 1024, seed=m)
    x = oq.round_f16(rng.standard_normal((m, 1024)).astype(np.float32))
    y = _qrow().qrow_matmul(_dev(codes, dev), _dev(scales, dev), _dev(x, dev, torch.float16))
    assert y.dtype == torch.float16
    err = oq.rel_l2(y.float().cpu().numpy(), oq.qrow_matmul_w8a16(codes, scales, x, "fp16"))
    assert err <= BF16_TOL, err


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("n,k", [(1536, 1536), (512, 8960), (40, 48)])
def test_row_stable_batch_invariance(dev, dtype, n, k):
    """Row m of a row-stable batched call is bit-identical to a B=1 call
    (QStore.matmul_row_stable, qstore.py:49-76) and to the plain decode (M=1) call."""
    rng, codes, scales = _case(n, k, seed=11)
    x = torch.from_numpy(rng.standard_normal((32, k)).astype(np.float32)).to(dev).to(dtype)
    c, s = _dev(codes, dev), _dev(scales, dev)
    full = _qrow().qrow_matmul(c, s, x, row_stable=True)
    for m in (0, 5, 17, 31):
        one = _qrow().qrow_matmul(c, s, x[m : m + 1], row_stable=True)
        assert torch.equal(one[0], full[m])
        assert torch.equal(_qrow().qrow_matmul(c, s, x[m : m + 1])[0], full[m])
    ref = oq.qrow_matmul_f32(codes, scales, x.float().cpu().numpy())
    tol = F32_TOL if dtype == torch.float32 else BF16_TOL
    assert oq.rel_l2(full.float().cpu().numpy(), ref) <= 3 * tol


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,k", [(1536, 1536), (300, 8960), (64, 1000)])
def test_register_rows_match_single_row(dev, dtype, n, k):
    """Up to 4 bf16/f16 rows share one register-activation launch: every row is
    bit-identical to its own M=1 call, including the padded rows of M=3 (SwiGLU too)."""
    rng, codes, scales = _case(n, k, seed=17)
    _, codes2, scales2 = _case(n, k, seed=18)
    x = torch.from_numpy(rng.standard_normal((4, k)).astype(np.float32)).to(dev).to(dtype)
    c, s = _dev(codes, dev), _dev(scales, dev)
    for m in (2, 3, 4):
        full = _qrow().qrow_matmul(c, s, x[:m])
        for r in range(m):
            assert torch.equal(_qrow().qrow_matmul(c, s, x[r : r + 1])[0], full[r])
    if dtype == torch.bfloat16 and k % 16 == 0:
        gate = _qrow().CompactQRowPage("g", 0, n, k, c, s)
        up = _qrow().CompactQRowPage("u", 0, n, k, _dev(codes2, dev), _dev(scales2, dev))
        for m in (2, 3, 4):
            full = _qrow().fused_qrow_swiglu(gate, up, x[:m])[0]
            for r in range(m):
                assert torch.equal(_qrow().fused_qrow_swiglu(gate, up, x[r : r + 1])[0][0], full[r])


@pytest.mark.parametrize("m", [5, 16, 32])
def test_mfma_path_rows_independent_of_batch(dev, m):
    """Within the MFMA path (M >= 5) a row does not depend on the other rows."""
    rng, codes, scales = _case(1536, 1536, seed=13)
    x = torch.from_numpy(rng.standard_normal((m, 1536)).astype(np.float32)).to(dev).to(torch.bfloat16)
    c, s = _dev(codes, dev), _dev(scales, dev)
    full = _qrow().qrow_matmul(c, s, x)
    x2 = x.clone()
    x2[1:] = x2[1:].flip(0) if m > 2 else x2[1:]
    perm = _qrow().qrow_matmul(c, s, x2)
    assert torch.equal(perm[0], full[0])


@pytest.mark.parametrize("n,k,swiglu", [(1536, 1536, False), (256, 1536, False), (1536, 8960, False),
                                        (8960, 1536, True), (200, 384, True), (70, 1024, False)])
@pytest.mark.parametrize("m", [5, 16, 23, 32])
def test_batched_rows_equal_rows_alone(dev, n, k, swiglu, m):
    """qs_qrow_matmul_batched / qs_qrow_swiglu_batched: every row of an M-row call is bit for
    bit the row computed alone through the same entry point, and the batch matches the
    oracle to the bf16 tolerance."""
    q = _qrow()
    rng, codes, scales = _case(n, k, seed=m + n + k)
    _, codes2, scales2 = _case(n, k, seed=m + n + k + 1)
    x = oq.round_bf16(rng.standard_normal((m, k)).astype(np.float32))
    xd = _dev(x, dev, torch.bfloat16)
    pages = [(_dev(codes, dev), _dev(scales, dev))]
    if swiglu:
        pages.append((_dev(codes2, dev), _dev(scales2, dev)))
    full = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    q._run_batched(xd, pages, [full], swiglu=swiglu)
    for r in (0, m // 2, m - 1):
        one = torch.empty((1, n), dtype=torch.bfloat16, device=dev)
        q._run_batched(xd[r:r + 1].contiguous(), pages, [one], swiglu=swiglu)
        assert torch.equal(one[0], full[r]), r
    ref = oq.qrow_swiglu(codes, scales, codes2, scales2, x) if swiglu else oq.qrow_matmul_w8a16(codes, scales, x)
    assert oq.rel_l2(full.float().cpu().numpy(), ref) <= BF16_TOL
    if not swiglu and q._batched_eligible(xd, [pages[0][0]]):  # the public wrapper's path
        assert torch.equal(q.qrow_matmul(pages[0][0], pages[0][1], xd), full)
    if swiglu and q._batched_eligible(xd, [p[0] for p in pages], swiglu=True):
        g = q.CompactQRowPage("g", 0, n, k, *pages[0])
        u = q.CompactQRowPage("u", 0, n, k, *pages[1])
        assert torch.equal(q.fused_qrow_swiglu(g, u, xd)[0], full)


def test_multi_linear_equals_individual(dev):
    rng = np.random.default_rng(12)
    k = 1536
    pages = []
    for n in (1536, 256, 256):
        c = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        s = (rng.uniform(0.5, 1.5, size=n) / 127).astype(np.float32)
        pages.append((_dev(c, dev), _dev(s, dev)))
    x = torch.from_numpy(rng.standard_normal((4, k)).astype(np.float32)).to(dev).to(torch.bfloat16)
    outs = _qrow().qrow_matmul_multi(pages, x)
    xb = x.float().cpu().numpy()
    for (c, s), o in zip(pages, outs):
        ref = oq.qrow_matmul_w8a16(c.cpu().numpy(), s.cpu().numpy(), xb)
        assert oq.rel_l2(o.float().cpu().numpy(), ref) <= BF16_TOL
        single = _qrow().qrow_matmul(c, s, x)
        assert torch.allclose(o.float(), single.float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("m", [1, 2, 3, 4, 16, 32])
@pytest.mark.parametrize("n,k", [(8960, 1536), (1000, 1536), (200, 128), (96, 64), (5, 4)])
def test_swiglu(dev, m, n, k):
    rng = np.random.default_rng(m + n)
    gq = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    uq = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    gs = (rng.uniform(0.5, 1.5, size=n) / 127).astype(np.float32)
    us = (rng.uniform(0.5, 1.5, size=n) / 127).astype(np.float32)
    x = oq.round_bf16(rng.standard_normal((m, k)).astype(np.float32))
    from mrun_pub_amd.qrow import CompactQRowPage, fused_qrow_swiglu

    gp = CompactQRowPage("gate", 0, n, k, _dev(gq, dev), _dev(gs, dev))
    up = CompactQRowPage("up", 0, n, k, _dev(uq, dev), _dev(us, dev))
    y, tag = fused_qrow_swiglu(gp, up, _dev(x, dev, torch.bfloat16))
    assert y.dtype == torch.bfloat16 and tag.startswith("hip-gfx950")
    err = oq.rel_l2(y.float().cpu().numpy(), oq.qrow_swiglu(gq, gs, uq, us, x))
    assert err <= BF16_TOL, err


@pytest.mark.parametrize("n,k", [(8960, 1536), (8193, 512), (12000, 256), (16384, 2048), (16385, 1040),
                                 (20000, 1536)])
def test_swiglu_rows_equal_row_blocks(dev, n, k):
    """At M = 1 a SwiGLU with more rows than one resident round of waves (8192 on 256 CUs)
    runs its last rows in a later round: every output equals the same row computed in
    launches of at most 4096 rows bit for bit, whatever the row count and tail kind, and
    the oracle within the bf16 tolerance."""
    from mrun_pub_amd.qrow import CompactQRowPage, fused_qrow_swiglu

    rng = np.random.default_rng(n + k)
    gq = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    uq = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    gs = (rng.uniform(0.5, 1.5, size=n) / 127).astype(np.float32)
    us = (rng.uniform(0.5, 1.5, size=n) / 127).astype(np.float32)
    x = oq.round_bf16(rng.standard_normal((1, k)).astype(np.float32))
    gqd, uqd, gsd, usd = (_dev(a, dev) for a in (gq, uq, gs, us))
    xd = _dev(x, dev, torch.bfloat16)
    full = fused_qrow_swiglu(CompactQRowPage("g", 0, n, k, gqd, gsd), CompactQRowPage("u", 0, n, k, uqd, usd), xd)[0]
    parts = []
    for a in range(0, n, 4096):
        e = min(n, a + 4096)
        parts.append(fused_qrow_swiglu(CompactQRowPage("g", 0, e - a, k, gqd[a:e], gsd[a:e]),
                                       CompactQRowPage("u", 0, e - a, k, uqd[a:e], usd[a:e]), xd)[0])
    assert torch.equal(full, torch.cat(parts, dim=1))
    err = oq.rel_l2(full.float().cpu().numpy(), oq.qrow_swiglu(gq, gs, uq, us, x))
    assert err <= BF16_TOL, err


def test_errors_are_reference_exceptions(dev):
    from mrun_pub_amd.qrow import CompactQRowPage, fused_qrow_matmul, fused_qrow_swiglu

    codes = torch.zeros((8, 16), dtype=torch.int8, device=dev)
    scales = torch.ones(8, dtype=torch.float32, device=dev)
    page = CompactQRowPage("p", 0, 8, 16, codes, scales)
    with pytest.raises(ValueError, match="activation width"):
        fused_qrow_matmul(page, torch.zeros((1, 15), device=dev))
    with pytest.raises(ValueError, match="one device"):
        fused_qrow_matmul(page, torch.zeros((1, 16)))
    with pytest.raises(ValueError, match="block_m"):
        fused_qrow_matmul(page, torch.zeros((1, 16), device=dev), block_m=8)
    with pytest.raises(ValueError, match="BF16"):
        fused_qrow_swiglu(page, page, torch.zeros((1, 16), device=dev))


# ---- head: fused top-2 and fp32 rerank ---------------------------------------------------------


def _page(codes, scales, dev, start_row=0):
    from mrun_pub_amd.qrow import CompactQRowPage

    n, k = codes.shape
    return CompactQRowPage("lm_head", start_row, start_row + n, k, _dev(codes, dev), _dev(scales, dev))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_top2_reference_kat(dev, dtype):
    """reference tests/test_dense_qstore_cuda.py:246-287 on the device (K=4: generic path)."""
    codes = np.array(
        [[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 0], [0, 0, 0, 1], [1, 1, 0, 0], [-1, 0, 1, 0], [1, 1, 0, 0]],
        dtype=np.int8,
    )
    page = _page(codes, np.ones(7, np.float32), dev, start_row=11)
    x = torch.tensor([[2.0, 3.0, -1.0, 0.5], [-2.0, 0.0, 4.0, 1.0]], device=dev).to(dtype)
    q = _qrow()
    cand, vals, tag, _ = q.fused_qrow_top2(page, x)
    assert cand.cpu().tolist() == [[15, 17], [16, 13]] and cand.dtype == torch.int32
    assert vals.cpu().tolist() == [[5.0, 5.0], [6.0, 4.0]]
    assert tag.startswith("hip-gfx950")
    best, best_v = q.rerank_qrow_candidates_fp32(page, x, cand)
    assert best.cpu().tolist() == [15, 16] and best_v.cpu().tolist() == [5.0, 6.0]
    fused, _, ftag, _ = q.fused_qrow_reranked_argmax(page, x)
    assert torch.equal(fused, best) and ftag.endswith("+fp32-candidate-rerank-v1")


def test_top2_semantic_row_count_kat(dev):
    """reference tests/test_dense_qstore_cuda.py:289-311: padding rows never compete."""
    page = _page(np.array([[2, 0], [0, 2], [1, 1], [100, 100]], np.int8), np.ones(4, np.float32), dev)
    x = torch.ones((1, 2), device=dev)
    q = _qrow()
    assert int(q.fused_qrow_reranked_argmax(page, x)[0].item()) == 3
    assert int(q.fused_qrow_reranked_argmax(page, x, semantic_row_count=3)[0].item()) == 0
    for invalid, error in ((True, TypeError), (1, ValueError), (5, ValueError), (2.5, TypeError)):
        with pytest.raises(error, match="semantic_row_count"):
            q.fused_qrow_top2(page, x, semantic_row_count=invalid)
    with pytest.raises(ValueError, match="head tiles"):
        q.fused_qrow_top2(page, x, block_n=32)
    with pytest.raises(ValueError, match="outside the compact head page"):
        q.rerank_qrow_candidates_fp32(page, x, torch.tensor([[4]], device=dev))


def _exact_head(v, k, m, seed):
    """Codes x scale 2^-6 x activations on a 1/16 grid: every product and sum is exact in
    fp32 and the weights are exact in bf16/fp16, so logits (and their ties) are exact."""
    rng = np.random.default_rng(seed)
    codes = rng.integers(-127, 128, size=(v, k), dtype=np.int8)
    scales = np.full(v, 2.0 ** -6, np.float32)
    x = (rng.integers(-8, 9, size=(m, k)) / 16.0).astype(np.float32)
    return codes, scales, x


@pytest.mark.parametrize("v,k", [(5000, 1536), (4099, 1024), (3001, 2304), (777, 8960), (600, 1000)])
@pytest.mark.parametrize("m", [1, 2, 5])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_top2_exact_heads(dev, v, k, m, dtype):
    """Every row tail kind (none, 4/8/12-byte, ragged -> generic path), batches of MB rows."""
    codes, scales, x = _exact_head(v, k, m, seed=v + k + m)
    start, rows = 37, v - 3
    page = _page(codes, scales, dev, start_row=start)
    cand, vals, _, _ = _qrow().fused_qrow_top2(page, _dev(x, dev, dtype), semantic_row_count=rows)
    dname = {torch.bfloat16: "bf16", torch.float32: "fp32", torch.float16: "fp16"}[dtype]
    ri, rv = oq.qrow_top2(oq.head_logits(codes, scales, x, dname), start_row=start, row_count=rows)
    assert np.array_equal(cand.cpu().numpy(), ri)
    assert np.array_equal(vals.cpu().numpy(), rv)
    best, bv = _qrow().rerank_qrow_candidates_fp32(page, _dev(x, dev, dtype), cand)
    oi, ov = oq.rerank_fp32(codes, scales, x, ri, start_row=start)
    assert np.array_equal(best.cpu().numpy(), oi) and np.array_equal(bv.cpu().numpy(), ov)


def test_top2_full_vocabulary_decode(dev):
    """A 151,936 x 1536 int8 head (Qwen2-1.5B's lm_head shape), one bf16 decode row."""
    codes, scales, x = _exact_head(151936, 1536, 1, seed=9)
    page = _page(codes, scales, dev)
    cand, vals, _, _ = _qrow().fused_qrow_top2(page, _dev(x, dev, torch.bfloat16))
    ri, rv = oq.qrow_top2(oq.head_logits(codes, scales, x, "bf16"))
    assert np.array_equal(cand.cpu().numpy(), ri) and np.array_equal(vals.cpu().numpy(), rv)


def test_top2_random_floats_within_tolerance(dev):
    """General inputs: the chosen rows are the best up to fp32 summation order."""
    rng, codes, scales = _case(20000, 1536, seed=4)
    x = oq.round_bf16(rng.standard_normal((2, 1536)).astype(np.float32))
    page = _page(codes, scales, dev)
    cand, vals, _, _ = _qrow().fused_qrow_top2(page, _dev(x, dev, torch.bfloat16))
    L = oq.head_logits(codes, scales, x, "bf16").astype(np.float64)
    ci, cv = cand.cpu().numpy(), vals.cpu().numpy()
    for m in range(2):
        top = np.sort(L[m])[::-1]
        tol = 1e-5 * np.abs(L[m]).max()
        assert abs(L[m, ci[m, 0]] - top[0]) <= tol and abs(L[m, ci[m, 1]] - top[1]) <= tol
        assert np.allclose(cv[m], L[m, ci[m]], rtol=0, atol=tol) and ci[m, 0] != ci[m, 1]
