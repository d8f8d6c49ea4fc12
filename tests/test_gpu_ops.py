"""The qstore_hip custom operators on the device: each against the CPU oracle, a chain of
them captured in a CUDA (HIP) graph and replayed, and a function of them compiled by
torch.compile (aot_eager backend, full graph), both equal to eager bit for bit."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import lowbit as ol
from oracle import moe as om
from oracle import qrow as oq
from oracle import w8a8 as ow

pytestmark = pytest.mark.gpu

BF16_TOL, F32_TOL = 1e-3, 1e-5


@pytest.fixture(scope="module")
def Q():
    import mrun_pub_amd.ops  # noqa: F401  (registers the operators)

    return torch.ops.qstore_hip


def _case(seed, n, k):
    rng = np.random.default_rng(seed)
    codes = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    scales = (rng.uniform(0.5, 1.5, size=n) / 127).astype(np.float32)
    return rng, codes, scales


def _d(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def _operands(dev):
    """A small decode step's worth of operands for every operator."""
    rng, gc, gs = _case(1, 512, 256)
    _, uc, us = _case(2, 512, 256)
    _, dc, ds = _case(3, 256, 512)
    x = oq.round_bf16(rng.standard_normal((2, 256)).astype(np.float32))
    E, k, H, I, T = 16, 4, 256, 128, 12
    gu = rng.integers(-127, 128, size=(E, 2 * I, H), dtype=np.int8)
    gus = (rng.uniform(0.5, 1.5, size=(E, 2 * I)) / 127).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    src = oq.round_bf16(rng.standard_normal((T, H)).astype(np.float32))
    W = rng.standard_normal((96, 256)).astype(np.float32)
    packed, lsc = ol.quant_row_int3(W, G=128)
    return dict(
        gc=_d(gc, dev), gs=_d(gs, dev), uc=_d(uc, dev), us=_d(us, dev), dc=_d(dc, dev), ds=_d(ds, dev),
        x=_d(x, dev, torch.bfloat16), gu=_d(gu, dev), gus=_d(gus, dev), logits=_d(logits, dev),
        src=_d(src, dev, torch.bfloat16), packed=_d(packed, dev), lsc=_d(lsc, dev),
        np=dict(gc=gc, gs=gs, uc=uc, us=us, dc=dc, ds=ds, x=x, gu=gu, gus=gus, logits=logits, src=src,
                packed=packed, lsc=lsc, E=E, k=k, H=H, I=I, T=T),
    )


def _step(Q, o):
    """A chain through most operators; every intermediate feeds a later call."""
    h = Q.qrow_swiglu(o["gc"], o["gs"], o["uc"], o["us"], o["x"])           # [2, 512] bf16
    y = Q.qrow_matmul(o["dc"], o["ds"], h, False)                            # [2, 256] bf16
    y32 = Q.w8a8_matmul(o["dc"], o["ds"], h, None, 4, torch.float32)         # [2, 256] f32
    top_i, top_v = Q.qrow_top2(o["gc"], o["gs"], y, 0, 512)
    w, idx = Q.moe_router(o["logits"], o["np"]["k"], True, torch.bfloat16)
    tok, coef, starts, counts, inv = Q.moe_route(idx, w, o["np"]["E"])
    qx, sx = Q.act_quant(o["src"].index_select(0, tok), None)
    act = Q.grouped_int8_mm(qx, sx, o["gu"], o["gus"], starts, counts, None, 0, True, torch.bfloat16)
    red = Q.route_reduce(act.float(), coef.float(), inv, o["np"]["T"], o["np"]["k"])
    lb = Q.lowbit_matmul(o["packed"], o["lsc"], None, y32, 3, 128, 256)
    act16 = Q.grouped_w8a16_mm(o["src"], o["gu"], o["gus"], starts, counts, tok, None, 0, True, torch.bfloat16)
    return h, y, y32, top_i, top_v, w, idx, tok, act, red, lb, act16


def test_ops_against_oracle(dev, Q):
    o = _operands(dev)
    n = o["np"]
    h, y, y32, top_i, top_v, w, idx, tok, act, red, lb, act16 = _step(Q, o)
    h_ref = oq.qrow_swiglu(n["gc"], n["gs"], n["uc"], n["us"], n["x"])
    assert oq.rel_l2(h.float().cpu().numpy(), h_ref) <= BF16_TOL
    hb = h.float().cpu().numpy()
    assert oq.rel_l2(y.float().cpu().numpy(), oq.qrow_matmul_w8a16(n["dc"], n["ds"], hb)) <= BF16_TOL
    assert oq.rel_l2(y32.cpu().numpy(), ow.w8a8_matmul(n["dc"], n["ds"], hb, protect_k=4)) <= F32_TOL
    L = oq.head_logits(n["gc"], n["gs"], y.float().cpu().numpy(), "bf16")
    ri, _ = oq.qrow_top2(L)
    got_i = top_i.cpu().numpy()
    for m in range(2):  # chosen rows are the best up to fp32 summation order
        tol = 1e-5 * np.abs(L[m]).max()
        assert abs(L[m, got_i[m, 0]] - L[m, ri[m, 0]]) <= tol
    rw, ridx = om.router(n["logits"], n["k"])
    assert np.array_equal(idx.cpu().numpy(), ridx)
    r_tok = om.route_stable(ridx, rw, n["E"])[0]
    assert np.array_equal(tok.cpu().numpy(), r_tok)
    q_r, s_r = om.quantize_rows(n["src"][r_tok])
    tk, cf, st, cn, iv = om.route_stable(ridx, rw, n["E"])
    act_ref = om.grouped_int8_mm(q_r, s_r, n["gu"], n["gus"], st, cn, swiglu=True)
    assert np.array_equal(act.float().cpu().numpy(), act_ref)
    act16_ref = om.grouped_w8a16_mm(n["src"][r_tok], n["gu"], n["gus"], st, cn, swiglu=True)
    assert oq.rel_l2(act16.float().cpu().numpy(), act16_ref) <= BF16_TOL
    red_ref = om.stable_route_reduce(act_ref, cf, iv, n["T"], n["k"])
    assert np.array_equal(red.cpu().numpy(), red_ref)
    lb_ref = ol.lowbit_matmul(n["packed"], n["lsc"], y32.cpu().numpy(), 256, 3, 128)
    assert oq.rel_l2(lb.cpu().numpy(), lb_ref) <= F32_TOL
    assert torch.equal(Q.int8_gemm(_d(q_r, dev), o["gu"][0]).cpu(),
                       torch.from_numpy(ow.int8_gemm(q_r, n["gu"][0])))
    assert torch.equal(Q.qrow_dequant(o["dc"], o["ds"], torch.float32).cpu(),
                       torch.from_numpy(oq.dequant_qrow(n["dc"], n["ds"])))


def test_ops_captured_in_graph(dev, Q):
    """Capture the chain once, replay it three times with eager work and syncs between;
    every replay equals the eager result bit for bit."""
    o = _operands(dev)
    eager = _step(Q, o)
    torch.cuda.synchronize()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        _step(Q, o)  # warm-up on the capture stream
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = _step(Q, o)
    for rep in range(3):
        _step(Q, o)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(out, eager):
            assert torch.equal(a, b), f"replay {rep}"


def test_ops_under_torch_compile(dev, Q):
    o = _operands(dev)

    def f(gc, gs, uc, us, dc, ds, x):
        h = Q.qrow_swiglu(gc, gs, uc, us, x)
        return Q.qrow_matmul(dc, ds, h, False) * 2

    compiled = torch.compile(f, backend="aot_eager", fullgraph=True)
    args = (o["gc"], o["gs"], o["uc"], o["us"], o["dc"], o["ds"], o["x"])
    assert torch.equal(compiled(*args), f(*args))
