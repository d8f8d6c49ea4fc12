"""HIP kernels vs golden vectors written from the reference itself (tests/golden/)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import qrow as oq

pytestmark = pytest.mark.gpu

GOLD = __import__("pathlib").Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(GOLD / name, allow_pickle=False)


def test_w8a8_kernels_vs_reference(dev):
    from mrun_pub_amd import w8a8

    g = _load("w8a8.npz")
    acc = w8a8._int8_gemm(torch.from_numpy(g["gemm_qx"]).to(dev), torch.from_numpy(g["gemm_qw"]).to(dev))
    assert np.array_equal(acc.cpu().numpy(), g["gemm_acc"])
    qw, sw, x = (torch.from_numpy(g[n]).to(dev) for n in ("q_w", "sc_w", "x"))
    y0 = w8a8.w8a8_matmul(qw, sw, x).cpu().numpy()
    assert np.array_equal(y0.view(np.uint32), g["y_k0"].view(np.uint32))
    for k in (4, 8):
        assert oq.rel_l2(w8a8.w8a8_matmul(qw, sw, x, protect_k=k).cpu().numpy(), g[f"y_k{k}"]) < 1e-5
    ys = w8a8.w8a8_matmul(qw, sw, x, protect_idx=torch.from_numpy(g["protect_idx"]).to(dev)).cpu().numpy()
    assert oq.rel_l2(ys, g["y_static"]) < 1e-5


@pytest.mark.parametrize("tag", ["f32", "bf16"])
def test_route_and_reduce_vs_reference(dev, tag):
    from mrun_pub_amd import moe

    g = _load("moe.npz")
    top = torch.from_numpy(g["top"]).to(dev)
    w = torch.from_numpy(g["w32"])
    w = (w if tag == "f32" else w.to(torch.bfloat16)).to(dev)
    tok, coef, starts, counts, inv, _ = moe.grouped_route_tensors_with_inverse(top, w, num_experts=16)
    for name, arr in (("tok", tok), ("starts", starts), ("counts", counts), ("inv", inv)):
        assert np.array_equal(arr.cpu().numpy(), g[f"{name}_{tag}"]), name
    assert np.array_equal(coef.float().cpu().numpy(), g[f"coef_{tag}"])
    if tag == "f32":
        red = moe.stable_route_reduce(torch.from_numpy(g["eo32"]).to(dev), coef, tok, counts, top,
                                      torch.arange(16, device=dev), inverse_assignments=inv)
        assert np.array_equal(red.cpu().numpy(), g["red_f32"])
    else:
        eob = torch.from_numpy(g["eo_bf16_as_f32"]).to(dev).to(torch.bfloat16)
        red = moe.stable_route_reduce(eob, coef, tok, counts, top, torch.arange(16, device=dev))
        assert np.array_equal(red.cpu().numpy(), g["red_bf16"])


def test_lowbit_dequant_vs_reference_codec(dev):
    from mrun_pub_amd import lowbit

    from oracle import lowbit as ol

    g = _load("codecs.npz")
    K = g["W"].shape[1]
    for bits, p, s in ((3, g["p3g4"], g["s3g4"]), (2, g["p2g4"], g["s2g4"])):
        page = lowbit.LowbitPage("w", bits, 4, K, torch.from_numpy(p).to(dev), torch.from_numpy(s).to(dev))
        got = lowbit.lowbit_dequant(page).cpu().numpy()
        assert np.array_equal(got, ol.dequant(p, s, K, bits, 4))
