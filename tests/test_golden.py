"""Oracle vs golden vectors written from the reference itself (tests/golden/make_golden.py).

CPU only.  Bit-exact where the reference's arithmetic is fixed (codecs, integer GEMM, route
plans, the reducer, W8A8 without the fp32 side path); the side path goes through the
reference's CPU BLAS, whose summation order is not fixed, so those cases use the fp32
output tolerance.
"""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import lowbit as ol
from oracle import moe as om
from oracle import qrow as oq
from oracle import w8a8 as ow

GOLD = Path(__file__).resolve().parent / "golden"


def _load(name):
    path = GOLD / name
    manifest = json.loads((GOLD / "golden_manifest.json").read_text())
    assert hashlib.sha256(path.read_bytes()).hexdigest() == manifest[name], f"{name} modified"
    return np.load(path, allow_pickle=False)


def test_w8a8_golden():
    g = _load("w8a8.npz")
    assert np.array_equal(ow.int8_gemm(g["gemm_qx"], g["gemm_qw"]), g["gemm_acc"])
    y0 = ow.w8a8_matmul(g["q_w"], g["sc_w"], g["x"], protect_k=0)
    assert np.array_equal(y0.view(np.uint32), g["y_k0"].view(np.uint32))
    for k in (4, 8):
        y = ow.w8a8_matmul(g["q_w"], g["sc_w"], g["x"], protect_k=k)
        assert oq.rel_l2(y, g[f"y_k{k}"]) < 1e-6
    ys = ow.w8a8_matmul(g["q_w"], g["sc_w"], g["x"], protect_idx=g["protect_idx"])
    assert oq.rel_l2(ys, g["y_static"]) < 1e-6


@pytest.mark.parametrize("tag,G", [("", 128), ("g4", 4)])
def test_lowbit_codec_golden(tag, G):
    g = _load("codecs.npz")
    p3, s3 = ol.quant_row_int3(g["W"], G=G)
    p2, s2 = ol.quant_row_int2(g["W"], G=G)
    assert np.array_equal(p3, g[f"p3{tag}"]) and np.array_equal(s3, g[f"s3{tag}"])
    assert np.array_equal(p2, g[f"p2{tag}"]) and np.array_equal(s2, g[f"s2{tag}"])


def test_int8_codec_golden():
    g = _load("codecs.npz")
    q, s = oq.quant_row_int8(g["W"])
    assert np.array_equal(q, g["q8"]) and np.array_equal(s, g["s8"])


@pytest.mark.parametrize("tag", ["f32", "bf16"])
def test_route_golden(tag):
    g = _load("moe.npz")
    w = g["w32"] if tag == "f32" else oq.round_bf16(g["w32"])
    tok, coef, starts, counts, inv = om.route_stable(g["top"], w, 16)
    for name, arr in (("tok", tok), ("coef", coef), ("starts", starts), ("counts", counts), ("inv", inv)):
        assert np.array_equal(arr, g[f"{name}_{tag}"]), name


def test_reduce_golden():
    g = _load("moe.npz")
    T, k = g["top"].shape
    _, coef, _, _, inv = om.route_stable(g["top"], g["w32"], 16)
    assert np.array_equal(om.stable_route_reduce(g["eo32"], coef, inv, T, k), g["red_f32"])
    cb = oq.round_bf16(coef)
    assert np.array_equal(om.stable_route_reduce(g["eo_bf16_as_f32"], cb, inv, T, k), g["red_bf16"])
