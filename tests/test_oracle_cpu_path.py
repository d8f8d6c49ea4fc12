"""The CPU baseline (reference CPU qrow path restated with torch CPU ops) against the oracle."""

from __future__ import annotations

import numpy as np
import torch

from oracle import cpu_path
from oracle import qrow as oq


def _case(n, k, seed):
    rng = np.random.default_rng(seed)
    return (rng.integers(-127, 128, size=(n, k), dtype=np.int8),
            (rng.uniform(0.5, 1.5, size=n) / 127).astype(np.float32), rng)


def test_dequant_bit_exact_vs_numpy():
    # reference tests/test_qstore_cache.py:49-64: fast dequant == numpy q.astype(f32) * sc
    q, s, _ = _case(64, 96, 0)
    got = cpu_path.dequant_qrow(q, s).numpy()
    want = q.astype(np.float32) * s[:, None]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(got.view(np.uint32), oq.dequant_qrow(q, s).view(np.uint32))


def test_bf16_matmul_matches_oracle():
    q, s, rng = _case(48, 128, 1)
    x = torch.from_numpy(rng.standard_normal((3, 128)).astype(np.float32)).to(torch.bfloat16)
    y = cpu_path.qstore_matmul(q, s, x)
    assert y.dtype == torch.bfloat16
    ref = oq.qrow_matmul_w8a16(q, s, x.float().numpy(), "bf16")
    assert oq.rel_l2(y.float().numpy(), ref) <= 1e-3


def test_fp32_matmul_matches_oracle():
    q, s, rng = _case(40, 64, 2)
    x = torch.from_numpy(rng.standard_normal((2, 64)).astype(np.float32))
    y = cpu_path.qstore_matmul(q, s, x, torch.float32).numpy()
    assert oq.rel_l2(y, oq.qrow_matmul_f32(q, s, x.numpy())) <= 1e-5


def test_w8a8_cpu_path_matches_golden():
    """The CPU W8A8 baseline reproduces the reference's own outputs (tests/golden/w8a8.npz)."""
    from pathlib import Path

    g = np.load(Path(__file__).resolve().parent / "golden" / "w8a8.npz", allow_pickle=False)
    q_w, sc_w, x = (torch.from_numpy(g[n]) for n in ("q_w", "sc_w", "x"))
    y0 = cpu_path.w8a8_matmul(q_w, sc_w, x, protect_k=0).numpy()
    assert np.array_equal(y0.view(np.uint32), g["y_k0"].view(np.uint32))
    for k in (4, 8):
        assert oq.rel_l2(cpu_path.w8a8_matmul(q_w, sc_w, x, protect_k=k).numpy(), g[f"y_k{k}"]) < 1e-6


def test_lowbit_cpu_path_matches_oracle():
    from oracle import lowbit as ol

    rng = np.random.default_rng(4)
    W = rng.standard_normal((70, 256)).astype(np.float32)
    for bits, quant in ((3, ol.quant_row_int3), (2, ol.quant_row_int2)):
        packed, scales = quant(W, G=128)
        x = rng.standard_normal((3, 256)).astype(np.float32)
        off = 4.0 if bits == 3 else 1.0
        y = cpu_path.lowbit_matmul(packed, scales, None, torch.from_numpy(x), 256, bits, 128, off, chunk_rows=32)
        assert oq.rel_l2(y.numpy(), ol.lowbit_matmul(packed, scales, x, 256, bits, 128)) <= 1e-5
    # asymmetric G64 with zero points
    packed, scales, zeros = ol.quant_row_asym(W, 3, G=64)
    x = rng.standard_normal((2, 256)).astype(np.float32)
    y = cpu_path.lowbit_matmul(packed, scales, zeros, torch.from_numpy(x), 256, 3, 64, 0.0)
    ref = ol.lowbit_matmul(packed, scales, x, 256, 3, 64, zeros=zeros)
    assert oq.rel_l2(y.numpy(), ref) <= 1e-5


def test_moe_cpu_path_matches_streamed_reference():
    from pathlib import Path

    from oracle import moe as om

    g = np.load(Path(__file__).resolve().parent / "golden" / "moe_forward.npz", allow_pickle=False)
    y = torch.from_numpy(g["bf16_y"])
    got = cpu_path.moe_layer(y, torch.from_numpy(g["bf16_top_idx"]), torch.from_numpy(g["bf16_top_w"]).to(torch.bfloat16),
                             g["gu_q"], g["gu_s"], g["dn_q"], g["dn_s"])
    h1 = (torch.from_numpy(g["bf16_h0"]).to(torch.bfloat16) + got).float().numpy()
    assert oq.rel_l2(h1, g["bf16_h1"]) < 1e-3
