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
