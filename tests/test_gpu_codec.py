"""Device codecs against the reference's golden vectors and the numpy oracle (bit-exact)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import lowbit as ol
from oracle import qrow as oq

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _codecs():
    from mrun_pub_amd import codecs

    return codecs


def _golden():
    return np.load(GOLDEN / "codecs.npz", allow_pickle=False)


def test_golden_codecs_from_the_reference(dev):
    """tests/golden/codecs.npz was written by the reference's own writers."""
    g = _golden()
    W = torch.from_numpy(g["W"]).to(dev)
    c = _codecs()
    q, s = c.quant_row_int8(W)
    assert np.array_equal(q.cpu().numpy(), g["q8"]) and np.array_equal(s.cpu().numpy(), g["s8"])
    for bits, G, pk, sk in ((3, 128, "p3", "s3"), (2, 128, "p2", "s2"), (3, 4, "p3g4", "s3g4"), (2, 4, "p2g4", "s2g4")):
        fn = c.quant_row_int3 if bits == 3 else c.quant_row_int2
        p, sc = fn(W, G=G)
        assert np.array_equal(p.cpu().numpy(), g[pk]), (bits, G)
        assert np.array_equal(sc.cpu().numpy().view(np.uint32), g[sk].view(np.uint32)), (bits, G)


def _matrix(rng, n, k):
    W = rng.standard_normal((n, k)).astype(np.float32)
    W[0] = 0.0                       # zero row: scale 1
    W[1, : k // 2] = 0.5             # constant run
    W[2] = np.round(W[2] * 4) / 4    # many exact quarter values: round-half-even ties
    W[3, ::3] = -0.0
    return W


@pytest.mark.parametrize("n,k", [(64, 1536), (7, 300), (33, 4100), (5, 301), (9, 4099)])
def test_int8_matches_oracle(dev, n, k):
    # K % 4 == 0 takes the 16-byte-load kernel, the rest the scalar one
    W = _matrix(np.random.default_rng(n + k), n, k)
    q, s = _codecs().quant_row_int8(torch.from_numpy(W).to(dev))
    rq, rs = oq.quant_row_int8(W)
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(s.cpu().numpy(), rs)


@pytest.mark.parametrize("bits", [3, 2])
@pytest.mark.parametrize("G", [4, 8, 64, 128, 300, 1000, 4096])
@pytest.mark.parametrize("k", [300, 4100, 512, 4096])
def test_lowbit_matches_oracle(dev, bits, G, k):
    """Group sizes around numpy's pairwise-sum branches (< 8, <= 128, recursive splits),
    ragged last groups, packed streams that end mid-byte; G = 128 with K % 128 == 0 takes
    the one-launch kernel (half a wave per group)."""
    W = _matrix(np.random.default_rng(bits * 1000 + G + k), 24, k)
    fn = _codecs().quant_row_int3 if bits == 3 else _codecs().quant_row_int2
    p, s = fn(torch.from_numpy(W).to(dev), G=G)
    rp, rs = (ol.quant_row_int3 if bits == 3 else ol.quant_row_int2)(W, G=G)
    assert np.array_equal(p.cpu().numpy(), rp)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), rs.view(np.uint32))


def test_codec_errors(dev):
    c = _codecs()
    with pytest.raises(ValueError):
        c.quant_row_int8(torch.zeros((2, 3), dtype=torch.float64, device=dev))
    with pytest.raises(ValueError):
        c.quant_row_int3(torch.zeros((2, 8), device=dev), G=0)
