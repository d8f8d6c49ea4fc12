"""The allocation-free head top-2 entry point (qs_qrow_top2_noalloc) against qs_qrow_top2.

Both are called through the C ABI with the same operands; the allocation-free call must
give the same indices and logits bit for bit.  Two calls run back to back on one device,
the second with a smaller input, so the second reads a scratch array that still holds
the first call's candidates.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _nat():
    import mrun_pub_amd._native as nat

    return nat


def _operands(dev, v, k, m, dtype, seed):
    rng = np.random.default_rng(seed)
    codes = torch.from_numpy(rng.integers(-127, 128, size=(v, k), dtype=np.int8)).to(dev)
    scales = torch.from_numpy((rng.uniform(0.5, 1.5, size=v) / 127).astype(np.float32)).to(dev)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(dev).to(dtype)
    return codes, scales, x


def _top2_with_workspace(dev, codes, scales, x, rows, start):
    nat = _nat()
    m, k = x.shape
    out_i = torch.full((m, 2), -7, dtype=torch.int32, device=dev)
    out_v = torch.full((m, 2), -7.0, dtype=torch.float32, device=dev)
    ws_bytes = int(nat.load().qs_qrow_top2_workspace_bytes(m, rows))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    nat.call("qs_qrow_top2", nat.ptr(x), nat.dtype_code(x.dtype), k, nat.ptr(codes), nat.ptr(scales),
             m, rows, k, start, nat.ptr(ws), ws_bytes, nat.ptr(out_i), nat.ptr(out_v), nat.stream_of(dev))
    return out_i, out_v


def _top2_noalloc(dev, codes, scales, x, rows, start):
    nat = _nat()
    m, k = x.shape
    out_i = torch.full((m, 2), -9, dtype=torch.int32, device=dev)
    out_v = torch.full((m, 2), -9.0, dtype=torch.float32, device=dev)
    nat.call("qs_qrow_top2_noalloc", nat.ptr(x), nat.dtype_code(x.dtype), k, nat.ptr(codes),
             nat.ptr(scales), m, rows, k, start, nat.ptr(out_i), nat.ptr(out_v), nat.stream_of(dev))
    return out_i, out_v


@pytest.mark.parametrize(
    "dtype,first,second",
    [
        # (v, k, m) of the first and the second call
        (torch.bfloat16, (151936, 1536, 2), (40000, 1536, 1)),  # register-activation search
        (torch.float32, (20000, 2048, 5), (9000, 2048, 3)),  # LDS search, several row batches
        (torch.bfloat16, (6000, 1000, 4), (3000, 1000, 2)),  # K % 16 != 0: per-element search
    ],
)
def test_noalloc_matches_workspace_entry_point(dev, dtype, first, second):
    for seed, (v, k, m) in enumerate((first, second)):
        codes, scales, x = _operands(dev, v, k, m, dtype, seed=100 + seed)
        rows, start = v - 5, 3 + seed
        ri, rv = _top2_with_workspace(dev, codes, scales, x, rows, start)
        ni, nv = _top2_noalloc(dev, codes, scales, x, rows, start)
        torch.cuda.synchronize()
        assert torch.equal(ni, ri), (v, k, m)
        assert torch.equal(nv.view(torch.int32), rv.view(torch.int32)), (v, k, m)
        assert int(ri.min()) >= start and int(ri.max()) < start + rows


def test_noalloc_rejects_sizes_beyond_scratch(dev):
    nat = _nat()
    limit = 4 << 20
    v, k = 151936, 1536
    m = 7  # 7 x ceil(151936 / 4) x 16 bytes > 4 MiB
    assert int(nat.load().qs_qrow_top2_workspace_bytes(m, v)) > limit
    codes, scales, x = _operands(dev, 64, k, m, torch.bfloat16, seed=1)
    out_i = torch.empty((m, 2), dtype=torch.int32, device=dev)
    out_v = torch.empty((m, 2), dtype=torch.float32, device=dev)
    # the size check runs before any launch, so the small operand buffers are never read
    with pytest.raises(ValueError, match="scratch"):
        nat.call("qs_qrow_top2_noalloc", nat.ptr(x), nat.dtype_code(x.dtype), k, nat.ptr(codes),
                 nat.ptr(scales), m, v, k, 0, nat.ptr(out_i), nat.ptr(out_v), nat.stream_of(dev))
