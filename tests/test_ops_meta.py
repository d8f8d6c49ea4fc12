"""The qstore_hip custom operators are registered and infer output shapes and dtypes on
meta tensors (their fake implementations), with no device."""

from __future__ import annotations

import pytest
import torch

M = torch.device("meta")


def _e(*shape, dtype=torch.float32):
    return torch.empty(*shape, dtype=dtype, device=M)


@pytest.fixture(scope="module")
def ops():
    import mrun_pub_amd.ops as o

    return torch.ops.qstore_hip, o


def test_every_operator_is_registered(ops):
    q, o = ops
    for name in o.OPS:
        assert hasattr(q, name), name


def test_fake_shapes(ops):
    q, _ = ops
    c, s = _e(96, 64, dtype=torch.int8), _e(96)
    x = _e(3, 5, 64, dtype=torch.bfloat16)
    y = q.qrow_matmul(c, s, x)
    assert y.shape == (3, 5, 96) and y.dtype == torch.bfloat16
    assert q.qrow_matmul(c, s, _e(2, 64)).dtype == torch.float32
    assert q.qrow_dequant(c, s, torch.float16).dtype == torch.float16
    assert q.qrow_swiglu(c, s, c, s, x).shape == (3, 5, 96)
    i, v = q.qrow_top2(c, s, _e(4, 64, dtype=torch.bfloat16), 10, 90)
    assert i.shape == (4, 2) and i.dtype == torch.int32 and v.dtype == torch.float32
    qx, sx = q.act_quant(_e(7, 64, dtype=torch.bfloat16), None)
    assert qx.shape == (7, 64) and qx.dtype == torch.int8 and sx.shape == (7,)
    assert q.int8_gemm(_e(7, 64, dtype=torch.int8), c).dtype == torch.int32
    assert q.w8a8_matmul(c, s, _e(7, 64), None, 8, torch.bfloat16).shape == (7, 96)
    w, idx = q.moe_router(_e(10, 32), 4, True, torch.bfloat16)
    assert w.shape == (10, 4) and idx.dtype == torch.int64
    tok, coef, st, cnt, inv = q.moe_route(_e(10, 4, dtype=torch.int64), _e(10, 4, dtype=torch.bfloat16), 32)
    assert tok.shape == (40,) and coef.dtype == torch.bfloat16 and st.shape == (32,) and inv.shape == (40,)
    g = q.grouped_int8_mm(_e(40, 64, dtype=torch.int8), _e(40), _e(32, 96, 64, dtype=torch.int8), _e(32, 96),
                          _e(32, dtype=torch.int32), _e(32, dtype=torch.int32), None, 0, True, torch.bfloat16)
    assert g.shape == (40, 48)
    g16 = q.grouped_w8a16_mm(_e(10, 64, dtype=torch.bfloat16), _e(32, 96, 64, dtype=torch.int8), _e(32, 96),
                             _e(32, dtype=torch.int32), _e(32, dtype=torch.int32), _e(40, dtype=torch.int64), None,
                             0, True, torch.bfloat16)
    assert g16.shape == (40, 48) and g16.dtype == torch.bfloat16
    assert q.route_reduce(_e(40, 16), _e(40), _e(40, dtype=torch.int64), 10, 4).shape == (10, 16)
    assert q.lowbit_matmul(_e(96, 24, dtype=torch.uint8), _e(96, 1), None, _e(2, 64), 3, 64, 64).shape == (2, 96)
