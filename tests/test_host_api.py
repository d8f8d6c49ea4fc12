"""Host-side API behaviour that needs no device: the W8A8 store binding, route-index range
checks on host tensors, embedding row-id normalisation."""

from __future__ import annotations

import numpy as np
import pytest
import torch


class _FakeStore:
    """A store with the two methods enable_w8a8 needs; only non-qrow blocks are called
    here, so no device work happens."""

    def __init__(self):
        self.calls = []

    def block_kind(self, name):
        return "fp32" if name.endswith("norm") else "qrow"

    def compact_page(self, name):  # pragma: no cover - qrow path not exercised on CPU
        raise AssertionError("qrow path needs a device")

    def matmul(self, name, x):
        self.calls.append(name)
        return x


def test_w8a8_binding_enable_twice_and_disable():
    from mrun_pub_amd.w8a8 import disable_w8a8, enable_w8a8

    st = _FakeStore()
    enable_w8a8(st, protect_k=8)
    first = vars(st)["matmul"]
    enable_w8a8(st, protect_k=2, protect_lists={"a": [1]})
    assert vars(st)["matmul"] is first  # no second wrapper around the first
    assert first.protect_k == 2 and first.protect_lists == {"a": [1]}
    x = torch.ones(2)
    assert st.matmul("l0.norm", x) is x and st.calls == ["l0.norm"]
    disable_w8a8(st)
    assert "matmul" not in vars(st) and "_w8a8_binding" not in vars(st)
    assert st.matmul("l0.norm", x) is x and st.calls == ["l0.norm", "l0.norm"]
    disable_w8a8(st)  # no-op when not enabled


def test_w8a8_binding_restores_an_instance_matmul():
    from mrun_pub_amd.w8a8 import disable_w8a8, enable_w8a8

    st = _FakeStore()

    def own(name, x):
        return None

    st.matmul = own
    enable_w8a8(st)
    disable_w8a8(st)
    assert vars(st)["matmul"] is own


def test_w8a8_binding_needs_store_methods():
    from mrun_pub_amd.w8a8 import enable_w8a8

    with pytest.raises(TypeError, match="compact_page"):
        enable_w8a8(object())


@pytest.mark.parametrize("bad", [-1, 16])
def test_route_rejects_out_of_range_host_indices(bad):
    from mrun_pub_amd import moe

    idx = torch.tensor([[0, 3], [bad, 2]], dtype=torch.int64)
    w = torch.ones(2, 2)
    with pytest.raises(ValueError, match="top_indices must lie in"):
        moe.grouped_route_tensors(idx, w, num_experts=16)


def test_row_id_normalisation():
    from mrun_pub_amd.qrow import normalize_row_ids

    flat, shape = normalize_row_ids(np.array([[0, -1], [3, -4]]), 4)
    assert shape == (2, 2) and flat.tolist() == [[0, 3], [3, 0]]
    with pytest.raises(IndexError):
        normalize_row_ids([4], 4)
    with pytest.raises(IndexError):
        normalize_row_ids([-5], 4)
    with pytest.raises(TypeError):
        normalize_row_ids([0.5], 4)
