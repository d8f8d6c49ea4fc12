"""Device stores over the store fixtures the reference's own code wrote or sealed
(tests/golden/refstore/, tests/golden/make_golden.py): weight / embed_rows / matmul equal
what the reference's QStore returned for the same files."""

from __future__ import annotations

import shutil
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import qrow as oq

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"
F32_TOL = 1e-5


def _g():
    return np.load(GOLD / "refstore.npz", allow_pickle=False)


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("kind", ["dense", "dense_resident", "paged"])
def test_reference_layout_store_on_device(dev, tmp_path, kind):
    from mrun_pub_amd.dense_store import DenseQStore
    from mrun_pub_amd.paged import PagedQStore

    g = _g()
    d = tmp_path / "legacy"
    shutil.copytree(GOLD / "refstore" / "legacy", d)
    if kind == "paged":
        st = PagedQStore(d, device=dev, compute_dtype="fp32", slots=2)
    else:
        st = DenseQStore(d, device=dev, compute_dtype="fp32")
        if kind == "dense_resident":
            st.prepare_fully_resident()
    ids = g["legacy_ids"]
    x = torch.from_numpy(g["legacy_x"]).to(dev)
    for name in ("L0.q", "L0.up"):
        assert np.array_equal(_bits(st.weight(name).cpu().numpy()), _bits(g[f"legacy_weight_{name}"]))
        e = st.embed_rows(name, ids)
        assert e.dtype == torch.float32 and tuple(e.shape) == (*ids.shape, 16)
        assert np.array_equal(_bits(e.cpu().numpy()), _bits(g[f"legacy_embed_{name}"]))
        y = st.matmul(name, x).cpu().numpy()
        assert oq.rel_l2(y, g[f"legacy_matmul_{name}"]) <= F32_TOL
    with pytest.raises(IndexError):
        st.embed_rows("L0.q", np.array([32]))
    st.close()


def test_reference_layout_store_bf16_weight(dev, tmp_path):
    from mrun_pub_amd.dense_store import DenseQStore

    g = _g()
    shutil.copytree(GOLD / "refstore" / "legacy", tmp_path / "legacy")
    st = DenseQStore(tmp_path / "legacy", device=dev, compute_dtype="bf16")
    w = st.weight("L0.up")
    assert w.dtype == torch.bfloat16
    assert np.array_equal(_bits(w.float().cpu().numpy()), _bits(g["legacy_weight_bf16_L0.up"]))
    # embed_rows keeps the reference's fp32 qrow contract whatever the compute dtype
    assert st.embed_rows("L0.up", np.array([1, 2])).dtype == torch.float32


def test_reference_sealed_v3_store_on_device(dev, tmp_path):
    from mrun_pub_amd.dense_store import DenseQStore

    g = _g()
    shutil.copytree(GOLD / "refstore" / "v3", tmp_path / "v3")
    st = DenseQStore(tmp_path / "v3", device=dev, compute_dtype="fp32")
    assert st.reader.content_identity_verified
    assert np.array_equal(_bits(st.weight("lm_head").cpu().numpy()), _bits(g["v3_weight_lm_head"]))
    assert np.array_equal(_bits(st.weight("L0.down").cpu().numpy()), _bits(g["v3_weight_L0.down"]))
    y = st.matmul("L0.gate", torch.from_numpy(g["v3_x"]).to(dev)).cpu().numpy()
    assert oq.rel_l2(y, g["v3_matmul_L0.gate"]) <= F32_TOL
    assert np.array_equal(st.fp32("L0.norm").cpu().numpy(), g["v3_fp32_L0.norm"])
    assert st.block_kind("lm_head") == "qrow" and st.block_kind("L0.norm") == "fp32"


@pytest.mark.parametrize("n,k", [(300, 1536), (77, 1000), (5, 16)])
def test_embed_rows_gather_dequant(dev, n, k):
    """qs_qrow_dequant_rows: both kernels (K % 16 == 0 and any K) against the closed form."""
    from mrun_pub_amd import qrow

    rng = np.random.default_rng(n + k)
    codes = rng.integers(-128, 128, size=(n, k), dtype=np.int8)
    scales = (rng.uniform(0.5, 1.5, n) / 127).astype(np.float32)
    ids = rng.integers(-n, n, size=(4, 7))
    e = qrow.qrow_embed_rows(torch.from_numpy(codes).to(dev), torch.from_numpy(scales).to(dev), ids)
    ref = oq.dequant_qrow(codes, scales)[ids]
    assert np.array_equal(_bits(e.cpu().numpy()), _bits(ref))
    empty = qrow.qrow_embed_rows(torch.from_numpy(codes).to(dev), torch.from_numpy(scales).to(dev),
                                 np.zeros((0,), np.int64))
    assert tuple(empty.shape) == (0, k)
