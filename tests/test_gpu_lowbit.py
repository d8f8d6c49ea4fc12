"""GPU parity of the packed int3/int2 kernels against the CPU oracle (through the C ABI)."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from oracle import lowbit as ol
from oracle import qrow as oq

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5


def _lb():
    from mrun_pub_amd import lowbit

    return lowbit


def _page(dev, packed, scales, K, bits, G, zeros=None):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    return _lb().LowbitPage("w", bits, G, K, t(packed), t(scales), None if zeros is None else t(zeros))


def _sym(rng, N, K, bits, G=128):
    codes = rng.integers(1 if bits == 3 else 0, 8 if bits == 3 else 3, size=(N, K), dtype=np.uint8)
    scales = rng.uniform(0.001, 0.02, size=(N, K // G)).astype(np.float32)
    return ol.pack_codes(codes, bits), scales


def _asym(rng, N, K, bits, G=64):
    lvl = (1 << bits) - 1
    codes = rng.integers(0, lvl + 1, size=(N, K), dtype=np.uint8)
    s = (rng.uniform(0.5, 1.5, size=(N, K // G)) / lvl).astype(np.float16)
    z = rng.uniform(0, lvl, size=(N, K // G)).astype(np.float16)
    return ol.pack_codes(codes, bits), s, z


@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("K,G", [(17, 4), (256, 128), (192, 64)])
def test_dequant_bit_exact(dev, bits, K, G):
    rng = np.random.default_rng(bits * K)
    W = rng.standard_normal((9, K)).astype(np.float32)
    packed, scales = (ol.quant_row_int3 if bits == 3 else ol.quant_row_int2)(W, G=G)
    got = _lb().lowbit_dequant(_page(dev, packed, scales, K, bits, G)).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ol.dequant(packed, scales, K, bits, G).view(np.uint32))


@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("N,K", [(33, 256), (1030, 4160)])
def test_dequant_asym_bit_exact(dev, bits, N, K):
    """(1030, 4160): many workgroups, rows of 1040 four-code pieces across their boundaries."""
    rng = np.random.default_rng(bits + N)
    packed, s, z = _asym(rng, N, K, bits)
    got = _lb().lowbit_dequant(_page(dev, packed, s, K, bits, 64, z)).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ol.dequant(packed, s, K, bits, 64, zeros=z).view(np.uint32))


@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("N,K", [(11008, 4096), (4096, 11008), (40, 384)])
@pytest.mark.parametrize("m", [1, 2, 8])
def test_gemv_asym_g64_bf16_config5(dev, bits, N, K, m):
    """G=64 asymmetric fp16 scale/zero, bf16 activations [1..8, K]."""
    rng = np.random.default_rng(bits + N + m)
    packed, s, z = _asym(rng, N, K, bits)
    x = oq.round_bf16(rng.standard_normal((m, K)).astype(np.float32))
    y = _lb().lowbit_matmul(_page(dev, packed, s, K, bits, 64, z), torch.from_numpy(x).to(dev).to(torch.bfloat16))
    assert y.dtype == torch.float32 and y.shape == (m, N)
    ref = ol.lowbit_matmul(packed, s, x, K, bits, 64, zeros=z)
    assert oq.rel_l2(y.cpu().numpy(), ref) <= F32_TOL


@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("m", [1, 3, 7, 20])
def test_gemv_reference_layout(dev, bits, xdt, m):
    """Reference layout: symmetric codes, fixed offset, fp32 scales, G=128; fp32 output."""
    rng = np.random.default_rng(bits * 100 + m)
    N, K = 1000, 1024
    packed, scales = _sym(rng, N, K, bits)
    x = rng.standard_normal((m, K)).astype(np.float32)
    xt = torch.from_numpy(x).to(xdt)
    y = _lb().lowbit_matmul(_page(dev, packed, scales, K, bits, 128), xt.to(dev))
    ref = ol.lowbit_matmul(packed, scales, xt.float().numpy(), K, bits, 128)
    assert oq.rel_l2(y.cpu().numpy(), ref) <= F32_TOL


@pytest.mark.parametrize("bits,K", [(3, 320), (2, 320), (3, 64), (2, 8192), (2, 16384), (2, 24576), (3, 12288)])
@pytest.mark.parametrize("m", [1, 2, 5])
def test_gemv_odd_layouts(dev, bits, K, m):
    """Rows that are not 16-byte multiples (int3 K=320: 120-byte rows) take the unstaged
    kernel; the rest exercise partial chunks and K splits of the staged kernel, and at
    M <= 2 the decode kernel's 1, 2, 4 and 6 pieces per lane."""
    rng = np.random.default_rng(bits * K + m)
    packed, s, z = _asym(rng, 77, K, bits)
    x = oq.round_bf16(rng.standard_normal((m, K)).astype(np.float32))
    for xdt in (torch.bfloat16, torch.float32):
        y = _lb().lowbit_matmul(_page(dev, packed, s, K, bits, 64, z), torch.from_numpy(x).to(dev).to(xdt))
        ref = ol.lowbit_matmul(packed, s, x, K, bits, 64, zeros=z)
        assert oq.rel_l2(y.cpu().numpy(), ref) <= F32_TOL


def test_rows_independent_of_batch(dev):
    rng = np.random.default_rng(9)
    packed, s, z = _asym(rng, 512, 1024, 3)
    x = torch.from_numpy(rng.standard_normal((8, 1024)).astype(np.float32)).to(dev).to(torch.bfloat16)
    page = _page(dev, packed, s, 1024, 3, 64, z)
    full = _lb().lowbit_matmul(page, x, row_stable=True)
    for r in (0, 3, 7):
        assert torch.equal(_lb().lowbit_matmul(page, x[r : r + 1])[0], full[r])
    for xdt in (torch.float32, torch.bfloat16):  # batched rows agree within tolerance too
        xb = x.to(xdt)
        ref = _lb().lowbit_matmul(page, xb, row_stable=True)
        assert oq.rel_l2(_lb().lowbit_matmul(page, xb).cpu().numpy(), ref.cpu().numpy()) <= F32_TOL


def test_reference_store_reader(dev, tmp_path):
    # the same on-disk layout the reference's QStoreInt3 test writes (test_qstore_int3.py:24-56)
    import json

    rng = np.random.default_rng(1)
    W = rng.standard_normal((70, 256)).astype(np.float32)
    packed, scales = ol.quant_row_int3(W, G=128)
    d = tmp_path / "toy-int3"
    d.mkdir()
    (d / "weights.i3").write_bytes(packed.tobytes())
    (d / "scales.f32").write_bytes(scales.tobytes())
    (d / "extras.f32").write_bytes(np.zeros(1, np.float32).tobytes())
    (d / "manifest.json").write_text(json.dumps({
        "model_name": "toy", "arch": "qwen2", "dtype": "int3", "group_size": 128, "config": {},
        "blocks": {"W": {"kind": "qrow3", "shape": [70, 256], "w_off": 0, "row_bytes": packed.shape[1],
                         "s_off": 0, "n_groups": scales.shape[1], "group_size": 128},
                   "W2": {"alias": "W"}}}))
    store = _lb().DeviceLowbitQStore(d, device=dev)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    y = store.matmul("W2", torch.from_numpy(x).to(dev))
    assert oq.rel_l2(y.cpu().numpy(), ol.lowbit_matmul(packed, scales, x, 256, 3, 128)) <= F32_TOL
    full = ol.dequant(packed, scales, 256, 3, 128)
    assert np.array_equal(store.weight("W").cpu().numpy(), full)
    # embed_rows (qstore.py:1382-1395): any id shape, negative ids from the end
    ids = np.array([[0, 69, -1], [5, 5, 33]])
    e = store.embed_rows("W2", ids)
    assert e.shape == (2, 3, 256) and e.dtype == torch.float32
    assert np.array_equal(e.cpu().numpy(), full[ids])
    with pytest.raises(IndexError):
        store.embed_rows("W", np.array([70]))


# the single-launch multi-row kernel: one wave per workgroup (K = 256), both group-count
# forms (K = 4096 / 11008), M from 3 to 16 and M > 16 (chunks of 16 rows), N not a
# multiple of the 32-row tile; K = 320 (odd group count) takes the other kernels
@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("N,K", [(80, 256), (100, 4096), (72, 11008), (40, 320)])
@pytest.mark.parametrize("m", [3, 16, 21])
def test_gemv_multirow_bf16(dev, bits, N, K, m):
    rng = np.random.default_rng(bits * 7 + N + m)
    packed, s, z = _asym(rng, N, K, bits)
    x = oq.round_bf16(rng.standard_normal((m, K)).astype(np.float32))
    y = _lb().lowbit_matmul(_page(dev, packed, s, K, bits, 64, z), torch.from_numpy(x).to(dev).to(torch.bfloat16))
    ref = ol.lowbit_matmul(packed, s, x, K, bits, 64, zeros=z)
    assert oq.rel_l2(y.cpu().numpy(), ref) <= F32_TOL


@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("m", [4, 9])
def test_gemv_multirow_reference_layout_g128(dev, bits, m):
    """fp32 scales with the fixed offset, G = 128 (both row-tile forms: K = 1024 / 16384)."""
    for K in (1024, 16384):
        rng = np.random.default_rng(bits * 11 + m + K)
        packed, scales = _sym(rng, 96, K, bits)
        x = oq.round_bf16(rng.standard_normal((m, K)).astype(np.float32))
        y = _lb().lowbit_matmul(_page(dev, packed, scales, K, bits, 128), torch.from_numpy(x).to(dev).to(torch.bfloat16))
        ref = ol.lowbit_matmul(packed, scales, x, K, bits, 128)
        assert oq.rel_l2(y.cpu().numpy(), ref) <= F32_TOL


@pytest.mark.parametrize("bits", [3, 2])
@pytest.mark.parametrize("cache_mb", [None, 0.0, 0.01])
def test_reference_store_matches_the_reference_reader(dev, bits, cache_mb):
    """The reference's own QStoreInt3 / QStoreInt2 on a reference-layout store
    (tests/golden/lowbit_store.npz, 24-row matmul chunks, an fp32 extras block, an alias)
    against the device reader with every block resident (``cache_mb=None``), every block
    streamed in 24-row chunks (0), and the first block resident and the second streamed
    (0.01 MB holds A only).  Products within 1e-5, rows, fp32 blocks and the dequantized
    weight bit for bit; a streamed block equals the resident one within the same bound."""
    from pathlib import Path

    gold = Path(__file__).resolve().parent / "golden"
    g = np.load(gold / "lowbit_store.npz", allow_pickle=False)
    d = gold / "lowbit_store" / f"toy-int{bits}"
    store = _lb().DeviceLowbitQStore(d, device=dev, cache_mb=cache_mb)
    resident = _lb().DeviceLowbitQStore(d, device=dev)
    t = f"i{bits}"
    x = torch.from_numpy(g["x"]).to(dev)
    for name in ("A", "B"):
        y = store.matmul(name, x)
        assert oq.rel_l2(y.cpu().numpy(), g[f"{t}_{name}_matmul"]) <= F32_TOL
        yr = store.matmul_row_stable(name, x)
        assert oq.rel_l2(yr.cpu().numpy(), g[f"{t}_{name}_row_stable"]) <= F32_TOL
        for r in range(3):  # row-stable rows equal single-row products
            assert torch.equal(yr[r], store.matmul_row_stable(name, x[r:r + 1])[0])
        assert oq.rel_l2(y.cpu().numpy(), resident.matmul(name, x).cpu().numpy()) <= F32_TOL
        man = json.loads((d / "manifest.json").read_text())["blocks"][name]
        packed = np.fromfile(d / f"weights.i{bits}", dtype=np.uint8)[man["w_off"]:]
        out = man["shape"][0]
        packed = packed[: out * man["row_bytes"]].reshape(out, man["row_bytes"])
        sc = np.fromfile(d / "scales.f32", dtype=np.float32)[man["s_off"] // 4:][: out * man["n_groups"]]
        full = ol.dequant(packed, sc.reshape(out, man["n_groups"]), 320, bits, 128)
        assert np.array_equal(store.weight(name).cpu().numpy(), full)
        blocks = list(store.row_blocks(name, bs=16))
        assert [(a, b) for a, b, _ in blocks] == [(a, min(a + 16, out)) for a in range(0, out, 16)]
        assert np.array_equal(torch.cat([w for _, _, w in blocks]).cpu().numpy(), full)
    e = store.embed_rows("A2", g["ids"])
    assert np.array_equal(e.cpu().numpy(), g[f"{t}_A2_embed"])
    assert np.array_equal(store.fp32("norm").cpu().numpy(), g[f"{t}_norm"])
    streamed = {None: 0, 0.0: 2, 0.01: 1}[cache_mb]
    assert store.stats["resident_blocks"] == 2 - streamed
    if streamed:
        assert store.stats["streamed_chunks"] > store.stats["streamed_calls"] > 0
    store.close()
    resident.close()


@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("K,G", [(17, 4), (320, 128), (100, 32), (200, 64), (1000, 128), (77, 77)])
@pytest.mark.parametrize("m", [1, 3, 11])
def test_gemv_any_layout(dev, bits, K, G, m):
    """Layouts the tiled kernels refuse -- group sizes other than 64 / 128, a short last
    group (scales [N, ceil(K/G)]), rows that are not 4-byte multiples -- in the reference's
    symmetric layout (fixed offset, fp32 scales) and the asymmetric one (fp16 scale + zero),
    more than eight activation rows included, against the oracle."""
    rng = np.random.default_rng(bits * 1000 + K + G + m)
    N, ng = 45, -(-K // G)
    codes = rng.integers(0, 1 << bits, size=(N, K), dtype=np.uint8)
    packed = ol.pack_codes(codes, bits)
    scales = rng.uniform(0.001, 0.02, size=(N, ng)).astype(np.float32)
    s16 = (rng.uniform(0.5, 1.5, size=(N, ng)) / 7).astype(np.float16)
    z16 = rng.uniform(0, (1 << bits) - 1, size=(N, ng)).astype(np.float16)
    x = oq.round_bf16(rng.standard_normal((m, K)).astype(np.float32))
    for xdt in (torch.bfloat16, torch.float32):
        xd = torch.from_numpy(x).to(dev).to(xdt)
        y = _lb().lowbit_matmul(_page(dev, packed, scales, K, bits, G), xd)
        assert oq.rel_l2(y.cpu().numpy(), ol.lowbit_matmul(packed, scales, x, K, bits, G)) <= F32_TOL
        y = _lb().lowbit_matmul(_page(dev, packed, s16, K, bits, G, z16), xd)
        assert oq.rel_l2(y.cpu().numpy(), ol.lowbit_matmul(packed, s16, x, K, bits, G, zeros=z16)) <= F32_TOL
