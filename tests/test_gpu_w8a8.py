"""GPU parity of the W8A8 kernels against the CPU oracle (through the C ABI)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import qrow as oq
from oracle import w8a8 as ow

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
BF16_TOL = 1e-3


def _w():
    from mrun_pub_amd import w8a8

    return w8a8


def _weights(out, inn, seed):
    rng = np.random.default_rng(seed)
    q_w = rng.integers(-127, 128, size=(out, inn), dtype=np.int8)
    sc_w = (rng.uniform(0.5, 1.5, size=out) / 127).astype(np.float32)
    return rng, q_w, sc_w


@pytest.mark.parametrize(
    "t,n,k",
    [
        (512, 1024, 4096),
        (96, 640, 384),
        (7, 33, 80),
        (5, 3, 4),
        (300, 256, 192),
        # DMA-fed kernel edges: one and two 64-byte K steps (the copy ring runs past K),
        # and the 256 x 256 tiles with ragged M and N; K % 128 == 0 takes the 128-byte-step
        # kernel (one pair at K = 128, two at K = 256)
        (40, 200, 64),
        (260, 130, 128),
        (1030, 8200, 64),
        (1030, 8200, 256),
        # long K: 112 pairs of the copy ring, sums up to 14336 * 128 * 128 (below 2^31)
        (64, 512, 14336),
        (3, 300, 8192 + 64),
        # few rows: 128 x 128, 128 x 64 and 64 x 64 tiles (ragged M and N)
        (200, 8200, 256),
        (100, 1000, 384),
        (40, 5000, 128),
    ],
)
def test_int8_gemm_int32_bit_exact(dev, t, n, k):
    rng = np.random.default_rng(t + n + k)
    qx = rng.integers(-128, 128, size=(t, k), dtype=np.int8)
    qw = rng.integers(-128, 128, size=(n, k), dtype=np.int8)
    acc = _w()._int8_gemm(torch.from_numpy(qx).to(dev), torch.from_numpy(qw).to(dev))
    assert acc.dtype == torch.int32
    assert np.array_equal(acc.cpu().numpy(), ow.int8_gemm(qx, qw))


def test_int8_gemm_extreme_values(dev):
    qx = np.full((64, 4096), 127, np.int8)
    qw = np.full((128, 4096), -127, np.int8)
    qw[1] = 127
    acc = _w()._int8_gemm(torch.from_numpy(qx).to(dev), torch.from_numpy(qw).to(dev)).cpu().numpy()
    assert (acc[:, 0] == -4096 * 127 * 127).all() and (acc[:, 1] == 4096 * 127 * 127).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("t,k", [(33, 4096), (9, 4100), (3, 20000), (5, 8), (70, 8192)])
def test_act_quant_bit_exact(dev, dtype, t, k):
    # wave-per-row kernel (K % chunk == 0, K within the register budget) and the
    # workgroup-per-row kernel for the rest
    rng = np.random.default_rng(3)
    x = rng.standard_normal((t, k)).astype(np.float32)
    x[0] = 0.0
    x[1, :4] = [1.5, 2.5, -0.5, 127.0]
    x[min(5, t - 1), 7] = 2000.0
    xt = torch.from_numpy(x).to(dtype)
    xs = xt.float().numpy()
    keep = np.ones(k, np.float32)
    keep[[7, k // 2]] = 0.0
    for kp in (None, keep):
        q, s = _w().quantize_activation(xt.to(dev), None if kp is None else torch.from_numpy(kp).to(dev))
        qr, sr = ow.act_quant(xs, kp)
        assert np.array_equal(q.cpu().numpy(), qr)
        assert np.array_equal(s.cpu().numpy().view(np.uint32), sr.view(np.uint32))


@pytest.mark.parametrize(
    "t,k,kk",
    [(64, 4096, 8), (130, 512, 4), (3, 20000, 5), (1, 64, 64), (700, 1000, 13), (9, 12000, 16), (2, 4097, 16),
     (4, 70, 16), (1, 16, 16), (33, 16384, 17)],
)
def test_outlier_topk_matches_oracle(dev, t, k, kk):
    from mrun_pub_amd import _native as nat

    rng = np.random.default_rng(t + k)
    x = rng.standard_normal((t, k)).astype(np.float32)
    x[:, rng.permutation(k)[: kk // 2 + 1]] *= 50.0
    x[0, 1] = x[0, 2] = x[-1, min(40, k - 1)] = 1000.0  # ties resolve to the lower column
    xd = torch.from_numpy(x).to(dev)
    colmax = torch.empty(k, dtype=torch.float32, device=dev)
    idx = torch.empty(kk, dtype=torch.int64, device=dev)
    keep = torch.empty(k, dtype=torch.float32, device=dev)
    nat.call("qs_outlier_topk", nat.ptr(xd), nat.QS_F32, k, t, k, kk, nat.ptr(colmax), nat.ptr(idx),
             nat.ptr(keep), nat.stream_of(dev))
    ref = ow.protect_topk(x, kk)
    assert idx.cpu().numpy().tolist() == ref.tolist()
    kref = np.ones(k, np.float32)
    kref[ref] = 0.0
    assert np.array_equal(keep.cpu().numpy(), kref)
    assert np.array_equal(colmax.cpu().numpy(), np.abs(x).max(axis=0))


@pytest.mark.parametrize("k,kk", [(4096, 8), (10000, 16), (300, 3)])
def test_outlier_topk_all_ties(dev, k, kk):
    """Every column has the same maximum: the lowest kk column indices, in order."""
    from mrun_pub_amd import _native as nat

    x = np.ones((3, k), np.float32)
    xd = torch.from_numpy(x).to(dev)
    colmax = torch.empty(k, dtype=torch.float32, device=dev)
    idx = torch.empty(kk, dtype=torch.int64, device=dev)
    keep = torch.empty(k, dtype=torch.float32, device=dev)
    nat.call("qs_outlier_topk", nat.ptr(xd), nat.QS_F32, k, 3, k, kk, nat.ptr(colmax), nat.ptr(idx),
             nat.ptr(keep), nat.stream_of(dev))
    assert idx.cpu().numpy().tolist() == list(range(kk)) == ow.protect_topk(x, kk).tolist()
    assert keep.cpu().numpy()[:kk].sum() == 0 and keep.cpu().numpy()[kk:].min() == 1.0


@pytest.mark.parametrize("t", [1, 17, 512])
def test_w8a8_no_protection_bit_exact(dev, t):
    rng, q_w, sc_w = _weights(1536, 1024, t)
    x = rng.standard_normal((t, 1024)).astype(np.float32)
    y = _w().w8a8_matmul(torch.from_numpy(q_w).to(dev), torch.from_numpy(sc_w).to(dev), torch.from_numpy(x).to(dev))
    assert np.array_equal(y.cpu().numpy().view(np.uint32), ow.w8a8_matmul(q_w, sc_w, x).view(np.uint32))


@pytest.mark.parametrize("t,n", [(300, 1000), (17, 640), (1030, 8200), (2048, 2048)])
def test_w8a8_bf16_out_bit_exact(dev, t, n):
    """bf16 output = RNE of the bit-exact fp32 result; ragged M and N edges of both tile
    shapes (the row strips leave through LDS except at a ragged N edge)."""
    rng, q_w, sc_w = _weights(n, 512, t)
    x = rng.standard_normal((t, 512)).astype(np.float32)
    y = _w().w8a8_matmul(torch.from_numpy(q_w).to(dev), torch.from_numpy(sc_w).to(dev), torch.from_numpy(x).to(dev),
                         out_dtype=torch.bfloat16)
    ref = torch.from_numpy(ow.w8a8_matmul(q_w, sc_w, x)).to(torch.bfloat16)
    assert torch.equal(y.cpu(), ref)


@pytest.mark.parametrize("ydt", ["f32", "bf16"])
@pytest.mark.parametrize("t,n,k", [(300, 1000, 512), (300, 1004, 512), (300, 1002, 512), (1030, 8196, 256),
                                   (300, 1004, 320), (1030, 8200, 192)])
def test_gemm_epilogue_store_layouts(dev, t, n, k, ydt):
    """The epilogue stores whole row segments through LDS when the output rows are 16-byte
    aligned (N * bytes % 16 == 0 and an aligned y), 4-wide from registers when only
    N % 4 == 0, element by element otherwise; ragged M and N edges store from registers.
    Every layout, and y placed past a 16-byte boundary, gives (float(acc) * a_s) * b_s
    in fp32 (bf16: its round to nearest even) bit for bit."""
    from mrun_pub_amd import _native as nat

    g = torch.Generator(device=dev)
    g.manual_seed(t + 7 * n + k)
    qx = torch.randint(-127, 128, (t, k), dtype=torch.int8, device=dev, generator=g)
    qw = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev, generator=g)
    a_s = torch.rand(t, device=dev, generator=g) / 100 + 1e-3
    b_s = torch.rand(n, device=dev, generator=g) / 100 + 1e-3
    code = nat.QS_F32 if ydt == "f32" else nat.QS_BF16
    dt = torch.float32 if ydt == "f32" else torch.bfloat16
    # |acc| <= k * 127 * 127 < 2^24: the float64 product is the exact integer and float(acc)
    # is exact, so the reference is two fp32 products (tile shapes: 256 x 128 below M * N =
    # 1024 * 8192, 256 x 256 from there; K % 128 == 64 takes the 64-byte-step kernel, which
    # shares the epilogue)
    acc = qx.cpu().numpy().astype(np.float64) @ qw.cpu().numpy().astype(np.float64).T
    ref = (torch.from_numpy(acc.astype(np.float32)) * a_s.cpu()[:, None]) * b_s.cpu()[None, :]
    ref = ref.to(dt)
    for shift in (0, 1):
        buf = torch.full((t * n + 8,), float("nan"), dtype=dt, device=dev)
        y = buf[shift : shift + t * n].view(t, n)  # shift 1: y starts 2 or 4 bytes past alignment
        assert (y.data_ptr() % 16 == 0) == (shift == 0)
        nat.call("qs_w8a8_gemm", nat.ptr(qx), nat.ptr(a_s), nat.ptr(qw), nat.ptr(b_s), None, None, 0, nat.ptr(y),
                 code, t, n, k, nat.stream_of(dev))
        torch.cuda.synchronize()
        got = y.cpu()
        assert torch.equal(got.view(torch.int16 if ydt == "bf16" else torch.int32),
                           ref.view(torch.int16 if ydt == "bf16" else torch.int32)), (shift, t, n, k, ydt)
        assert torch.isnan(buf[:shift].float()).all() and torch.isnan(buf[shift + t * n :].float()).all()


@pytest.mark.parametrize(
    "t,n,p,ydt",
    [(300, 1000, 0, "f32"), (300, 1000, 1, "bf16"), (300, 1000, 3, "f32"), (64, 640, 8, "f32"),
     (1028, 8200, 8, "bf16"), (1028, 8200, 5, "f32"), (256, 384, 12, "f32")],
)
def test_gemm_dma_epilogue_operands_match_staged(dev, t, n, p, ydt):
    """The DMA GEMM fetches its epilogue operands (act / weight scales, and the side
    operands for P <= 8) into LDS with the main loop's copies when their row slices are
    16-byte aligned whole chunks; the same values at a 4-byte offset take the staged
    epilogue.  Both agree bit for bit, over ragged M / N edges of both tile shapes."""
    from mrun_pub_amd import _native as nat

    K = 512
    g = torch.Generator(device=dev)
    g.manual_seed(t * 31 + n + p)
    qx = torch.randint(-127, 128, (t, K), dtype=torch.int8, device=dev, generator=g)
    qw = torch.randint(-127, 128, (n, K), dtype=torch.int8, device=dev, generator=g)
    a_s = torch.rand(t, device=dev, generator=g) / 100 + 1e-3
    b_s = torch.rand(n, device=dev, generator=g) / 100 + 1e-3
    xp = torch.randn(t, max(p, 1), device=dev, generator=g)[:, :p].contiguous()
    wp = torch.randn(n, max(p, 1), device=dev, generator=g)[:, :p].contiguous()

    def shifted(a):  # same values, 4 bytes past a 16-byte boundary
        buf = torch.zeros(a.numel() + 4, dtype=a.dtype, device=dev)
        buf[1 : 1 + a.numel()] = a.reshape(-1)
        return buf[1 : 1 + a.numel()]

    code = nat.QS_F32 if ydt == "f32" else nat.QS_BF16
    dt = torch.float32 if ydt == "f32" else torch.bfloat16
    outs = []
    for ops in ((a_s, b_s, xp, wp), tuple(shifted(x) for x in (a_s, b_s, xp, wp))):
        y = torch.full((t, n), float("nan"), dtype=dt, device=dev)
        nat.call("qs_w8a8_gemm", nat.ptr(qx), nat.ptr(ops[0]), nat.ptr(qw), nat.ptr(ops[1]),
                 nat.ptr(ops[2]) if p else None, nat.ptr(ops[3]) if p else None, p, nat.ptr(y), code, t, n, K,
                 nat.stream_of(dev))
        outs.append(y)
    torch.cuda.synchronize()
    assert not torch.isnan(outs[0].float()).any()
    assert torch.equal(outs[0].view(torch.int16 if ydt == "bf16" else torch.int32),
                       outs[1].view(torch.int16 if ydt == "bf16" else torch.int32))
    # and the fp32 result is the reference formula: side + (float(acc) * a_s) * b_s
    rows = torch.arange(0, t, 37, device=dev)
    acc = (qx[rows].double() @ qw.double().T)
    ref = (acc.float() * a_s[rows, None]) * b_s[None, :]
    if p:
        ref = ref + (xp[rows].double() @ wp.double().T).float()
    assert torch.allclose(outs[0][rows].float(), ref.to(dt).float(), rtol=1e-2 if ydt == "bf16" else 1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("t,k,kk,ties", [(1, 512, 1, False), (37, 4096, 8, False), (512, 4096, 8, False),
                                         (1500, 2048, 16, False), (64, 1024, 4, False), (9, 4096, 8, True),
                                         (3, 768, 16, True)])
def test_protect_quant_equals_separate_kernels(dev, dtype, t, k, kk, ties):
    """qs_w8a8_protect_quant (column maxima, then selection + quantization + side operands in
    one launch) equals qs_outlier_topk + qs_act_quant_i8 + qs_w8a8_side_gather bit for bit,
    with an exact tie between two outlier columns, more than 1024 rows, and columns that all
    tie (the selection's many-candidates path)."""
    from mrun_pub_amd import _native as nat

    n = 300
    g = torch.Generator(device=dev)
    g.manual_seed(t + k + kk)
    x = torch.randn(t, k, device=dev, generator=g)
    x[:, torch.randint(0, k, (3,), generator=g, device=dev)] *= 20.0
    x[:, 7] = 50.0
    x[:, 9] = 50.0
    if ties:
        x = torch.where(torch.arange(t, device=dev)[:, None] % 2 == 0, 1.0, -0.5).expand(t, k).clone()
    x = x.to(dtype).contiguous()
    qw = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev, generator=g)
    sw = (torch.rand(n, device=dev, generator=g) + 0.5) / 127
    code, st = nat.dtype_code(dtype), nat.stream_of(dev)
    colmax = torch.empty(k, device=dev)
    idx = torch.empty(kk, dtype=torch.int64, device=dev)
    keep = torch.empty(k, device=dev)
    nat.call("qs_outlier_topk", nat.ptr(x), code, k, t, k, kk, nat.ptr(colmax), nat.ptr(idx), nat.ptr(keep), st)
    q1, s1 = _w().quantize_activation(x, keep)
    xp1 = torch.empty((t, kk), device=dev)
    wp1 = torch.empty((n, kk), device=dev)
    nat.call("qs_w8a8_side_gather", nat.ptr(x), code, k, nat.ptr(qw), nat.ptr(sw), nat.ptr(idx), kk, t, n, k,
             nat.ptr(xp1), nat.ptr(wp1), st)
    colws = torch.empty(((t + 1023) // 1024) * k, device=dev)
    q2 = torch.empty((t, k), dtype=torch.int8, device=dev)
    s2 = torch.empty(t, device=dev)
    xp2 = torch.empty((t, kk), device=dev)
    wp2 = torch.empty((n, kk), device=dev)
    idx2 = torch.empty(kk, dtype=torch.int64, device=dev)
    keep2 = torch.empty(k, device=dev)
    nat.call("qs_w8a8_protect_quant", nat.ptr(x), code, k, t, k, kk, nat.ptr(qw), nat.ptr(sw), n, nat.ptr(colws),
             nat.ptr(q2), nat.ptr(s2), nat.ptr(xp2), nat.ptr(wp2), nat.ptr(idx2), nat.ptr(keep2), st)
    torch.cuda.synchronize()
    assert torch.equal(idx2, idx) and torch.equal(keep2, keep)
    assert torch.equal(q2, q1) and torch.equal(s2.view(torch.int32), s1.view(torch.int32))
    assert torch.equal(xp2.view(torch.int32), xp1.view(torch.int32))
    assert torch.equal(wp2.view(torch.int32), wp1.view(torch.int32))
    # the product entry point on the fused front end equals the path with the same columns given
    if dtype != torch.float16:
        y1 = _w().w8a8_matmul(qw, sw, x, protect_k=kk)
        y2 = _w().w8a8_matmul(qw, sw, x, protect_idx=idx)
        assert torch.equal(y1.view(torch.int32), y2.view(torch.int32))


@pytest.mark.parametrize("protect_k", [4, 8, 16, 24])
def test_w8a8_outlier_protection(dev, protect_k):
    rng, q_w, sc_w = _weights(640, 4096, protect_k)
    x = rng.standard_normal((64, 4096)).astype(np.float32)
    x[:, rng.permutation(4096)[:4]] *= 20.0  # 0.1% outlier channels x20
    y = _w().w8a8_matmul(
        torch.from_numpy(q_w).to(dev), torch.from_numpy(sc_w).to(dev), torch.from_numpy(x).to(dev), protect_k=protect_k
    )
    ref = ow.w8a8_matmul(q_w, sc_w, x, protect_k=protect_k)
    assert ow.protect_topk(x, protect_k).tolist()  # same columns chosen: checked via result
    assert oq.rel_l2(y.cpu().numpy(), ref) <= F32_TOL


def test_w8a8_static_list_matches_topk(dev):
    rng, q_w, sc_w = _weights(256, 512, 9)
    x = rng.standard_normal((8, 512)).astype(np.float32)
    x[:, [3, 300, 301]] *= 300.0
    dq, ds, dx = (torch.from_numpy(a).to(dev) for a in (q_w, sc_w, x))
    idx = torch.from_numpy(ow.protect_topk(x, 4)).to(dev)
    y_static = _w().w8a8_matmul(dq, ds, dx, protect_idx=idx)
    y_topk = _w().w8a8_matmul(dq, ds, dx, protect_k=4)
    assert torch.equal(y_static, y_topk)


@pytest.mark.parametrize("m", [512, 2048])
def test_w8a8_prefill_config3_bf16(dev, m):
    """BASELINE config 3 shape: [M,4096] bf16 with 0.1% outliers x20, W [14336,4096]."""
    rng, q_w, sc_w = _weights(14336, 4096, m)
    x = rng.standard_normal((m, 4096)).astype(np.float32)
    x[:, rng.permutation(4096)[:4]] *= 20.0
    xb = oq.round_bf16(x)
    dq, ds = torch.from_numpy(q_w).to(dev), torch.from_numpy(sc_w).to(dev)
    dx = torch.from_numpy(xb).to(dev).to(torch.bfloat16)
    q, s = _w().quantize_activation(dx)
    qr, sr = ow.act_quant(xb)
    assert np.array_equal(q.cpu().numpy(), qr) and np.array_equal(s.cpu().numpy(), sr)
    # the oracle's int32 accumulators for every row: int8 products summed in float64 are
    # exact (|acc| <= 127 * 127 * 4096 < 2^53), checked against the integer GEMM on a sample
    acc_ref = np.rint(qr.astype(np.float64) @ q_w.astype(np.float64).T).astype(np.int64)
    rows = np.arange(0, m, 97)
    assert np.array_equal(acc_ref[rows], ow.int8_gemm(qr[rows], q_w))
    acc = _w()._int8_gemm(q, dq).cpu().numpy()
    assert np.array_equal(acc, acc_ref)
    # the fused GEMM + epilogue against the epilogue applied to the oracle's accumulators
    y = _w().w8a8_matmul(dq, ds, dx, out_dtype=torch.bfloat16)
    ref = oq.round_bf16((acc_ref.astype(np.float32) * sr[:, None]).astype(np.float32) * sc_w[None, :])
    assert np.array_equal(y.float().cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_enable_w8a8_on_dense_store(dev, tmp_path):
    from mrun_pub_amd.dense_store import DenseQStore
    from mrun_pub_amd.store import write_qstore
    from mrun_pub_amd.w8a8 import disable_w8a8, enable_w8a8

    rng, q_w, sc_w = _weights(128, 256, 21)
    d = write_qstore(tmp_path / "s", {"L0.q": (q_w, sc_w)}, {"L0.norm": np.ones(256, np.float32)})
    store = DenseQStore(d, device=dev, compute_dtype="fp32")
    x = rng.standard_normal((4, 256)).astype(np.float32)
    base = store.matmul("L0.q", torch.from_numpy(x).to(dev))
    enable_w8a8(store, protect_k=8)
    yq = store.matmul("L0.q", torch.from_numpy(x).to(dev))
    assert oq.rel_l2(yq.cpu().numpy(), ow.w8a8_matmul(q_w, sc_w, x, protect_k=8)) <= F32_TOL
    disable_w8a8(store)
    assert torch.equal(store.matmul("L0.q", torch.from_numpy(x).to(dev)), base)


def test_enable_w8a8_twice_then_disable(dev, tmp_path):
    """A second enable only changes the settings; disable restores the original matmul, and
    non-qrow blocks keep going to it while enabled."""
    from mrun_pub_amd.dense_store import DenseQStore
    from mrun_pub_amd.store import write_qstore
    from mrun_pub_amd.w8a8 import disable_w8a8, enable_w8a8

    rng, q_w, sc_w = _weights(96, 128, 22)
    d = write_qstore(tmp_path / "s", {"L0.q": (q_w, sc_w)}, {"L0.norm": np.ones(128, np.float32)})
    store = DenseQStore(d, device=dev, compute_dtype="fp32")
    x = torch.from_numpy(rng.standard_normal((3, 128)).astype(np.float32)).to(dev)
    base = store.matmul("L0.q", x)
    enable_w8a8(store, protect_k=8)
    enable_w8a8(store, protect_k=4)
    y4 = store.matmul("L0.q", x)
    assert oq.rel_l2(y4.cpu().numpy(), ow.w8a8_matmul(q_w, sc_w, x.cpu().numpy(), protect_k=4)) <= F32_TOL
    with pytest.raises(ValueError, match="not a qrow block"):
        store.matmul("L0.norm", x)  # routed to the original matmul, which refuses fp32 blocks
    disable_w8a8(store)
    assert "matmul" not in vars(store)
    assert torch.equal(store.matmul("L0.q", x), base)
    disable_w8a8(store)  # no-op


@pytest.mark.parametrize("m", [512, 2048])
def test_w8a8_protect8_config3(dev, m):
    """The bench's ``w8a8_matmul_protect8`` call at config-3 size: bf16 x [M,4096] with 0.1%
    outlier channels x20, W [14336,4096], protect_k=8 (the reference's default for
    ``enable_w8a8``, w8a8.py:130-160).  fp32 output within 1e-5 of the oracle; the bf16
    output is that value rounded once (1e-3)."""
    rng, q_w, sc_w = _weights(14336, 4096, 300 + m)
    x = rng.standard_normal((m, 4096)).astype(np.float32)
    x[:, rng.permutation(4096)[:4]] *= 20.0
    xb = oq.round_bf16(x)
    dq, ds = torch.from_numpy(q_w).to(dev), torch.from_numpy(sc_w).to(dev)
    dx = torch.from_numpy(xb).to(dev).to(torch.bfloat16)
    ref = ow.w8a8_matmul(q_w, sc_w, xb, protect_k=8)
    y = _w().w8a8_matmul(dq, ds, dx, protect_k=8)
    assert y.dtype == torch.float32 and y.shape == (m, 14336)
    err = oq.rel_l2(y.cpu().numpy(), ref)
    assert err <= F32_TOL, err
    yb = _w().w8a8_matmul(dq, ds, dx, protect_k=8, out_dtype=torch.bfloat16)
    err = oq.rel_l2(yb.float().cpu().numpy(), oq.round_bf16(ref))
    assert err <= 1e-3, err
    # protection matters at this size: without it the error is far larger
    y0 = _w().w8a8_matmul(dq, ds, dx)
    assert oq.rel_l2(y0.cpu().numpy(), ref) > 10 * F32_TOL
