"""GPU parity of the config-2 decode pass as ``bench.py`` times it, against the CPU oracle.

* The three-linear q/k/v launch (``qrow_matmul_multi`` and ``DenseQStore.matmul_multi``,
  1536 + 256 + 256 rows, K = 1536) at M in {1, 5, 16, 23, 32}: the VALU register kernels
  below 5 rows, the 16-row tiles at 5 and the batched ``k_bd2`` grid (one launch, each
  workgroup picking its linear by row tile) from 16.
* Chained decoder layers exactly as ``bench.DecodeChain.per_linear`` runs them (q/k/v ->
  o -> paired gate/up + SwiGLU -> down -> next layer), at M in {1, 4, 16, 32}: every
  launch against the oracle applied to that launch's own input, the pass end to end
  against the oracle applied in the same order, and HIP graph replays against eager.

Reference call order: the q/k/v/o and MLP calls of paged_forward.py:481-542.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import qrow as oq

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-3  # rel-L2 of one bf16 launch against the oracle on the same input
HIDDEN, KV, INTER = 1536, 256, 8960


def _qrow():
    from mrun_pub_amd import qrow

    return qrow


def _lin(rng, n, k):
    codes = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    scales = (rng.uniform(0.5, 1.5, size=n) / 127).astype(np.float32)
    return codes, scales


def _dev(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def _host(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


@pytest.mark.parametrize("m", [1, 5, 16, 23, 32])
def test_qkv_multi_launch_config2(dev, m, tmp_path):
    q = _qrow()
    rng = np.random.default_rng(100 + m)
    names = ("L0.q_proj", "L0.k_proj", "L0.v_proj")
    lins = [_lin(rng, n, HIDDEN) for n in (HIDDEN, KV, KV)]
    x = oq.round_bf16(rng.standard_normal((m, HIDDEN)).astype(np.float32))
    xd = _dev(x, dev, torch.bfloat16)
    pages = [(_dev(c, dev), _dev(s, dev)) for c, s in lins]
    outs = q.qrow_matmul_multi(pages, xd)
    batched = q._batched_eligible(xd, [c for c, _ in pages])
    assert batched == (m >= q.BATCHED_MIN_M)
    for (c, s), (dc, ds), o in zip(lins, pages, outs):
        assert o.shape == (m, c.shape[0]) and o.dtype == torch.bfloat16
        err = oq.rel_l2(_host(o), oq.qrow_matmul_w8a16(c, s, x))
        assert err <= BF16_TOL, err
        if batched:
            # one grid over three linears: each linear equals its own single-linear launch
            assert torch.equal(o, q.qrow_matmul(dc, ds, xd))
    # a row of the launch equals that row computed alone through the same kernel family
    for r in sorted({0, m // 2, m - 1}):
        if batched:
            one = [torch.empty((1, int(c.shape[0])), dtype=torch.bfloat16, device=dev) for c, _ in pages]
            q._run_batched(xd[r:r + 1].contiguous(), pages, one, swiglu=False)
        elif m <= 4:
            one = q.qrow_matmul_multi(pages, xd[r:r + 1])
        else:  # 16-row tiles: rows alone take the register kernel, so permute the others instead
            perm = torch.cat([xd[r:r + 1], xd[:r], xd[r + 1:]]).flip(0).contiguous()
            one = [o[m - 1:m] for o in q.qrow_matmul_multi(pages, perm)]
        for o1, o in zip(one, outs):
            assert torch.equal(o1[0], o[r]), r
    # the store surface: DenseQStore.matmul_multi, paged from the reader and fully resident
    from mrun_pub_amd.dense_store import DenseQStore
    from mrun_pub_amd.store import write_qstore

    d = write_qstore(tmp_path / "s", dict(zip(names, lins)), {"L0.norm": np.ones(HIDDEN, np.float32)})
    store = DenseQStore(d, device=dev, compute_dtype="bf16", compact_cache_mb=64)
    for o, so in zip(outs, store.matmul_multi(list(names), xd)):
        assert torch.equal(o, so)
    store.prepare_fully_resident()
    for o, so in zip(outs, store.matmul_multi(list(names), xd)):
        assert torch.equal(o, so)
    assert store.stats.projection_calls >= 6
    store.close()


def _layers(dev, rng, n_layers):
    import bench
    from mrun_pub_amd.qrow import CompactQRowPage

    host, pages = [], []
    for li in range(n_layers):
        h, p = {}, {}
        for name, (n, k) in bench.SHAPES.items():
            c, s = _lin(rng, n, k)
            h[name] = (c, s)
            p[name] = CompactQRowPage(f"L{li}.{name}", 0, n, k, _dev(c, dev), _dev(s, dev))
        host.append(h)
        pages.append(p)
    return host, pages


def _oracle_layer(h, x):
    """One decoder layer's linears in DecodeChain order, each a bf16 W8A16 launch."""
    qo = oq.qrow_matmul_w8a16(*h["q"], x)
    ko = oq.qrow_matmul_w8a16(*h["k"], x)
    vo = oq.qrow_matmul_w8a16(*h["v"], x)
    oo = oq.qrow_matmul_w8a16(*h["o"], qo)
    hh = oq.qrow_swiglu(*h["gate"], *h["up"], oo)
    return qo, ko, vo, oo, hh, oq.qrow_matmul_w8a16(*h["down"], hh)


def _check_launches(chain, h, x_in: np.ndarray, tag: str):
    """Every launch of the chain's last layer against the oracle on that launch's input
    (the chain's own buffers): q/k/v from the layer input, o from q, SwiGLU from o,
    down from the SwiGLU output."""
    q, k, v, o, hh = (_host(t) for t in (chain.q, chain.k, chain.v, chain.o, chain.h))
    checks = (
        ("q", q, oq.qrow_matmul_w8a16(*h["q"], x_in)),
        ("k", k, oq.qrow_matmul_w8a16(*h["k"], x_in)),
        ("v", v, oq.qrow_matmul_w8a16(*h["v"], x_in)),
        ("o", o, oq.qrow_matmul_w8a16(*h["o"], q)),
        ("swiglu", hh, oq.qrow_swiglu(*h["gate"], *h["up"], o)),
    )
    for name, got, ref in checks:
        err = oq.rel_l2(got, ref)
        assert err <= BF16_TOL, (tag, name, err)
    return hh


@pytest.mark.parametrize("m", [1, 4, 16, 32])
def test_chained_decoder_layers_config2(dev, m):
    import bench

    rng = np.random.default_rng(200 + m)
    host, pages = _layers(dev, rng, 2)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    x = oq.round_bf16(rng.standard_normal((m, HIDDEN)).astype(np.float32))
    chain = bench.DecodeChain(torch, dev, pages, m, gen)
    chain.x0.copy_(_dev(x, dev, torch.bfloat16))  # bf16-representable values: exact copy
    first = bench.DecodeChain(torch, dev, pages[:1], m, gen)
    first.x0.copy_(chain.x0)

    # layer 0 alone (a one-layer chain on the same input), launch by launch
    y0 = first.per_linear()
    hh0 = _check_launches(first, host[0], x, "layer0")
    err = oq.rel_l2(_host(y0), oq.qrow_matmul_w8a16(*host[0]["down"], hh0))
    assert err <= BF16_TOL, ("layer0 down", err)
    # the two-layer pass: its layer-0 output is the one-layer chain's, bit for bit, and
    # layer 1's launches are checked on the inputs they were given
    y = chain.per_linear()
    assert torch.equal(chain.d[0], y0)
    hh1 = _check_launches(chain, host[1], _host(chain.d[0]), "layer1")
    err = oq.rel_l2(_host(y), oq.qrow_matmul_w8a16(*host[1]["down"], hh1))
    assert err <= BF16_TOL, ("layer1 down", err)

    # end to end from the layer input, the oracle applied in the same order.  Ten chained
    # bf16 roundings separate the two: wherever the fp32 sums differ in their last bits,
    # the rounding can land one bf16 ulp (2^-8 relative) apart, and the next launch carries
    # that difference on, so the bound is a few ulps rather than the one-launch 1e-3 (on
    # these inputs the oracle chain summed in float32 instead of float64 already ends
    # 2e-3 .. 7e-3 away from itself after two layers).
    ref = x
    for h in host:
        ref = _oracle_layer(h, ref)[-1]
    err = oq.rel_l2(_host(y), ref)
    assert err <= 2e-2, err

    # the bench replays the pass as a HIP graph: every replay recomputes the eager result
    eager = y.clone()
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            out = chain.per_linear()
    torch.cuda.synchronize()
    for _ in range(3):
        for t in (chain.q, chain.k, chain.v, chain.o, chain.h, *chain.d):
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
