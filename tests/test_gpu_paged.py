"""Resident (DenseQStore) and paged (pinned host -> HBM ring) stores on the GPU.

Mirrors the reference ring contract (tests/test_ring_and_host_tier.py:321-335 in the
reference: ring results equal the plain paged path bit for bit, and the ring hits) and
checks both stores against the CPU oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import qrow as oq

pytestmark = pytest.mark.gpu

SHAPES = {  # a miniature decoder layer pair; K=80 exercises the non-MFMA kernels
    "l0.q": (192, 256), "l0.k": (64, 256), "l0.v": (64, 256), "l0.o": (256, 192),
    "l0.gate": (384, 256), "l0.up": (384, 256), "l0.down": (256, 384),
    "l1.q": (192, 256), "l1.gate": (384, 256), "l1.up": (384, 256), "l1.down": (256, 384),
    "odd": (33, 80),
}


@pytest.fixture(scope="module")
def store_dir(tmp_path_factory):
    from mrun_pub_amd.store import write_qstore

    rng = np.random.default_rng(7)
    blocks = {
        n: (rng.integers(-127, 128, size=s, dtype=np.int8), (rng.uniform(0.5, 1.5, s[0]) / 127).astype(np.float32))
        for n, s in SHAPES.items()
    }
    d = tmp_path_factory.mktemp("qs")
    write_qstore(d, blocks, {"norm": np.ones(256, np.float32)}, aliases={"lm_head": "l0.q"})
    return d, blocks


def _pass(store, xs):
    """One decode-style pass touching every block in a fixed order."""
    out = []
    for layer in ("l0", "l1"):
        out.append(store.matmul(f"{layer}.q", xs[256]))
        if layer == "l0":
            out.append(store.matmul("l0.k", xs[256]))
            out.append(store.matmul_row_stable("l0.v", xs[256]))
            out.append(store.matmul("l0.o", xs[192]))
        out.append(store.fused_swiglu(f"{layer}.gate", f"{layer}.up", xs[256])[0])
        out.append(store.matmul(f"{layer}.down", xs[384]))
    out.append(store.matmul("odd", xs[80]))
    out.append(store.weight("lm_head"))
    return out


def _inputs(dev, m, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(3)
    return {k: torch.randn(m, k, generator=g).to(dtype).to(dev) for k in (80, 192, 256, 384)}


@pytest.mark.parametrize("m", [1, 4])
def test_dense_store_matches_oracle(dev, store_dir, m):
    from mrun_pub_amd.dense_store import DenseQStore

    d, blocks = store_dir
    xs = _inputs(dev, m)
    for resident in (False, True):
        st = DenseQStore(d, device=dev, compute_dtype="bf16", compact_cache_mb=1.0)
        if resident:
            st.prepare_fully_resident()
        y = st.matmul("l0.down", xs[384]).float().cpu().numpy()
        ref = oq.qrow_matmul_w8a16(*blocks["l0.down"], xs[384].float().cpu().numpy(), "bf16")
        assert oq.rel_l2(y, ref) <= 1e-3
        g = st.fused_swiglu("l0.gate", "l0.up", xs[256])[0].float().cpu().numpy()
        gref = oq.qrow_swiglu(*blocks["l0.gate"], *blocks["l0.up"], xs[256].float().cpu().numpy())
        assert oq.rel_l2(g, gref) <= 1e-3
        w = st.weight("lm_head").float().cpu().numpy()
        assert np.array_equal(w.view(np.uint32), oq.qrow_weight(*blocks["l0.q"], "bf16").view(np.uint32))
        np.testing.assert_array_equal(st.fp32("norm").cpu().numpy(), np.ones(256, np.float32))
        st.close()


@pytest.mark.parametrize("slots,depth", [(3, 2), (2, 1), (5, 3)])
@pytest.mark.parametrize("m", [1, 3])
def test_paged_ring_bit_exact_and_hitting(dev, store_dir, slots, depth, m):
    from mrun_pub_amd.dense_store import DenseQStore
    from mrun_pub_amd.paged import PagedQStore

    d, _ = store_dir
    xs = _inputs(dev, m)
    resident = DenseQStore(d, device=dev, compute_dtype="bf16")
    resident.prepare_fully_resident()
    plain = _pass(resident, xs)
    paged = PagedQStore(d, device=dev, compute_dtype="bf16", slots=slots, depth=depth)
    runs = [_pass(paged, xs) for _ in range(3)]
    stats = paged.ring_stats()
    paged.synchronize()
    for run in runs:
        for got, want in zip(run, plain):
            assert torch.equal(got, want), "paged ring path must equal the resident path bit for bit"
    assert stats["hits"] > 0, f"ring never hit: {stats}"
    if slots > 2:
        # pass 1: all 13 accesses miss; later passes miss only the block read twice in a row
        # (lm_head -> l0.q at a pass end, l0.q at the next start), as the reference oracle does
        assert stats["misses"] <= 13 + 2, stats
    paged.disable_ring()
    assert paged.ring_stats() is None
    for got, want in zip(_pass(paged, xs), plain):
        assert torch.equal(got, want)
    paged.close()
    resident.close()


def test_paged_fp32_compute_matches_oracle(dev, store_dir):
    from mrun_pub_amd.paged import PagedQStore

    d, blocks = store_dir
    st = PagedQStore(d, device=dev, compute_dtype="fp32")
    x = torch.randn(2, 384, generator=torch.Generator().manual_seed(1)).to(dev)
    for _ in range(2):
        y = st.matmul("l0.down", x).cpu().numpy()
        ref = oq.qrow_matmul_f32(*blocks["l0.down"], x.cpu().numpy())
        assert oq.rel_l2(y, ref) <= 1e-5
        rows = list(st.row_blocks("l0.down", bs=100))
        assert [(a, b) for a, b, _ in rows] == [(0, 100), (100, 200), (200, 256)]
        w = torch.cat([r for _, _, r in rows]).cpu().numpy()
        assert np.array_equal(w.view(np.uint32), oq.qrow_weight(*blocks["l0.down"], "fp32").view(np.uint32))
    st.close()


def test_paged_errors(dev, store_dir):
    from mrun_pub_amd.dense_store import DenseQStore
    from mrun_pub_amd.paged import PagedQStore

    d, _ = store_dir
    st = PagedQStore(d, device=dev)
    with pytest.raises(KeyError):
        st.matmul("nope", torch.zeros(1, 256, dtype=torch.bfloat16, device=dev))
    with pytest.raises(KeyError):
        st.matmul("norm", torch.zeros(1, 256, dtype=torch.bfloat16, device=dev))
    other = DenseQStore(d, device=dev).compact_page("l0.q")
    with pytest.raises(RuntimeError, match="not held"):
        st.ring.release(other)
    with pytest.raises(ValueError):  # activation width mismatch surfaces as the reference's ValueError
        st.matmul("l0.q", torch.zeros(1, 255, dtype=torch.bfloat16, device=dev))
    assert all(h == 0 for h in st.ring.held), "a failed call must release its slot"
    st.close()


def test_pager_release_many_refuses_a_slot_listed_twice(dev):
    """A release batch that names one slot twice is refused with nothing changed (its second
    reference would hand the batch's event back to the pool while the slot still waits on
    it); distinct batches keep working, and a refill of a released slot lands whole."""
    import ctypes

    from mrun_pub_amd import _native as nat

    arena = torch.zeros(4 * 4096, dtype=torch.uint8, device=dev)
    handle = ctypes.c_void_p()
    nat.call("qs_pager_create", nat.ptr(arena), 4096, 4, 4096, ctypes.byref(handle))
    try:
        stream = nat.stream_of(dev)
        with pytest.raises(ValueError, match="listed twice"):
            nat.call("qs_pager_release_many", handle, (ctypes.c_int * 3)(1, 2, 1), 3, stream)
        nat.call("qs_pager_release_many", handle, (ctypes.c_int * 2)(1, 2), 2, stream)
        nat.call("qs_pager_release_many", handle, (ctypes.c_int * 1)(1), 1, stream)
        host = torch.arange(4096, dtype=torch.int32).to(torch.uint8).pin_memory()
        for slot in (1, 2):
            nat.call("qs_pager_submit", handle, slot, host.data_ptr(), 4096, 0)
            nat.call("qs_pager_seal", handle, slot)
        nat.call("qs_pager_acquire_many", handle, (ctypes.c_int * 2)(1, 2), 2, stream)
        torch.cuda.synchronize()
        assert torch.equal(arena[4096:8192].cpu(), host) and torch.equal(arena[8192:12288].cpu(), host)
        assert not arena[:4096].any() and not arena[12288:].any()
    finally:
        nat.call("qs_pager_destroy", handle)


@pytest.mark.parametrize("buffers,slots,depth", [(3, 3, 2), (2, 2, 1), (1, 4, 3), (4, 5, 3)])
@pytest.mark.parametrize("m", [1, 4])
def test_bounded_staging_pages_a_store_larger_than_its_pinned_budget(dev, store_dir, buffers, slots, depth, m):
    """Bounded mode (``staging_buffers``): pinned memory holds ``buffers`` blocks of the
    largest size only (a fraction of the store), every transfer is re-staged from the
    store's mapping, and the results equal the resident store bit for bit -- with the ring
    hitting, after mispredicts, and with the ring off (every block a miss)."""
    from mrun_pub_amd.dense_store import DenseQStore
    from mrun_pub_amd.paged import MappedStagingTier, PagedQStore

    d, _ = store_dir
    xs = _inputs(dev, m)
    resident = DenseQStore(d, device=dev, compute_dtype="bf16")
    store_bytes = resident.prepare_fully_resident()
    plain = _pass(resident, xs)
    # small chunks so the parallel piece copy runs on these blocks too
    paged = PagedQStore(d, device=dev, compute_dtype="bf16", slots=slots, depth=depth, staging_buffers=buffers)
    assert isinstance(paged.tier, MappedStagingTier) and len(paged.tier.buffers) == buffers
    paged.tier.chunk_bytes = 16 << 10
    assert paged.tier.nbytes < store_bytes  # the store does not fit in the pinned budget
    runs = [_pass(paged, xs) for _ in range(3)]
    # a mispredicted order (reversed pass), then the learned order again
    runs.append(list(reversed(_pass_reversed(paged, xs))))
    runs.append(_pass(paged, xs))
    stats = paged.ring_stats()
    paged.synchronize()
    for run in runs:
        for got, want in zip(run, plain):
            assert torch.equal(got, want), "bounded staging must equal the resident path bit for bit"
    assert stats["hits"] > 0 and paged.tier.stats["staged_blocks"] >= stats["hits"] + stats["misses"] - 2
    paged.disable_ring()
    for got, want in zip(_pass(paged, xs), plain):
        assert torch.equal(got, want)
    paged.close()
    resident.close()


def _pass_reversed(store, xs):
    """The calls of ``_pass`` in reverse order (outputs listed in reverse)."""
    out = [store.weight("lm_head"), store.matmul("odd", xs[80])]
    for layer in ("l1", "l0"):
        out.append(store.matmul(f"{layer}.down", xs[384]))
        out.append(store.fused_swiglu(f"{layer}.gate", f"{layer}.up", xs[256])[0])
        if layer == "l0":
            out.append(store.matmul("l0.o", xs[192]))
            out.append(store.matmul_row_stable("l0.v", xs[256]))
            out.append(store.matmul("l0.k", xs[256]))
        out.append(store.matmul(f"{layer}.q", xs[256]))
    return out


def test_pager_submit_run_fills_consecutive_slots(dev):
    """``qs_pager_submit_run`` moves one contiguous host range into consecutive slots in
    transfer pieces (here 3 slots of 4096 bytes with 5000-byte pieces, so pieces straddle
    slots), seals every slot, leaves the other slots untouched, waits for a slot's previous
    consumer, and refuses a run past the last slot."""
    import ctypes

    from mrun_pub_amd import _native as nat

    arena = torch.zeros(6 * 4096, dtype=torch.uint8, device=dev)
    handle = ctypes.c_void_p()
    nat.call("qs_pager_create", nat.ptr(arena), 4096, 6, 5000, ctypes.byref(handle))
    try:
        stream = nat.stream_of(dev)
        host = (torch.arange(3 * 4096, dtype=torch.int32) % 251).to(torch.uint8).pin_memory()
        nat.call("qs_pager_release_many", handle, (ctypes.c_int * 2)(2, 3), 2, stream)  # a consumer to wait for
        nat.call("qs_pager_submit_run", handle, 1, 3, host.data_ptr())
        nat.call("qs_pager_acquire_many", handle, (ctypes.c_int * 3)(1, 2, 3), 3, stream)
        torch.cuda.synchronize()
        assert torch.equal(arena[4096:4 * 4096].cpu(), host)
        assert not arena[:4096].any() and not arena[4 * 4096:].any()
        for slot in (1, 2, 3):
            assert nat.load().qs_pager_slot_landed(handle, slot) == 1
        with pytest.raises(ValueError):
            nat.call("qs_pager_submit_run", handle, 4, 3, host.data_ptr())
        with pytest.raises(ValueError):
            nat.call("qs_pager_submit_run", handle, 0, 0, host.data_ptr())
    finally:
        nat.call("qs_pager_destroy", handle)
