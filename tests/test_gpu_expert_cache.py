"""Paged experts on the device: results equal the resident backend's bit for bit."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _mods():
    from mrun_pub_amd import expert_cache, moe

    return expert_cache, moe


def _setup(tmp_path, dev, L=3, E=16, H=256, I=128, seed=0):
    ec, moe = _mods()
    rng = np.random.default_rng(seed)
    gu = rng.integers(-127, 128, size=(L, E, 2 * I, H), dtype=np.int8)
    gus = (rng.uniform(0.5, 1.5, size=(L, E, 2 * I)) / 127).astype(np.float32)
    dn = rng.integers(-127, 128, size=(L, E, H, I), dtype=np.int8)
    dns = (rng.uniform(0.5, 1.5, size=(L, E, H)) / 127).astype(np.float32)
    store = ec.PackedInt8ExpertStore(ec.write_int8_expert_store(tmp_path, gu, gus, dn, dns))
    resident = moe.Int8ExpertBackend(
        [moe.Int8ExpertLayer.from_arrays(*(torch.from_numpy(a[l]) for a in (gu, gus, dn, dns)), dev) for l in range(L)]
    )
    return store, resident


def _steps(dev, L, E, T=6, k=4, steps=4, seed=1):
    g = torch.Generator(device="cpu").manual_seed(seed)
    out = []
    for _ in range(steps):
        for layer in range(L):
            logits = torch.randn(T, E, generator=g)
            w, idx = torch.softmax(logits, -1).topk(k, -1)
            x = torch.randn(T, 256, generator=g).to(torch.bfloat16)
            out.append((layer, x.to(dev), idx.to(dev), (w / w.sum(-1, keepdim=True)).to(torch.bfloat16).to(dev)))
    return out


@pytest.mark.parametrize("tier,prefetch,policy,binding", [
    (True, False, "global-lru-v1", "slot-indirect-v1"),
    (True, True, "layer-frequency-lru-v1", "slot-indirect-v1"),
    (False, True, "global-lru-v1", "slot-indirect-v1"),
    (False, False, "layer-frequency-lru-v1", "compact-copy-v1"),
])
def test_paged_backend_equals_resident(dev, tmp_path, tier, prefetch, policy, binding):
    ec, moe = _mods()
    store, resident = _setup(tmp_path, dev)
    host = ec.HostPageTier(store, host_cache_mb=30 * store.layout.page_stride / 1e6) if tier else None
    if host is not None:
        host.warm()
    # 40 slots for 3 layers x 16 experts (about 12 routed per layer and step): hits and evictions
    cache = ec.ExpertPageCache(store, device=dev, cache_mb=40 * store.layout.page_stride / 1e6, max_active_pages=16,
                               host_tier=host, route_prefetch=prefetch, cache_policy=policy,
                               page_binding_policy=binding)
    paged = moe.Int8ExpertBackend(page_cache=cache)
    for layer, x, idx, w in _steps(dev, 3, 16):
        want = resident.moe(layer, x, idx, w)
        got = paged.moe(layer, x, idx, w)
        assert torch.equal(got, want), (layer, tier, prefetch, policy)
        if binding == "compact-copy-v1":
            sel, page = cache.acquire(layer, idx)
            assert page.gate_up.shape[0] == sel.numel()
    st = cache.stats.as_dict()
    assert st["page_misses"] > 0 and st["page_hits"] > 0 and st["evictions"] > 0
    cache.close()


def test_route_prefetch_stages_evicted_next_layer_pages(dev, tmp_path):
    """A 6-slot cache for 2 x 8 pages and at most 4 routed experts per step: the next
    layer's pages are mostly evicted, so the previous step's routes for it are staged one
    layer early (and results still match)."""
    ec, moe = _mods()
    store, resident = _setup(tmp_path, dev, L=2, E=8)
    cache = ec.ExpertPageCache(store, device=dev, cache_mb=0, max_active_pages=6, route_prefetch=True)
    paged = moe.Int8ExpertBackend(page_cache=cache)
    for layer, x, idx, w in _steps(dev, 2, 8, T=2, k=2, steps=4):
        assert torch.equal(paged.moe(layer, x, idx, w), resident.moe(layer, x, idx, w))
    assert cache.prefetch_stats["prefetched_pages"] > 0 and cache.prefetch_stats["prefetch_rounds"] > 0
    cache.close()


def test_paged_w8a16_backend_equals_resident(dev, tmp_path):
    """The weight-only flow over paged experts (slot-indirect binding, evictions) gives the
    resident weight-only flow's results bit for bit."""
    ec, moe = _mods()
    store, resident = _setup(tmp_path, dev)
    resident = moe.Int8ExpertBackend(resident.layers, w8a16=True)
    cache = ec.ExpertPageCache(store, device=dev, cache_mb=40 * store.layout.page_stride / 1e6, max_active_pages=16)
    paged = moe.Int8ExpertBackend(page_cache=cache, w8a16=True)
    for layer, x, idx, w in _steps(dev, 3, 16):
        assert torch.equal(paged.moe(layer, x, idx, w), resident.moe(layer, x, idx, w)), layer
    assert cache.stats.evictions > 0
    cache.close()


def test_cache_holds_everything_after_one_pass(dev, tmp_path):
    ec, moe = _mods()
    store, resident = _setup(tmp_path, dev, L=2, E=8)
    cache = ec.ExpertPageCache(store, device=dev, cache_mb=1e4, max_active_pages=8)
    assert cache.capacity == 16
    paged = moe.Int8ExpertBackend(page_cache=cache)
    steps = _steps(dev, 2, 8, k=8, steps=3)
    for layer, x, idx, w in steps:
        assert torch.equal(paged.moe(layer, x, idx, w), resident.moe(layer, x, idx, w))
    assert cache.stats.page_misses == 16 and cache.stats.evictions == 0
    assert cache.stats.host_to_device_bytes == 16 * store.layout.page_stride
    cache.close()


def _state(cache):
    st = cache.stats.as_dict()
    return list(cache.entries.items()), sorted(cache.decode_protected), st


@pytest.mark.parametrize("slots", [48, 40])  # every page resident / some layers paged
@pytest.mark.parametrize("policy", ["global-lru-v1", "layer-frequency-lru-v1"])
def test_device_slot_table_matches_host_binding(dev, tmp_path, slots, policy):
    """Layers whose pages are all resident bind their slots through the device table with
    no host sync; outputs and the cache's LRU order, protection set and statistics equal
    those of the host-side binding on the same sequence."""
    ec, moe = _mods()
    store, resident = _setup(tmp_path, dev)
    runs = []
    for use_table in (True, False):
        cache = ec.ExpertPageCache(store, device=dev, cache_mb=slots * store.layout.page_stride / 1e6,
                                   max_active_pages=16, cache_policy=policy)
        if not use_table:
            cache.acquire_layer_table = lambda *a, **k: None
        paged = moe.Int8ExpertBackend(page_cache=cache)
        outs = []
        steps = _steps(dev, 3, 16, T=24, k=4, steps=4)
        for i, (layer, x, idx, w) in enumerate(steps):
            outs.append(paged.moe(layer, x, idx, w, prefill=(i % 5 == 0)))
        torch.cuda.synchronize()
        runs.append((outs, _state(cache), dict(cache.device_table_stats)))
        cache.close()
    (o1, s1, d1), (o2, s2, d2) = runs
    assert all(torch.equal(a, b) for a, b in zip(o1, o2))
    assert s1 == s2
    if slots == 48:
        assert d1["device_table_layers"] > 0  # the fast binding was taken
    ref = [resident.moe(layer, x, idx, w) for layer, x, idx, w in _steps(dev, 3, 16, T=24, k=4, steps=4)]
    assert all(torch.equal(a, b) for a, b in zip(o1, ref))


def test_preload_makes_layers_use_the_device_table(dev, tmp_path):
    ec, moe = _mods()
    store, resident = _setup(tmp_path, dev, L=2, E=8)
    cache = ec.ExpertPageCache(store, device=dev, cache_mb=1e4, max_active_pages=4)
    assert cache.preload() == 16
    assert cache.stats.host_to_device_bytes == 16 * store.layout.page_stride
    paged = moe.Int8ExpertBackend(page_cache=cache)
    steps = _steps(dev, 2, 8, k=2, steps=2)
    for layer, x, idx, w in steps:
        assert torch.equal(paged.moe(layer, x, idx, w), resident.moe(layer, x, idx, w))
    assert cache.device_table_stats["device_table_layers"] == len(steps)
    assert cache.stats.page_misses == 0 and cache.stats.page_hits == cache.stats.page_requests > 0
    cache.close()
    # a cache smaller than the model preloads what fits and demand-fills the rest
    small = ec.ExpertPageCache(store, device=dev, cache_mb=10 * store.layout.page_stride / 1e6, max_active_pages=8)
    assert small.preload() == 10
    paged = moe.Int8ExpertBackend(page_cache=small)
    for layer, x, idx, w in steps:
        assert torch.equal(paged.moe(layer, x, idx, w), resident.moe(layer, x, idx, w))
    small.close()
