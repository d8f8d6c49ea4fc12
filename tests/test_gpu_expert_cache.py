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


# ---- transient-frequency-v1 prefill and the page trace on the device --------------------------


def _gold_cache_store(tmp_path, cfg):
    """An int8 expert store with the golden run's geometry (H 4, I 2: one 4096-byte page)."""
    ec, _ = _mods()
    rng = np.random.default_rng(cfg["seed"])
    L, E = cfg["layers"], cfg["experts"]
    arrays = (rng.integers(-127, 128, size=(L, E, 4, 4), dtype=np.int8), rng.random((L, E, 4), dtype=np.float32),
              rng.integers(-127, 128, size=(L, E, 4, 2), dtype=np.int8), rng.random((L, E, 4), dtype=np.float32))
    return ec.PackedInt8ExpertStore(ec.write_int8_expert_store(tmp_path / cfg["name"], *arrays))


@pytest.mark.parametrize("which", [0, 1, 2, 3])
def test_cache_replays_the_reference_cache_and_moves_the_right_bytes(dev, tmp_path, which):
    """The reference cache's recorded sequences (tests/golden/page_cache.json) through the
    HIP-backed cache: the same decisions, statistics and trace, and after every call every
    cache slot holds its page's bytes and every slab position the routed page's bytes."""
    import json
    from pathlib import Path

    ec, _ = _mods()
    cfg = json.loads((Path(__file__).resolve().parent / "golden" / "page_cache.json").read_text())["configs"][which]
    store = _gold_cache_store(tmp_path, cfg)
    stride = store.layout.page_stride
    assert stride == cfg["page_stride"]
    pages = torch.from_numpy(np.array(store._pages()))  # noqa: SLF001 - the expected bytes
    cache = ec.ExpertPageCache(store, device=dev, cache_mb=cfg["capacity"] * stride / 1e6,
                               max_active_pages=cfg["max_active"], cache_policy=cfg["cache_policy"],
                               prefill_page_policy=cfg["prefill"], page_trace=True, route_prefetch=False)
    assert cache.capacity == cfg["capacity"]
    for i, op in enumerate(cfg["ops"]):
        where = (cfg["name"], i, op["op"])
        idx = torch.tensor([op.get("routed", [0])], device=dev)
        if op["op"] == "reset":
            cache.reset(clear_pages=op["clear_pages"])
        elif op["op"] == "acquire":
            sel, _, slots = cache.acquire_slot_binding(op["layer"], idx, protect=op["protect"])
            assert (sel.tolist(), slots.tolist()) == (op["selected"], op["slots"]), where
        else:
            sel, views, gs = cache.acquire_transient_prefill(op["layer"], idx)
            assert (sel.tolist(), gs.tolist()) == (op["selected"], op["group_slots"]), where
            torch.cuda.synchronize()
            slab = cache.slab.cpu()
            for g, e in enumerate(op["selected"]):
                assert torch.equal(slab[gs[g].item()], pages[store.global_page(op["layer"], e)]), where
        cache.release()
        torch.cuda.synchronize()
        assert [[k[0], k[1], v] for k, v in cache.entries.items()] == op["entries"], where
        assert sorted(list(k) for k in cache.decode_protected) == op["decode_protected"], where
        assert cache.layer_entry_counts == op["layer_entry_counts"], where
        stats = cache.stats.as_dict()
        assert [stats[k] for k in cfg["stats_keys"]] == op["stats"], where
        held = cache.cache.cpu()
        for (layer, expert, slot) in op["entries"]:
            assert torch.equal(held[slot], pages[store.global_page(layer, expert)]), (where, layer, expert)
    assert cache.export_page_trace() == cfg["trace"]
    cache.close()


def test_transient_prefill_equals_resident_and_keeps_the_decode_set(dev, tmp_path):
    """Under transient-frequency-v1 a prefill layer runs from the slab: its output equals the
    resident backend's bit for bit, the pages another request's decode steps protect stay
    in their slots, and only the hottest pages of the prompt are admitted (within the
    layer quota)."""
    ec, moe = _mods()
    store, resident = _setup(tmp_path, dev, L=2, E=16)
    # 16 cache slots (the active-set bound), quotas of 8 per layer, and a 16-page slab
    cache = ec.ExpertPageCache(store, device=dev, cache_mb=0, max_active_pages=16,
                               cache_policy="layer-frequency-lru-v1", prefill_page_policy="transient-frequency-v1")
    assert cache.capacity == 16 and cache.policy.layer_quotas == (8, 8)
    assert cache.slab is not None and cache.device_bytes == (16 + 16) * store.layout.page_stride
    paged = moe.Int8ExpertBackend(page_cache=cache)
    g = torch.Generator(device="cpu").manual_seed(7)

    def routes(T, k, experts):
        logits = torch.full((T, 16), -30.0)
        logits[:, experts] = torch.randn(T, len(experts), generator=g)
        w, idx = torch.softmax(logits, -1).topk(k, -1)
        x = torch.randn(T, 256, generator=g).to(torch.bfloat16)
        return x.to(dev), idx.to(dev), (w / w.sum(-1, keepdim=True)).to(torch.bfloat16).to(dev)

    # a decode request settles on four experts of each layer
    for layer in (0, 1):
        x, idx, w = routes(2, 4, [1, 3, 5, 7])
        assert torch.equal(paged.moe(layer, x, idx, w), resident.moe(layer, x, idx, w))
    decode_set = set(cache.decode_protected)
    slots_before = {k: cache.entries[k] for k in decode_set}
    assert len(decode_set) == 8
    # a long prompt scans every expert of both layers
    for layer in (0, 1):
        x, idx, w = routes(64, 8, list(range(16)))
        out = paged.moe(layer, x, idx, w, prefill=True)
        assert torch.equal(out, resident.moe(layer, x, idx, w))
    torch.cuda.synchronize()
    assert set(cache.decode_protected) == decode_set
    assert {k: cache.entries[k] for k in decode_set} == slots_before
    st = cache.stats
    assert st.transient_prefill_acquires == 2 and st.transient_prefill_pages == 32
    assert st.transient_prefill_resident_materialization_d2d_bytes == 8 * store.layout.page_stride
    # quota 8 per layer, 4 held by decode pages: four seats each for the prompt's hottest pages
    assert st.transient_prefill_admitted_pages == 8
    assert cache.layer_entry_counts == [8, 8]
    # the decode request goes on with its pages still resident (hits only)
    hits = st.page_hits
    for layer in (0, 1):
        x, idx, w = routes(2, 4, [1, 3, 5, 7])
        assert torch.equal(paged.moe(layer, x, idx, w), resident.moe(layer, x, idx, w))
    assert cache.stats.page_hits == hits + 8 and cache.stats.page_misses == st.page_misses
    # the same prompt again: pages admitted by the first prefill now come from the cache
    for layer in (0, 1):
        x, idx, w = routes(64, 8, list(range(16)))
        assert torch.equal(paged.moe(layer, x, idx, w, prefill=True), resident.moe(layer, x, idx, w))
    cache.close()


def test_page_trace_on_the_device_cache(dev, tmp_path):
    """Decode and prefill acquires are traced; tracing turns the device slot-table binding
    off (it reads routes on the host) and leaves results unchanged."""
    ec, moe = _mods()
    store, resident = _setup(tmp_path, dev, L=2, E=16)
    cache = ec.ExpertPageCache(store, device=dev, cache_mb=40 * store.layout.page_stride / 1e6, max_active_pages=16,
                               page_trace=True)
    cache.preload()
    paged = moe.Int8ExpertBackend(page_cache=cache)
    steps = _steps(dev, 2, 16, steps=2)
    for i, (layer, x, idx, w) in enumerate(steps):
        assert torch.equal(paged.moe(layer, x, idx, w, prefill=i < 2), resident.moe(layer, x, idx, w))
    assert cache.device_table_stats["device_table_layers"] == 0
    m = cache.export_page_trace()
    assert [(e["phase"], e["step"], e["layer"]) for e in m["events"]] == [
        ("prefill", 0, 0), ("prefill", 0, 1), ("decode", 0, 0), ("decode", 0, 1)]
    for e, (layer, _, idx, _) in zip(m["events"], steps):
        vals, counts = torch.unique(idx.cpu(), return_counts=True)
        assert e["pages"] == [[int(v), int(c)] for v, c in zip(vals, counts)]
    assert cache.page_trace_status()["events"] == 4 and cache.drain_page_trace() == m
    cache.close()
