"""Expert page store, host tier and slot policy (host logic, CPU)."""

from __future__ import annotations

import numpy as np
import pytest
import torch


def _ec():
    from mrun_pub_amd import expert_cache

    return expert_cache


def _arrays(rng, L=2, E=3, H=64, I=32):
    gu = rng.integers(-127, 128, size=(L, E, 2 * I, H), dtype=np.int8)
    gus = rng.uniform(0.5, 1.5, size=(L, E, 2 * I)).astype(np.float32)
    dn = rng.integers(-127, 128, size=(L, E, H, I), dtype=np.int8)
    dns = rng.uniform(0.5, 1.5, size=(L, E, H)).astype(np.float32)
    return gu, gus, dn, dns


def test_store_round_trip_and_tier(tmp_path):
    ec = _ec()
    gu, gus, dn, dns = _arrays(np.random.default_rng(0))
    store = ec.PackedInt8ExpertStore(ec.write_int8_expert_store(tmp_path, gu, gus, dn, dns))
    assert (store.layers, store.experts) == (2, 3)
    target = torch.empty((2, store.layout.page_stride), dtype=torch.uint8)
    store.gather(1, [2, 0], target)
    views = store.view_pages(target)
    assert np.array_equal(views.gate_up[0].numpy(), gu[1, 2]) and np.array_equal(views.down[1].numpy(), dn[1, 0])
    assert np.array_equal(views.gate_up_scales[0].numpy(), gus[1, 2])
    assert np.array_equal(views.down_scales[1].numpy(), dns[1, 0])
    # a two-page tier: warm fills pages 0 and 1, page 2 is admitted never (full), others from disk
    tier = ec.HostPageTier(store, host_cache_mb=2 * store.layout.page_stride / 1e6, try_pin=False)
    assert tier.capacity == 2 and tier.warm()["warmed_pages"] == 2
    assert tier.host_page(0, 1) is not None and tier.host_page(1, 0) is None
    out = torch.empty((2, store.layout.page_stride), dtype=torch.uint8)
    tier.gather(0, [0, 2], out)
    assert np.array_equal(store.view_pages(out).gate_up[1].numpy(), gu[0, 2])
    assert tier.stats["served_pages"] >= 1 and tier.stats["disk_pages"] >= 1


def test_store_rejects_foreign_manifests(tmp_path):
    ec = _ec()
    root = ec.write_int8_expert_store(tmp_path, *_arrays(np.random.default_rng(1), L=1, E=1))
    (root / "manifest.json").write_text((root / "manifest.json").read_text().replace(ec.STORE_CODEC, "fp8"))
    with pytest.raises(ValueError, match="codec"):
        ec.PackedInt8ExpertStore(root)


def _acquire(policy, layer, experts, protect=()):
    keys = [(layer, e) for e in sorted(set(experts))]
    misses = 0
    for key in keys:
        if key in policy.entries:
            policy.entries.move_to_end(key)
        else:
            policy.reserve(key, set(keys))
            misses += 1
    policy.stats.page_misses += misses
    policy.stats.page_hits += len(keys) - misses


def test_global_lru_coalesces_misses_and_reuses_hits():
    """The sequence of reference test_qwen3_moe_cuda.py:290-308 on a 2-slot cache."""
    ec = _ec()
    stats = ec.PageCacheStats()
    pol = ec.SlotPolicy(2, 2, ec.GLOBAL_LRU_CACHE_POLICY, stats)
    _acquire(pol, 0, [2, 0])
    assert stats.page_misses == 2
    _acquire(pol, 0, [0, 2])
    assert stats.page_hits == 2 and stats.page_misses == 2
    _acquire(pol, 1, [1, 2])
    assert stats.page_misses == 4 and len(pol.entries) == 2 and stats.evictions == 2


def test_active_set_is_never_evicted():
    ec = _ec()
    pol = ec.SlotPolicy(2, 1, ec.GLOBAL_LRU_CACHE_POLICY, ec.PageCacheStats())
    with pytest.raises(RuntimeError, match="active set"):
        _acquire(pol, 0, [0, 1, 2])


def test_layer_frequency_quota_evicts_within_the_layer():
    ec = _ec()
    stats = ec.PageCacheStats()
    pol = ec.SlotPolicy(4, 2, ec.LAYER_FREQUENCY_CACHE_POLICY, stats)
    assert pol.layer_quotas == (2, 2)
    _acquire(pol, 0, [0, 1])
    _acquire(pol, 1, [0, 1])
    _acquire(pol, 0, [2])  # layer 0 at quota: its own LRU page goes
    assert stats.same_layer_evictions == 1 and (0, 0) not in pol.entries and (1, 0) in pol.entries
    _acquire(pol, 1, [5, 6, 7][:1])
    assert stats.same_layer_evictions == 2 and (1, 0) not in pol.entries


def test_protected_pages_lose_protection_when_evicted():
    ec = _ec()
    stats = ec.PageCacheStats()
    pol = ec.SlotPolicy(1, 1, ec.GLOBAL_LRU_CACHE_POLICY, stats)
    _acquire(pol, 0, [3])
    pol.decode_protected.add((0, 3))
    _acquire(pol, 0, [4])
    assert stats.decode_protected_demotions == 1 and not pol.decode_protected
    with pytest.raises(ValueError, match="cache policy"):
        ec.SlotPolicy(1, 1, "mru", stats)


def test_victim_follows_the_rules_on_random_states():
    """The one-scan victim choice against the rules written as three filters (oldest
    first): same layer when the incoming layer is at its quota, then any layer above its
    quota, then the oldest unprotected page; global LRU takes the oldest."""
    import random

    ec = _ec()
    rng = random.Random(5)
    for trial in range(400):
        layers, cap = rng.randint(1, 4), rng.randint(2, 12)
        policy = rng.choice(["global-lru-v1", "layer-frequency-lru-v1"])
        pol = ec.SlotPolicy(cap, layers, policy, ec.PageCacheStats())
        keys = [(l, e) for l in range(layers) for e in range(6)]
        rng.shuffle(keys)
        for i, k in enumerate(keys[:cap]):
            pol.entries[k] = i
            pol.layer_entry_counts[k[0]] += 1
        order = list(pol.entries)
        protected = set(rng.sample(order, rng.randint(0, len(order))))
        incoming = rng.randrange(layers)
        free = [k for k in order if k not in protected]
        counts, quotas = pol.layer_entry_counts, pol.layer_quotas
        if not free:
            want = (None, "fallback_evictions")
        elif policy == "global-lru-v1":
            want = (free[0], "fallback_evictions")
        else:
            same = [k for k in free if k[0] == incoming]
            over = [k for k in free if counts[k[0]] > quotas[k[0]]]
            if same and counts[incoming] >= quotas[incoming]:
                want = (same[0], "same_layer_evictions")
            elif over:
                want = (over[0], "over_quota_evictions")
            else:
                want = (free[0], "fallback_evictions")
        assert pol.victim(incoming, protected) == want, (trial, policy, order, protected, incoming)


# ---- the host book against the reference's own cache ------------------------------------------


def test_page_book_replays_the_reference_cache():
    """tests/golden/page_cache.json holds the reference's ExpertPageCache (qwen3_moe_cuda.py:
    983-1777, run on the CPU) driven through seeded random sequences of decode and prefill
    slot-binding acquires, transient-frequency-v1 prefills and resets, with its state after
    every call.  The host book replays each sequence and must match every selected set,
    slot, slab position, LRU order, free list, protection set, layer count, statistic and
    the final page-trace manifest."""
    import json
    from pathlib import Path

    ec = _ec()
    data = json.loads((Path(__file__).resolve().parent / "golden" / "page_cache.json").read_text())
    kinds = set()
    for cfg in data["configs"]:
        trace = ec.PageTrace(layer_count=cfg["layers"], page_bytes=cfg["page_stride"])
        book = ec.PageBook(capacity=cfg["capacity"], layers=cfg["layers"], experts=cfg["experts"],
                           page_bytes=cfg["page_stride"], max_active_pages=cfg["max_active"],
                           cache_policy=cfg["cache_policy"], trace=trace)
        for i, op in enumerate(cfg["ops"]):
            where = (cfg["name"], i, op["op"])
            kinds.add(op["op"])
            if op["op"] == "reset":
                book.reset(clear_pages=op["clear_pages"])
            elif op["op"] == "acquire":
                ids, slots, _ = book.acquire(op["layer"], op["routed"], protect=op["protect"])
                assert (ids, slots) == (op["selected"], op["slots"]), where
            else:
                plan = book.transient(op["layer"], op["routed"])
                assert (plan.expert_ids, plan.group_slots()) == (op["selected"], op["group_slots"]), where
            assert [[k[0], k[1], v] for k, v in book.entries.items()] == op["entries"], where
            assert sorted(list(k) for k in book.decode_protected) == op["decode_protected"], where
            assert book.policy.layer_entry_counts == op["layer_entry_counts"], where
            assert book.policy.free_slots == op["free_slots"], where
            stats = book.stats.as_dict()
            assert sorted(stats) == cfg["stats_keys"]
            assert [stats[k] for k in cfg["stats_keys"]] == op["stats"], where
        assert trace.export() == cfg["trace"], cfg["name"]
        assert trace.status() == cfg["trace_status"], cfg["name"]
    assert kinds == {"acquire", "transient", "reset"}


def _plan(pol, layer, routed):
    from collections import Counter

    return pol.plan_transient_prefill(layer, Counter(routed))


def test_transient_prefill_reference_kats():
    """The policy decisions of the reference's transient-prefill tests
    (test_qwen3_moe_cuda.py:644-818) on a 3-slot, 2-layer cache (quotas 2 and 1)."""
    ec = _ec()
    stats = ec.PageCacheStats()
    pol = ec.SlotPolicy(3, 2, ec.LAYER_FREQUENCY_CACHE_POLICY, stats)
    plan = _plan(pol, 0, [2, 2, 2, 0, 0, 1])
    assert plan.expert_ids == [0, 1, 2] and plan.group_slots() == [1, 2, 0]
    assert set(pol.entries) == {(0, 0), (0, 2)} and pol.layer_entry_counts == [2, 0]
    assert plan.miss_count == 3 and len(plan.admitted) == 2
    _plan(pol, 1, [1, 1, 1, 2, 0])
    _acquire(pol, 0, [0, 2])
    pol.decode_protected.update({(0, 0), (0, 2)})
    sealed = dict(pol.entries)
    assert set(sealed) == {(0, 0), (0, 2), (1, 1)} and pol.layer_entry_counts == [2, 1]
    # a second scan runs the layer from the slab but cannot evict its sealed quota
    plan = _plan(pol, 0, [1, 1, 1, 2, 0])
    assert dict(pol.entries) == sealed and plan.preserved == 2 and not plan.admitted

    # a resident page is read out of its slot before the slot is reused by an admission
    pol = ec.SlotPolicy(3, 2, ec.LAYER_FREQUENCY_CACHE_POLICY, ec.PageCacheStats())
    _acquire(pol, 0, [0, 1])
    slot_of_0 = pol.entries[(0, 0)]
    plan = _plan(pol, 0, [2, 2, 2, 3, 3, 0])
    assert plan.expert_ids == [0, 2, 3] and plan.group_slots() == [2, 0, 1]
    assert plan.resident_slots == [slot_of_0] and set(pol.entries) == {(0, 2), (0, 3)}
    assert slot_of_0 in [slot for _, slot in plan.admitted]
    assert len(plan.stale) == 2 and plan.preserved == 0


def test_page_trace_reference_kat_and_caps():
    """The event semantics of test_qwen3_moe_cuda.py:310-355 and the caps of :399-460."""
    import hashlib
    import json
    from collections import Counter

    ec = _ec()
    tr = ec.PageTrace(layer_count=2, page_bytes=4096)
    for phase, layer, routed in (("prefill", 0, [2, 2, 0]), ("prefill", 1, [1, 1]), ("prefill", 0, [0]),
                                 ("decode", 0, [2]), ("decode", 1, [1]), ("decode", 0, [0])):
        tr.record(phase=phase, layer=layer, frequencies=Counter(routed))
    m = tr.export()
    assert m["events"] == [
        {"phase": "prefill", "step": 0, "layer": 0, "pages": [[0, 1], [2, 2]]},
        {"phase": "prefill", "step": 0, "layer": 1, "pages": [[1, 2]]},
        {"phase": "prefill", "step": 1, "layer": 0, "pages": [[0, 1]]},
        {"phase": "decode", "step": 0, "layer": 0, "pages": [[2, 1]]},
        {"phase": "decode", "step": 0, "layer": 1, "pages": [[1, 1]]},
        {"phase": "decode", "step": 1, "layer": 0, "pages": [[0, 1]]},
    ]
    core = {k: v for k, v in m.items() if k != "trace_sha256"}
    assert m["trace_sha256"] == hashlib.sha256(
        json.dumps(core, sort_keys=True, separators=(",", ":")).encode()).hexdigest()
    assert tr.status()["manifest_bytes"] == len(json.dumps(m, sort_keys=True, separators=(",", ":")).encode())
    assert tr.drain() == m and tr.export() is None and tr.sha256 is None
    with pytest.raises(ValueError, match="hard maximum"):
        ec.PageTrace(layer_count=2, page_bytes=1, max_events=ec.PAGE_TRACE_HARD_MAX_EVENTS + 1)
    with pytest.raises(ValueError, match="positive integer"):
        ec.PageTrace(layer_count=2, page_bytes=1, max_requests=True)
    with pytest.raises(ValueError, match="empty compact trace"):
        ec.PageTrace(layer_count=2, page_bytes=1, max_manifest_bytes=10)
    req = ec.PageTrace(layer_count=2, page_bytes=1, max_requests=1)
    with pytest.raises(ec.Qwen3MoePageTraceLimitError, match="request cap"):
        req.record(phase="prefill", layer=0, frequencies=Counter([0, 1]))
    assert req.export() is None
    ev = ec.PageTrace(layer_count=2, page_bytes=1, max_events=1)
    ev.record(phase="prefill", layer=0, frequencies=Counter([0]))
    with pytest.raises(ec.PageTraceLimitError, match="event cap"):
        ev.record(phase="prefill", layer=1, frequencies=Counter([1]))
    probe = ec.PageTrace(layer_count=2, page_bytes=1)
    probe.record(phase="prefill", layer=0, frequencies=Counter([0]))
    one = probe.manifest_bytes
    byte = ec.PageTrace(layer_count=2, page_bytes=1, max_manifest_bytes=one)
    byte.record(phase="prefill", layer=0, frequencies=Counter([0]))
    with pytest.raises(ec.PageTraceLimitError, match="manifest-byte cap"):
        byte.record(phase="prefill", layer=1, frequencies=Counter([1]))
    with pytest.raises(ValueError, match="phase"):
        probe.record(phase="warmup", layer=0, frequencies=Counter([0]))


def test_page_views_over_an_offset_arena():
    """Page views over a slice that starts inside a larger allocation (the transient slab
    after the cache slots) address that slice, not the allocation's start."""
    ec = _ec()
    gu, gus, dn, dns = _arrays(np.random.default_rng(5), L=1, E=3)
    import tempfile

    with tempfile.TemporaryDirectory() as tmp:
        store = ec.PackedInt8ExpertStore(ec.write_int8_expert_store(tmp, gu, gus, dn, dns))
        stride = store.layout.page_stride
        whole = torch.zeros((5, stride), dtype=torch.uint8)
        store.gather(0, [0, 1, 2], whole[2:])
        views = store.view_pages(whole[2:])
        for e in range(3):
            assert np.array_equal(views.gate_up[e].numpy(), gu[0, e])
            assert np.array_equal(views.down[e].numpy(), dn[0, e])
            assert np.array_equal(views.gate_up_scales[e].numpy(), gus[0, e])
            assert np.array_equal(views.down_scales[e].numpy(), dns[0, e])
