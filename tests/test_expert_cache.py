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
