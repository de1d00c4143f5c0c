"""ExpertCache.hotExperts and warm (expert_cache.zig:501-607) on the device:
the use counts of the routed experts a streaming model acquired, most used
first with ties by layer and expert; a fresh model warmed with that list
holds the hottest experts that fit before its first forward (entries naming
no streamed routed expert are skipped, an entry without uses stops the
walk), gives the cold model's forward bit for bit, and counts the warmed
experts as misses at their first use (expert_cache.zig:403-410)."""
import numpy as np
import pytest

import model_gen as mg
from ditch_amd.hip import Model

pytestmark = pytest.mark.gpu


def _fw(m, b):
    return m.forward(b[0], b[1], capture_rows=b[2], logit_rows=b[2])


def test_hot_experts_and_warm_start(dev):
    spec = mg.moe("int4", layers=3, dense_first=1, experts=16, top_k=4, seed=21)
    V = spec.config["vocab"]
    b1 = mg.batch(3, [40, 17, 64], V, seed=9)
    b2 = mg.batch(2, [5, 9], V, seed=10)
    gm = Model(dev, spec, expert_cache_bytes=1 << 40)
    try:
        for b in (b1, b1, b2):
            _fw(gm, b)
        hot = gm.hot_experts()
        st = gm.expert_cache_stats()
    finally:
        gm.free()
    assert hot == sorted(hot, key=lambda h: (-h[2], h[0], h[1]))
    assert all(spec.moe_layers[l] and e < 16 and 1 <= u <= 3 for l, e, u in hot)
    assert sum(u for _, _, u in hot) == st["hits"] + st["misses"]  # one use per acquisition
    assert hot[0][2] >= 2 and hot[-1][2] >= 1
    slot = st["slot_bytes"]

    cap = 10
    bad = [(99, 0, 50), (0, 0, 50), (1, 99, 50)]  # no such layer, a dense layer, no such expert
    wm = Model(dev, spec, expert_cache_bytes=cap * slot)
    cold = Model(dev, spec, expert_cache_bytes=cap * slot)
    try:
        n = wm.warm_experts(bad + hot)
        assert n == min(cap, len(hot))
        sw = wm.expert_cache_stats()
        assert sw["warmed"] == n and sw["resident"] == n and sw["hits"] == 0 and sw["misses"] == 0
        assert wm.warm_experts(hot) == 0  # every slot taken
        rw, lw = _fw(wm, b1)
        rc, lc = _fw(cold, b1)
        np.testing.assert_array_equal(lw, lc)
        np.testing.assert_array_equal(rw, rc)
        sw, sc = wm.expert_cache_stats(), cold.expert_cache_stats()
        assert sw["hits"] + sw["misses"] == sc["hits"] + sc["misses"]
        assert sw["hits"] == 0  # the warmed experts were reads, counted at first use
    finally:
        wm.free()
        cold.free()

    fresh = Model(dev, spec, expert_cache_bytes=cap * slot)
    try:
        assert fresh.warm_experts([(1, 0, 0)] + hot) == 0  # no uses: the walk stops
        assert fresh.expert_cache_stats()["resident"] == 0
    finally:
        fresh.free()


def test_pageable_experts_through_the_staging_ring(dev, monkeypatch):
    """Experts registered past the pinned limit stay in pageable memory and
    reach the cache through the pinned staging ring: the same forward, bit
    for bit, as with every expert pinned, in a cache of a quarter of them."""
    spec = mg.moe("int4", layers=3, dense_first=1, experts=16, top_k=4, seed=21)
    b = mg.batch(3, [40, 17, 64], spec.config["vocab"], seed=9)
    probe = Model(dev, spec, expert_cache_bytes=1 << 40)
    try:
        _fw(probe, b)
        slot = probe.expert_cache_stats()["slot_bytes"]
    finally:
        probe.free()
    budget = 8 * slot
    pinned = Model(dev, spec, expert_cache_bytes=budget)
    monkeypatch.setenv("DITCH_HIP_EXPERT_PINNED_LIMIT", str(3 * slot))  # a few pinned, the rest pageable
    paged = Model(dev, spec, expert_cache_bytes=budget)
    try:
        for _ in range(2):
            rp, lp = _fw(pinned, b)
            rq, lq = _fw(paged, b)
            np.testing.assert_array_equal(lq, lp)
            np.testing.assert_array_equal(rq, rp)
        sp, sq = pinned.expert_cache_stats(), paged.expert_cache_stats()
        assert sp["bytes_staged"] == 0 and sq["bytes_staged"] > 0
        # the pageable experts stay resident where pinned ones can go (a
        # pinned expert's refill is one DMA): fewer bytes staged than read
        assert sq["bytes_staged"] < sq["bytes_read"]
    finally:
        pinned.free()
        paged.free()
