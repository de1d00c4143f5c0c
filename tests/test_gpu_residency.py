"""compute.Residency behind the per-call entry points (compute.zig:567-693):
the reference's own residency test (compute.zig:835-888) on real weights.
Hot weights stay registered and the least recently used one is evicted; a
weight larger than the budget is used and dropped; new contents at a cached
address are a miss and the product follows them; forget_weights releases
everything; without stable host weights nothing is cached. Every product is
checked against float64 numpy at the VTable bar."""
import time

import numpy as np
import pytest
import torch

from ditch_amd import synth
from ditch_amd.weights import HostWeight

pytestmark = pytest.mark.gpu


def _ok(dev, x, w, wf):
    got = dev.matmulT(x, w)
    want = x.astype(np.float64) @ wf.astype(np.float64).T
    np.testing.assert_allclose(got, want, rtol=1e-3, atol=1e-4 * np.abs(want).max())


def test_residency_keeps_hot_weights_and_evicts_the_least_recently_used(dev):
    rng = np.random.default_rng(7)
    ws = [rng.standard_normal((37, 48)).astype(np.float32) for _ in range(3)]
    a, b, c = (HostWeight.f32(w) for w in ws)
    x = rng.standard_normal((5, 48)).astype(np.float32)
    try:
        dev.set_residency(1 << 30, True)
        assert dev.residency_stats()["enabled"] == 1
        _ok(dev, x, a, ws[0])
        st = dev.residency_stats()
        assert (st["misses"], st["hits"], st["entries"]) == (1, 0, 1)
        per = st["used"]
        assert per > 0
        dev.set_residency(2 * per, True)  # room for two
        _ok(dev, x, b, ws[1])
        _ok(dev, x, a, ws[0])  # a is now the most recent
        st = dev.residency_stats()
        assert (st["misses"], st["hits"], st["entries"], st["evictions"]) == (2, 1, 2, 0)
        _ok(dev, x, c, ws[2])  # c does not fit: b (least recently used) goes
        st = dev.residency_stats()
        assert (st["misses"], st["entries"], st["evictions"], st["used"]) == (3, 2, 1, 2 * per)
        _ok(dev, x, a, ws[0])
        _ok(dev, x, c, ws[2])
        assert dev.residency_stats()["hits"] == 3
        # the other per-call entry points share the cache
        n = dev.rowNorms(a)
        np.testing.assert_allclose(n, np.linalg.norm(ws[0].astype(np.float64), axis=1), rtol=1e-5)
        assert dev.residency_stats()["hits"] == 4

        # other weights at a cached address (a new mapping reusing it): a miss,
        # the stale copy released, and the product follows the new contents
        # (the signature samples the buffers, as compute.zig:617-628 does)
        ev = dev.residency_stats()["evictions"]
        ws[0][...] = rng.standard_normal(ws[0].shape).astype(np.float32)
        _ok(dev, x, a, ws[0])
        st = dev.residency_stats()
        assert st["evictions"] == ev + 1 and st["misses"] == 4 and st["entries"] == 2

        # a weight larger than the whole budget is used and not kept
        dev.set_residency(per // 2, True)
        assert dev.residency_stats()["entries"] == 0
        _ok(dev, x, b, ws[1])
        assert dev.residency_stats()["entries"] == 0

        # forgetting (a mapped file was closed) releases everything
        dev.set_residency(2 * per, True)
        _ok(dev, x, a, ws[0])
        _ok(dev, x, b, ws[1])
        assert dev.residency_stats()["entries"] == 2
        dev.forget_weights()
        st = dev.residency_stats()
        assert st["entries"] == 0 and st["used"] == 0
        _ok(dev, x, a, ws[0])
        assert dev.residency_stats()["entries"] == 1

        # without stable host weights nothing is cached at all
        dev.set_residency(2 * per, False)
        st0 = dev.residency_stats()
        assert st0["entries"] == 0 and st0["enabled"] == 0
        _ok(dev, x, a, ws[0])
        st = dev.residency_stats()
        assert st["entries"] == 0 and st["hits"] == st0["hits"] and st["misses"] == st0["misses"]
    finally:
        dev.set_residency(0, False)


def test_residency_every_format_and_the_second_call(dev):
    """Packed formats (their scale grids and zero points in the key and the
    signature) give the same products from the cache as from a fresh upload;
    the second call of a large Q8_0 weight skips the upload."""
    gen = torch.Generator().manual_seed(5)
    x = np.random.default_rng(3).standard_normal((7, 512)).astype(np.float32)
    try:
        dev.set_residency(1 << 32, True)
        for fmt in ("fp8", "mxfp4", "int4", "q8_0", "bf16"):
            w = synth.QUANTIZERS[fmt](torch.randn(96, 512, generator=gen) * 0.02)
            first = dev.matmulT(x, w)
            second = dev.matmulT(x, w)
            np.testing.assert_array_equal(first, second)
            dev.set_residency(0, False)
            fresh = dev.matmulT(x, w)
            dev.set_residency(1 << 32, True)
            np.testing.assert_array_equal(first, fresh)
        big = synth.q8_0_random(14336, 4096, gen)
        xb = np.random.default_rng(4).standard_normal((1, 4096)).astype(np.float32)
        t0 = time.perf_counter()
        o1 = dev.matmulT(xb, big)
        t1 = time.perf_counter()
        o2 = dev.matmulT(xb, big)
        t2 = time.perf_counter()
        np.testing.assert_array_equal(o1, o2)
        assert t2 - t1 < t1 - t0, (t1 - t0, t2 - t1)
    finally:
        dev.set_residency(0, False)
