"""The direction pipeline on the device against the oracle: the window mean,
winsorising and f64 sums (bit for bit: the same operations in the same order,
the order statistics exact), Moments, the difference-of-means directions and
the sketch basis (to f32 rounding: the device's dot products sum in another
order); and the whole path after a real forward: forward_device residuals
-> reduce -> means -> directions, against the oracle's forward."""
import numpy as np
import pytest

import model_gen as mg
from ditch_amd import hipmem
from ditch_amd.hip import Model
from oracle.ref import RefModel
from test_oracle_directions import _capture_layout, planted_case

pytestmark = pytest.mark.gpu


def _buf(a):
    return hipmem.Buffer.from_array(np.ascontiguousarray(a))


def dev_reduce(dev, res, first, take, q, with_sq=True, sum0=None):
    E, NC, H = res.shape
    P = first.size
    bres, bf, bt = _buf(res.astype(np.float32)), _buf(first), _buf(take)
    bv = hipmem.Buffer(P * E * H * 4)
    bs = _buf(np.zeros((E, H)) if sum0 is None else sum0)
    bq = _buf(np.zeros((E, H))) if with_sq else None
    dev.check(dev.lib.ditch_hip_residual_reduce_device(dev.h, bres.ptr, E, NC, H, bf.ptr, bt.ptr, P, q, bv.ptr,
                                                       bs.ptr, bq.ptr if bq else None, None))
    dev.sync()
    return (bv.download(np.float32, (P, E, H)), bs.download(np.float64, (E, H)),
            bq.download(np.float64, (E, H)) if bq else None)


@pytest.mark.parametrize("q", [-1.0, 0.5, 0.9, 0.999])
@pytest.mark.parametrize("H", [64, 896, 4096, 7168])
def test_residual_reduce_bit_exact(dev, ref, q, H):
    rng = np.random.default_rng(H + int(abs(q) * 1000))
    lens = [9, 1, 4, 30, 2]
    first, take, ncap = _capture_layout(lens, 4)
    E = 5
    res = (rng.standard_cauchy((E, ncap, H)) * 0.5).astype(np.float32)
    s0 = rng.standard_normal((E, H))  # sums carried over from an earlier batch
    gv, gs, gq = dev_reduce(dev, res, first, take, q, sum0=s0)
    cs, cq = s0.copy(), np.zeros((E, H))
    cv = ref.residual_reduce(res, first, take, q, cs, cq)
    np.testing.assert_array_equal(gv, cv)
    np.testing.assert_array_equal(gs, cs)
    np.testing.assert_array_equal(gq, cq)
    bm = hipmem.Buffer(E * H * 4)
    bs = _buf(gs)  # every device buffer stays referenced until the call has run
    dev.check(dev.lib.ditch_hip_residual_mean_device(dev.h, bm.ptr, bs.ptr, 7, E * H, None))
    dev.sync()
    np.testing.assert_array_equal(bm.download(np.float32, (E, H)), (cs / 7).astype(np.float32))


@pytest.mark.parametrize("orth", [False, True])
def test_directions_match_oracle(dev, ref, orth):
    rng = np.random.default_rng(3 + orth)
    E, H = 33, 4096
    good = rng.standard_normal((E, H)).astype(np.float32)
    bad = (good + rng.standard_normal((E, H)) * 0.2).astype(np.float32)
    bd, bg, bb = hipmem.Buffer(E * H * 4), _buf(good), _buf(bad)
    dev.check(dev.lib.ditch_hip_directions_device(dev.h, bd.ptr, bg.ptr, bb.ptr, E, H, int(orth), None))
    dev.sync()
    np.testing.assert_allclose(bd.download(np.float32, (E, H)), ref.directions(good, bad, orth), atol=2e-6)


def dev_sketch_basis(dev, center, v, first, good, k, orth, omega):
    P, E, H = v.shape
    m = omega.shape[0]
    by, bw = _buf(np.zeros((E, m, H))), _buf(np.zeros((E, m, m)))
    bo, bc, bv = _buf(omega), _buf(center), _buf(v)
    dev.check(dev.lib.ditch_hip_sketch_add_device(dev.h, by.ptr, bw.ptr, bo.ptr, m, bc.ptr, bv.ptr, P, E, H, None))
    bd, bf, bg = hipmem.Buffer(E * k * H * 4), _buf(first), _buf(good)
    dev.check(dev.lib.ditch_hip_basis_device(dev.h, bd.ptr, bf.ptr, bg.ptr, E, H, k, int(orth), by.ptr, bw.ptr, m,
                                             None))
    dev.sync()
    return by.download(np.float64, (E, m, H)), bw.download(np.float64, (E, m, m)), bd.download(np.float32, (E, k, H))


@pytest.mark.parametrize("k,orth", [(2, False), (3, True), (8, False), (16, False), (28, True)])
def test_sketch_and_basis_match_oracle(dev, ref, k, orth):
    """Sketch widths m = min(max(4k, 8), hidden) as the reference sizes them
    (directions.zig:62): 8 to 64 columns keep the basis's eigen-solver in
    LDS, 112 (k = 28) works in global scratch."""
    good, bad, bad_res, d1, d2 = planted_case(11 + k, entries=4, hidden=512, n=200)
    E, H = good.shape
    m = min(max(4 * k, 8), H)
    omega = np.random.default_rng(k).standard_normal((m, H)).astype(np.float32)
    first = ref.directions(good, bad, orth)
    gy, gw, gd = dev_sketch_basis(dev, good, bad_res, first, good, k, orth, omega)
    cy, cw = np.zeros((E, m, H)), np.zeros((E, m, m))
    ref.sketch_add(cy, cw, omega, good, bad_res)
    np.testing.assert_allclose(gy, cy, rtol=1e-9, atol=1e-9 * np.abs(cy).max())
    np.testing.assert_allclose(gw, cw, rtol=1e-9, atol=1e-9 * np.abs(cw).max())
    cd = ref.basis(first, good, k, orth, cy, cw)
    # the same directions; a component's sign is the eigen-solver's, fixed
    # across entries by the orientation pass
    for e in range(E):
        for d in range(k):
            c = float(gd[e, d] @ cd[e, d])
            if np.abs(cd[e, d]).max() == 0:
                assert np.abs(gd[e, d]).max() == 0
            else:
                assert abs(c) > 1 - 1e-4, (e, d, c)
    for e in range(1, E):
        for d in range(1, k):
            if np.abs(gd[e, d]).max() > 0:
                assert gd[e, d] @ gd[e - 1, d] >= 0
    assert abs(gd[0, 1] @ d2) > 0.95


def test_forward_then_direction_pipeline(dev, ref):
    """Two prompt sets through forward_device, window 2 with winsorising at
    0.99, the means, and the directions: every stage on device memory,
    against the oracle's forward and pipeline."""
    spec = mg.dense("bf16", hidden=256, inter=512, layers=3, vocab=2000, seed=5)
    c = spec.config
    E, H = c["layers"] + 1, c["hidden"]
    means = {}
    cm = RefModel(spec)
    gm = Model(dev, spec)
    try:
        for name, seed in (("good", 1), ("bad", 2)):
            lens = [12, 5, 30, 1, 17]
            tokens, rows, _ = mg.batch(len(lens), lens, c["vocab"], seed=seed)
            first, take, ncap = _capture_layout(lens, 2)
            cap, start = [], 0
            for ln, t in zip(lens, take):
                cap += list(range(start + ln - t, start + ln))
                start += ln
            rg, _ = gm.forward(tokens, rows, capture_rows=cap)
            rc, _ = cm.forward(tokens, rows, capture_rows=cap)
            np.testing.assert_allclose(rg, rc, rtol=1e-3, atol=1e-5)
            gv, gs, _ = dev_reduce(dev, rg, first, take, 0.99, with_sq=False)
            cs = np.zeros((E, H))
            ref.residual_reduce(rc, first, take, 0.99, cs, None)
            bm, bs = hipmem.Buffer(E * H * 4), _buf(gs)
            dev.check(dev.lib.ditch_hip_residual_mean_device(dev.h, bm.ptr, bs.ptr, len(lens), E * H, None))
            dev.sync()
            means[name] = (bm.download(np.float32, (E, H)), (cs / len(lens)).astype(np.float32))
            np.testing.assert_allclose(means[name][0], means[name][1], rtol=2e-3, atol=1e-4)
    finally:
        gm.free()
        cm.free()
    bd, bg, bb = hipmem.Buffer(E * H * 4), _buf(means["good"][0]), _buf(means["bad"][0])
    dev.check(dev.lib.ditch_hip_directions_device(dev.h, bd.ptr, bg.ptr, bb.ptr, E, H, 1, None))
    dev.sync()
    want = ref.directions(means["good"][1], means["bad"][1], True)
    got = bd.download(np.float32, (E, H))
    assert (np.einsum("eh,eh->e", got, want) > 1 - 1e-3).all()
