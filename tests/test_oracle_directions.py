"""Pins of the oracle's direction pipeline: the window mean / winsorising /
f64 sums of Engine.forEachResidual (engine.zig:414-431), Moments, the
difference-of-means directions (abliterate.zig:88-109), orthonormalize
(abliterate.zig:409-423), the symmetric eigen-solver and the Nystrom sketch
basis (directions.zig:80-134, 371-500).

Known answers come from the reference's own tests (cited); the rest from
mathematics checked with numpy in float64: order statistics, exact sums,
eigen-decompositions, and recovery of planted directions.
"""
import math

import numpy as np
import pytest


def test_symmetric_eigen_known_answer(ref):
    """directions.zig:503-512: eigenvalues of [[2,1,0],[1,2,0],[0,0,5]]."""
    a, _ = ref.symmetric_eigen(np.array([[2, 1, 0], [1, 2, 0], [0, 0, 5]], dtype=np.float64))
    np.testing.assert_allclose(sorted(np.diag(a)), [1, 3, 5], atol=1e-9)


@pytest.mark.parametrize("n", [2, 8, 17, 32])
def test_symmetric_eigen_matches_numpy(ref, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal((n, n))
    m = x @ x.T + np.diag(rng.uniform(0, 1, n))
    a, v = ref.symmetric_eigen(m)
    ev = np.diag(a)
    np.testing.assert_allclose(np.sort(ev), np.linalg.eigvalsh(m), rtol=1e-10, atol=1e-10 * np.abs(ev).max())
    np.testing.assert_allclose(v.T @ v, np.eye(n), atol=1e-10)
    np.testing.assert_allclose(m @ v, v * ev, atol=1e-9 * np.abs(ev).max())


def _capture_layout(lens, window):
    """engine.zig:395-410: the last min(window, len) rows of every prompt."""
    first, take, n_cap = [], [], 0
    for ln in lens:
        t = min(window, ln)
        first.append(n_cap)
        take.append(t)
        n_cap += t
    return np.array(first, np.uint32), np.array(take, np.uint32), n_cap


def test_quantile_known_answers(ref):
    """engine.zig:582-584: quantile([1,2,3,4], 0.5) = 2.5, quantile(.., 1) = 4;
    through the winsorising: |v| is clamped at that threshold."""
    res = np.array([[[1, -2, 3, -4]]], dtype=np.float32)  # one entry, one captured row
    first, take = np.array([0], np.uint32), np.array([1], np.uint32)
    v = ref.residual_reduce(res, first, take, 0.5)
    np.testing.assert_array_equal(v[0, 0], [1, -2, 2.5, -2.5])
    v = ref.residual_reduce(res, first, take, 1.0)  # q = 1 is no winsorising (q < 1 only)
    np.testing.assert_array_equal(v[0, 0], [1, -2, 3, -4])
    v = ref.residual_reduce(res, first, take, 0.999999)
    assert np.abs(v).max() <= 4 and np.abs(v).max() > 3.99


@pytest.mark.parametrize("q", [0.5, 0.9, 0.99])
def test_winsorising_threshold_is_the_linear_quantile(ref, q):
    rng = np.random.default_rng(int(q * 100))
    E, H = 3, 1000
    res = (rng.standard_cauchy((E, 1, H))).astype(np.float32)
    v = ref.residual_reduce(res, np.array([0], np.uint32), np.array([1], np.uint32), q)
    for e in range(E):
        srt = np.sort(np.abs(res[e, 0].astype(np.float64)))
        thr = np.quantile(srt, q, method="linear")
        got = float(np.abs(v[0, e]).max())
        # between the two order statistics it interpolates, and at the f64
        # linear quantile up to the f32 position q * (n - 1) the reference uses
        lo = int(np.floor(q * (H - 1)))
        assert srt[lo] <= got <= srt[min(lo + 1, H - 1)]
        assert abs(got - thr) <= 1e-4 * (srt[min(lo + 1, H - 1)] - srt[lo]) + 1e-6 * thr
        keep = np.abs(res[e, 0]) <= np.abs(v[0, e]).max()
        np.testing.assert_array_equal(v[0, e][keep], res[e, 0][keep])
        assert (np.sign(v[0, e]) == np.sign(res[e, 0])).all()


def test_window_mean_and_f64_sums(ref):
    rng = np.random.default_rng(5)
    lens = [5, 1, 3, 7]
    first, take, ncap = _capture_layout(lens, 3)
    E, H = 4, 64
    res = rng.standard_normal((E, ncap, H)).astype(np.float32)

    s = np.zeros((E, H))
    sq = np.zeros((E, H))
    v = ref.residual_reduce(res, first, take, -1.0, s, sq)
    for b in range(len(lens)):
        rows = res[:, first[b]:first[b] + take[b], :].astype(np.float64)
        np.testing.assert_allclose(v[b], rows.mean(axis=1), rtol=4e-7, atol=1e-7)
        if take[b] == 1:
            np.testing.assert_array_equal(v[b], res[:, first[b], :])  # window 1: the last row itself
    for e in range(E):
        for i in range(0, H, 7):
            assert s[e, i] == pytest.approx(math.fsum(float(v[b, e, i]) for b in range(len(lens))), abs=1e-15)
            assert sq[e, i] == pytest.approx(math.fsum(float(v[b, e, i]) ** 2 for b in range(len(lens))), abs=1e-15)


def test_directions_closed_form(ref):
    rng = np.random.default_rng(6)
    E, H = 5, 300
    good = rng.standard_normal((E, H)).astype(np.float32)
    bad = (good + rng.standard_normal((E, H)) * 0.3).astype(np.float32)
    d = ref.directions(good, bad, False)
    diff = bad.astype(np.float64) - good.astype(np.float64)
    want = diff / np.linalg.norm(diff, axis=1, keepdims=True)
    np.testing.assert_allclose(d, want, atol=2e-6)
    o = ref.directions(good, bad, True)
    g = good.astype(np.float64) / np.linalg.norm(good.astype(np.float64), axis=1, keepdims=True)
    proj = want - (want * g).sum(1, keepdims=True) * g
    np.testing.assert_allclose(o, proj / np.linalg.norm(proj, axis=1, keepdims=True), atol=2e-6)
    assert np.abs((o.astype(np.float64) * g).sum(1)).max() < 1e-6


def test_orthonormalize_is_gram_schmidt(ref):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((5, 200)).astype(np.float32)
    x[3] = 0  # a zero row stays zero (norm <= 1e-20)
    o = ref.orthonormalize(x)
    q, _ = np.linalg.qr(x[[0, 1, 2, 4]].astype(np.float64).T)
    np.testing.assert_allclose(np.abs(o[[0, 1, 2, 4]] @ q), np.eye(4), atol=1e-5)
    np.testing.assert_array_equal(o[3], 0)


def planted_case(seed, entries=2, hidden=24, n=300):
    """directions.zig:515-573: good residuals = noise around an offset; bad ones
    add 3 d1 (+ jitter) and a zero-mean spread of 2 along d2."""
    rng = np.random.default_rng(seed)
    planted = np.linalg.qr(rng.standard_normal((hidden, 2)))[0].T.astype(np.float32)
    d1, d2 = planted
    good = (0.5 * rng.standard_normal((entries, hidden))).astype(np.float32)
    a = 3.0 + 0.3 * rng.standard_normal(n)
    b = 2.0 * rng.standard_normal(n)
    bad_res = (good[None] + a[:, None, None] * d1 + b[:, None, None] * d2
               + 0.1 * rng.standard_normal((n, entries, hidden))).astype(np.float32)
    bad = bad_res.astype(np.float64).mean(axis=0).astype(np.float32)
    return good, bad, bad_res, d1, d2


def sketch_of(ref, center, v, k, seed):
    E, H = center.shape
    m = min(max(4 * k, 8), H)
    omega = np.random.default_rng(seed).standard_normal((m, H)).astype(np.float32)
    y = np.zeros((E, m, H))
    w = np.zeros((E, m, m))
    ref.sketch_add(y, w, omega, center, v)
    return y, w, omega


def test_two_planted_directions_are_recovered(ref):
    good, bad, bad_res, d1, d2 = planted_case(11)
    y, w, _ = sketch_of(ref, good, bad_res, 2, 3)
    first = ref.directions(good, bad, False)
    dirs = ref.basis(first, good, 2, False, y, w)
    for e in range(2):
        f, s = dirs[e, 0], dirs[e, 1]
        assert abs(f @ d1) > 0.95 and abs(s @ d2) > 0.95
        assert abs(f @ s) < 1e-4 and abs(np.linalg.norm(s) - 1) < 1e-4
    assert dirs[0, 1] @ dirs[1, 1] > 0  # consistent orientation across entries
    # k = 1 is the single-direction result exactly
    np.testing.assert_array_equal(ref.basis(first, good, 1, True, y, w)[:, 0], first)


def test_sketch_is_exact_on_low_rank_residuals(ref):
    """Centred residuals spanning fewer than m dimensions: the sketch is exact
    and the second direction is the top eigenvector of P C P (numpy, f64)."""
    rng = np.random.default_rng(12)
    E, H, P, r = 2, 40, 60, 4
    center = rng.standard_normal((E, H)).astype(np.float32)
    basis = np.linalg.qr(rng.standard_normal((H, r)))[0]
    coef = rng.standard_normal((P, E, r)) * np.array([5, 3, 2, 1])
    v = (center[None] + np.einsum("per,hr->peh", coef, basis)).astype(np.float32)
    y, w, _ = sketch_of(ref, center, v, 2, 4)
    first = np.zeros((E, H), np.float32)
    first[:, 0] = 1
    dirs = ref.basis(first, center, 2, False, y, w)
    for e in range(E):
        z = v[:, e, :].astype(np.float64) - center[e]
        c = z.T @ z
        p = np.eye(H)
        p[0, 0] = 0  # the first direction projected out
        evals, evecs = np.linalg.eigh(p @ c @ p)
        assert abs(dirs[e, 1] @ evecs[:, -1]) > 1 - 1e-5


DIR_MUTANTS = {
    "quantile upper neighbour dropped": ("size_t hi = lo + 1 < n - 1 ? lo + 1 : n - 1;", "size_t hi = lo;"),
    "window mean over take + 1": ("float inv = 1.0f / (float)(t_n > 1 ? t_n : 1);", "float inv = 1.0f / (float)(t_n + 1);"),
    "orthogonalisation sign": ("axpy(d, -p, gd, hidden);", "axpy(d, p, gd, hidden);"),
    "sketch centre ignored": ("z[i] = (double)r[i] - (double)c[i];", "z[i] = (double)r[i];"),
    "basis order ascending": ("gram[order[j - 1] * r + order[j - 1]] < gram[o * r + o]",
                              "gram[order[j - 1] * r + order[j - 1]] > gram[o * r + o]"),
}


def _all_direction_checks(r):
    test_quantile_known_answers(r)
    test_window_mean_and_f64_sums(r)
    test_directions_closed_form(r)
    test_two_planted_directions_are_recovered(r)
    test_sketch_is_exact_on_low_rank_residuals(r)


def test_planted_mistakes_fail_the_direction_pins():
    import tempfile
    from oracle.ref import Ref
    from test_oracle_pins import _build_mutant
    with tempfile.TemporaryDirectory() as tmp:
        survivors = []
        for name, (old, new) in DIR_MUTANTS.items():
            r = Ref(path=_build_mutant(tmp, name, old, new))
            try:
                _all_direction_checks(r)
                survivors.append(name)
            except AssertionError:
                pass
        assert not survivors, f"mistakes the pins do not catch: {survivors}"
