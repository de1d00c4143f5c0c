"""Pins of the oracle's edit in every row-normalisation mode
(abliterate.computeDelta, abliterate.zig:223-538) by the reference's own
tests (abliterate.zig:554-707: the direction vanishes for none/pre, the
rank-5 `full` delta reproduces the exact renormalised matrix on 6 x 5, the
input-side ablation removes the read pattern) and, at a realistic size, by
the randomised SVD's optimality: the `full` delta's error against the exact
renormalised delta is within a few percent of the best rank-r error
(numpy's SVD in float64)."""
import numpy as np
import pytest

from ditch_amd.weights import HostWeight

MODES = {"none": 0, "pre": 1, "full": 2}


def materialize(w, a, b):
    return w.astype(np.float64) + b.astype(np.float64) @ a.astype(np.float64)


def orthonormal_rows(rng, k, n):
    return np.linalg.qr(rng.standard_normal((n, k)))[0].T.astype(np.float32)


def exact_full(w, v, weight=1.0):
    """W' = diag(n) rownorm(Wn - weight V V^T Wn) (abliterate.zig:597-617)."""
    w = w.astype(np.float64)
    n = np.linalg.norm(w, axis=1)
    wn = w / n[:, None]
    a = v.astype(np.float64) @ wn
    rows = wn - weight * v.astype(np.float64).T @ a
    return rows / np.linalg.norm(rows, axis=1, keepdims=True) * n[:, None]


@pytest.mark.parametrize("k", [1, 2])
@pytest.mark.parametrize("mode", ["none", "pre", "full"])
def test_direction_vanishes_and_full_is_exact_on_6x5(ref, k, mode):
    rng = np.random.default_rng(7)
    w = rng.standard_normal((6, 5)).astype(np.float32)
    v = orthonormal_rows(rng, 2, 6)[:k]
    a, b = ref.edit_delta_ex(HostWeight.f32(w), v, 1.0, MODES[mode], lora_rank=5, seed=1)
    assert a.shape[0] == (5 if mode == "full" else k)
    wp = materialize(w, a, b)
    n = np.ones(6) if mode == "none" else np.linalg.norm(w.astype(np.float64), axis=1)
    if mode != "full":
        assert np.abs((v / n) @ wp).max() < 1e-4
    else:
        np.testing.assert_allclose(wp, exact_full(w, v), atol=1e-3)


def test_input_side_ablation(ref):
    rng = np.random.default_rng(3)
    w = rng.standard_normal((6, 5)).astype(np.float32)
    v = orthonormal_rows(rng, 1, 6)
    u = (v.astype(np.float64) @ w)[0]
    u /= np.linalg.norm(u)
    x = rng.standard_normal(5)
    x -= (x @ u) * u
    for mode in ("none", "pre"):
        a, b = ref.edit_delta_ex(HostWeight.f32(w), v, 1.0, MODES[mode], ablate=True)
        assert a.shape[0] == 2
        wp = materialize(w, a, b)
        n = np.ones(6) if mode == "none" else np.linalg.norm(w.astype(np.float64), axis=1)
        assert np.abs((v / n) @ wp).max() < 1e-4
        assert np.abs(wp @ u).max() < 1e-4
        a1, b1 = ref.edit_delta_ex(HostWeight.f32(w), v, 1.0, MODES[mode])
        np.testing.assert_allclose(wp @ x, materialize(w, a1, b1) @ x, atol=1e-4)
    a, b = ref.edit_delta_ex(HostWeight.f32(w), v, 1.0, 2, lora_rank=5, ablate=True)
    assert a.shape[0] == 6
    assert np.abs(materialize(w, a, b) @ u).max() < 1e-3


@pytest.mark.parametrize("rows,cols,k,r", [(200, 150, 2, 3), (96, 256, 1, 4)])
def test_full_mode_is_near_the_best_rank_r_error(ref, rows, cols, k, r):
    """The exact renormalised delta D* = W'_exact - W; the randomised SVD's
    rank-r delta is within 10 % of the optimal rank-r error ||D* - D*_r||."""
    rng = np.random.default_rng(rows)
    w = rng.standard_normal((rows, cols)).astype(np.float32)
    v = orthonormal_rows(rng, k, rows)
    a, b = ref.edit_delta_ex(HostWeight.f32(w), v, 1.0, 2, lora_rank=r, seed=5)
    assert a.shape[0] == r
    dstar = exact_full(w, v) - w.astype(np.float64)
    s = np.linalg.svd(dstar, compute_uv=False)
    best = np.sqrt((s[r:] ** 2).sum())
    err = np.linalg.norm(dstar - b.astype(np.float64) @ a.astype(np.float64))
    assert err <= 1.10 * best + 1e-6 * np.linalg.norm(dstar), (err, best)


def test_jacobi_f32_eigen(ref):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((10, 10)).astype(np.float32)
    m = (x @ x.T).astype(np.float32)
    a, v = ref.jacobi_f32(m)
    np.testing.assert_allclose(np.sort(np.diag(a)), np.linalg.eigvalsh(m.astype(np.float64)), rtol=1e-4, atol=1e-3)
    np.testing.assert_allclose(v.T @ v, np.eye(10), atol=1e-5)


def test_edit_gaussian_is_standard_normal(ref):
    z = ref.edit_gaussian(200000, 42).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    assert abs((np.abs(z) < 1.96).mean() - 0.95) < 0.005
    np.testing.assert_array_equal(ref.edit_gaussian(1000, 42), z[:1000].astype(np.float32))
    assert not np.array_equal(ref.edit_gaussian(1000, 43), z[:1000].astype(np.float32))


EDIT_MUTANTS = {
    "full c without -1": ("c[i] = 1.0f / s - 1.0f;", "c[i] = 1.0f / s;"),
    "pre b without norms": ("pb[i * k + j] = -weight * v[j * rows + i] * norms[i];",
                            "pb[i * k + j] = -weight * v[j * rows + i];"),
    "normalised directions not divided": ("vn[j * rows + i] = norms[i] > 0 ? v[j * rows + i] / norms[i] : 0;",
                                          "vn[j * rows + i] = v[j * rows + i];"),
    "ablation without the primary delta": ("rc |= ref_matmulT(wu, u, k, w, r_out, pa, pb, threads);",
                                           "rc |= ref_matmulT(wu, u, k, w, 0, NULL, NULL, threads);"),
    "svd order ascending": ("while (j > 0 && bbt[order[j - 1] * q + order[j - 1]] < bbt[ov * q + ov]) {",
                            "while (j > 0 && bbt[order[j - 1] * q + order[j - 1]] > bbt[ov * q + ov]) {"),
}


def test_planted_mistakes_fail_the_edit_pins():
    import tempfile
    from oracle.ref import Ref
    from test_oracle_pins import _build_mutant
    with tempfile.TemporaryDirectory() as tmp:
        survivors = []
        for name, (old, new) in EDIT_MUTANTS.items():
            r = Ref(path=_build_mutant(tmp, name, old, new))
            try:
                for k in (1, 2):
                    for mode in MODES:
                        test_direction_vanishes_and_full_is_exact_on_6x5(r, k, mode)
                test_input_side_ablation(r)
                test_full_mode_is_near_the_best_rank_r_error(r, 200, 150, 2, 3)
                survivors.append(name)
            except AssertionError:
                pass
        assert not survivors, f"mistakes the pins do not catch: {survivors}"
