"""Generation on the device (generateKeep, model.zig:5378-5444): the token
picker against the reference's sampler test (model.zig:5270-5286),
numpy's top-k / top-p distribution and the oracle's Sampler over the same
Zig random stream (token for token), the persistent KV cache against the
one-shot forward, greedy generation checked against the oracle by teacher
forcing (each generated token is the oracle's most likely next token, up to
near-ties at the logit tolerance), EOS and full-cache stops, and seeded
sampling."""
import numpy as np
import pytest

import model_gen as mg
from ditch_amd import abi, hipmem
from ditch_amd.hip import Model
from oracle.ref import RefModel

pytestmark = pytest.mark.gpu


def make_sampler(dev, sampler):
    return abi.sampler(dev.lib, sampler.get("seed", 0), sampler["temperature"], sampler["top_k"], sampler["top_p"])


def pick(dev, logits, sampler=None):
    """Device picks of the rows in order; `sampler` a dict (a new Sampler)
    or an abi.Sampler (advanced in place)."""
    import ctypes
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    n, V = logits.shape
    bl, bo = hipmem.Buffer.from_array(logits), hipmem.Buffer(n * 4)
    smp = make_sampler(dev, sampler) if isinstance(sampler, dict) else sampler
    dev.check(dev.lib.ditch_hip_pick_tokens_device(dev.h, bo.ptr, bl.ptr, n, V,
                                                   ctypes.byref(smp) if smp is not None else None, None))
    dev.sync()
    return bo.download(np.uint32, (n,))


def test_sampler_reference_test(dev):
    """model.zig:5270-5286: greedy at temperature 0, top-k 1 is greedy, top-k 2
    keeps tokens 4 and 1 at 3/4 and 1/4, top-p 0.5 keeps token 4 alone."""
    logits = np.array([0.0, 2.0, 1.0, -1.0, 2.0 + np.log(np.float32(3.0))], dtype=np.float32)
    assert pick(dev, logits[None], {"temperature": 0, "top_k": 50, "top_p": 1})[0] == 4
    assert pick(dev, logits[None])[0] == 4
    rows = np.tile(logits, (20, 1))
    assert (pick(dev, rows, {"temperature": 1, "top_k": 1, "top_p": 1, "seed": 1}) == 4).all()
    n = 20000
    got = pick(dev, np.tile(logits, (n, 1)), {"temperature": 1, "top_k": 2, "top_p": 1, "seed": 7})
    counts = np.bincount(got, minlength=5)
    assert counts[0] + counts[2] + counts[3] == 0
    assert abs(counts[4] / n - 0.75) < 0.02
    got = pick(dev, np.tile(logits, (200, 1)), {"temperature": 1, "top_k": 50, "top_p": 0.5, "seed": 7})
    assert (got == 4).all()


def test_argmax_first_maximum_and_wide_rows(dev):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((7, 151936)).astype(np.float32)
    x[3, [5, 90000, 150000]] = 50.0  # ties: the first index wins
    x[5, :] = -np.inf
    x[6, 77] = np.nan
    want = np.argmax(np.where(np.isnan(x), -np.inf, x), axis=1)
    want[5] = 0
    np.testing.assert_array_equal(pick(dev, x), want)


@pytest.mark.parametrize("top_k,top_p,temp", [(50, 0.95, 1.0), (256, 1.0, 0.7), (5, 0.6, 2.0)])
def test_sampling_distribution_matches_numpy(dev, top_k, top_p, temp):
    """Every draw lies in numpy's top-k / top-p set (stable order: larger
    value, then smaller index) and the frequencies follow its softmax."""
    rng = np.random.default_rng(top_k)
    V = 128256
    row = (rng.standard_normal(V) * 2).astype(np.float32)
    row[[10, 20]] = row.max() + 0.5  # a tie at the top
    order = np.argsort(-row.astype(np.float64), kind="stable")[:top_k]
    vals = row[order]
    p = np.exp((vals - vals[0]).astype(np.float64) / temp)
    csum = np.cumsum(p)
    kept = int(np.searchsorted(csum, top_p * p.sum(), side="left")) + 1
    kept = min(kept, top_k)
    probs = p[:kept] / p[:kept].sum()
    n = 20000
    got = pick(dev, np.tile(row, (n, 1)), {"temperature": temp, "top_k": top_k, "top_p": top_p, "seed": 3})
    allowed = set(order[:kept].tolist())
    assert set(got.tolist()) <= allowed
    freq = np.array([(got == t).mean() for t in order[:kept]])
    assert np.abs(freq - probs).max() < 0.02


@pytest.mark.parametrize("top_k,top_p,temp", [(40, 0.9, 0.8), (256, 1.0, 1.5), (1, 1.0, 1.0)])
def test_pick_matches_the_oracle_sampler(dev, ref, top_k, top_p, temp):
    """The Sampler's picks, token for token, against the oracle's Sampler
    over the same Zig stream: 300 rows (two launches), one call of 300 and
    calls of 120 + 180 rows continuing one sampler; the samplers' states
    agree afterwards."""
    rng = np.random.default_rng(top_k)
    logits = (rng.standard_normal((300, 32000)) * 3).astype(np.float32)
    st = ref.sampler_init(21)
    want = ref.sampler_pick(logits, st, temp, top_k, top_p)
    cfg = {"temperature": temp, "top_k": top_k, "top_p": top_p, "seed": 21}
    s1 = make_sampler(dev, cfg)
    np.testing.assert_array_equal(pick(dev, logits, s1), want)
    assert list(s1.rng) == [int(x) for x in st]
    s2 = make_sampler(dev, cfg)
    got = np.concatenate([pick(dev, logits[:120], s2), pick(dev, logits[120:], s2)])
    np.testing.assert_array_equal(got, want)
    assert list(s2.rng) == list(s1.rng)


def test_greedy_pick_draws_nothing(dev):
    s = make_sampler(dev, {"temperature": 0.0, "top_k": 50, "top_p": 1.0, "seed": 4})
    before = list(s.rng)
    pick(dev, np.random.default_rng(0).standard_normal((5, 100)).astype(np.float32), s)
    assert list(s.rng) == before


def _teacher_forcing_ok(ref, spec, prompts, outs):
    """The oracle's logits at every generated position: each generated token
    is its most likely next token, up to a near-tie of 1e-3 of max |logit|."""
    cm = RefModel(spec)
    try:
        for p, gen in zip(prompts, outs):
            seq = list(p) + list(gen[:-1])
            rows = [(0, i) for i in range(len(seq))]
            lr = list(range(len(p) - 1, len(seq)))
            _, lc = cm.forward(np.asarray(seq, np.uint32), rows, logit_rows=lr)
            scale = np.abs(lc).max()
            for t, row in zip(gen, lc):
                assert row[t] >= row.max() - 1e-3 * scale, (t, row.argmax(), row.max() - row[t])
    finally:
        cm.free()


GEN_MODELS = {
    "dense_mxfp4": lambda: mg.dense("mxfp4", hidden=256, inter=512, layers=2, vocab=3000, seed=3),
    "moe_int4": lambda: mg.moe("int4", layers=2, dense_first=1, experts=8, top_k=2, vocab=3000, seed=4),
    "mla_fp8": lambda: mg.mla("fp8", vocab=3000, seed=6),
}


@pytest.mark.parametrize("name", list(GEN_MODELS))
def test_greedy_generation_matches_oracle(dev, ref, name):
    spec = GEN_MODELS[name]()
    rng = np.random.default_rng(len(name))
    prompts = [list(rng.integers(0, 3000, n)) for n in (9, 1, 30)]
    gm = Model(dev, spec)
    cache = gm.kv_cache(4, 64)
    try:
        outs, first = gm.generate(cache, prompts, 12, first_logits=True)
        assert [len(o) for o in outs] == [12, 12, 12]
        # the prefill's logits equal the prompt forward's
        for b, p in enumerate(prompts):
            _, lg = gm.forward(np.asarray(p, np.uint32), [(0, i) for i in range(len(p))], logit_rows=[len(p) - 1])
            np.testing.assert_allclose(first[b], lg[0], atol=1e-4 * np.abs(lg).max())
        # the same again through a fresh cache gives the same tokens
        outs2, _ = gm.generate(cache, prompts, 12)
        assert outs2 == outs
    finally:
        gm.kv_cache_free(cache)
        gm.free()
    _teacher_forcing_ok(ref, spec, prompts, outs)


def test_cache_chunked_prefill_equals_one_shot(dev, ref):
    """forward_cached over each prompt's first rows, then the rest (reading
    the keys the first call wrote), against the oracle's one-shot forward."""
    spec = GEN_MODELS["dense_mxfp4"]()
    lens = [20, 7, 40]
    tokens, rows, last = mg.batch(3, lens, spec.config["vocab"], seed=2)
    rows = np.asarray(rows, dtype=np.uint32)
    first = rows[:, 1] < 5
    gm = Model(dev, spec)
    cache = gm.kv_cache(3, 64)
    try:
        V = spec.config["vocab"]
        outs = []
        for sel in (first, ~first):
            idx = np.nonzero(sel)[0]
            lr = np.array([np.nonzero(idx == l)[0][0] for l in last if l in set(idx)], dtype=np.uint64)
            bt = hipmem.Buffer.from_array(np.ascontiguousarray(tokens[idx]))
            br = hipmem.Buffer.from_array(np.ascontiguousarray(rows[idx]))
            bl = hipmem.Buffer.from_array(lr) if lr.size else None
            blog = hipmem.Buffer(max(lr.size, 1) * V * 4)
            dev.check(dev.lib.ditch_hip_forward_cached(gm.h, cache, bt.ptr, br.ptr, idx.size,
                                                       bl.ptr if bl else None, lr.size, blog.ptr, lr.size * V * 4))
            dev.sync()
            outs.append(blog.download(np.float32, (lr.size, V)) if lr.size else None)
        lg = outs[1]  # every prompt's last row is in the second call
    finally:
        gm.kv_cache_free(cache)
        gm.free()
    cm = RefModel(spec)
    try:
        _, lc = cm.forward(tokens, [tuple(r) for r in rows], logit_rows=last)
    finally:
        cm.free()
    assert np.abs(lg - lc).max() <= 1e-3 * np.abs(lc).max()


def test_generation_stops_at_eos_and_full_cache(dev):
    spec = GEN_MODELS["dense_mxfp4"]()
    rng = np.random.default_rng(9)
    prompts = [list(rng.integers(0, 3000, n)) for n in (5, 8, 16)]
    gm = Model(dev, spec)
    cache = gm.kv_cache(3, 16)
    try:
        outs, _ = gm.generate(cache, prompts, 6)
        eos = int(outs[0][2])
        outs_e, _ = gm.generate(cache, prompts, 6, eos=[eos])
        cut = outs[0].index(eos) + 1
        assert outs_e[0] == outs[0][:cut]
        assert len(outs[2]) == 1  # a prompt of 16 fills the 16-position cache
        assert len(outs[1]) == 6
    finally:
        gm.kv_cache_free(cache)
        gm.free()


def test_sampled_generation_is_seeded(dev):
    spec = GEN_MODELS["moe_int4"]()
    rng = np.random.default_rng(11)
    prompts = [list(rng.integers(0, 3000, n)) for n in (6, 12)]
    gm = Model(dev, spec)
    cache = gm.kv_cache(2, 64)
    try:
        s = {"temperature": 1.0, "top_k": 50, "top_p": 0.95, "seed": 5}
        a, _ = gm.generate(cache, prompts, 20, sampler=s)
        b, _ = gm.generate(cache, prompts, 20, sampler=s)
        c, _ = gm.generate(cache, prompts, 20, sampler=dict(s, seed=6))
        assert a == b and a != c
    finally:
        gm.kv_cache_free(cache)
        gm.free()


def test_sampled_generation_matches_the_oracle_sampler(dev, ref):
    """generateKeep with a Sampler (model.zig:5378-5444): the oracle's logits
    at every generated position (teacher forcing on the device's tokens),
    picked by the oracle's Sampler over the same Zig stream in the
    reference's order (prompt order within a step), give the device's
    tokens, up to what the logit tolerance leaves open (near-equal logits
    that sort either way: at least 90 % of the picks are exact); the
    caller's sampler ends where the oracle's does."""
    spec = GEN_MODELS["dense_mxfp4"]()
    rng = np.random.default_rng(12)
    prompts = [list(rng.integers(0, 3000, n)) for n in (6, 12, 9)]
    steps = 10
    cfg = {"temperature": 0.9, "top_k": 40, "top_p": 0.95, "seed": 77}
    gm = Model(dev, spec)
    cache = gm.kv_cache(3, 64)
    try:
        smp = make_sampler(dev, cfg)
        outs, _ = gm.generate(cache, prompts, steps, sampler=smp)
    finally:
        gm.kv_cache_free(cache)
        gm.free()
    assert [len(o) for o in outs] == [steps] * 3
    cm = RefModel(spec)
    try:
        per_prompt = []
        for p, gen in zip(prompts, outs):
            seq = list(p) + list(gen[:-1])
            rows = [(0, i) for i in range(len(seq))]
            _, lc = cm.forward(np.asarray(seq, np.uint32), rows, logit_rows=list(range(len(p) - 1, len(seq))))
            per_prompt.append(lc)
    finally:
        cm.free()
    st = ref.sampler_init(cfg["seed"])
    draws = ref.zig_draws(3 * steps, cfg["seed"], "f64")  # one float(f64) per pick
    exact = 0
    for t in range(steps):
        rows = np.stack([per_prompt[b][t] for b in range(3)])
        want = ref.sampler_pick(rows, st, cfg["temperature"], cfg["top_k"], cfg["top_p"])
        for b in range(3):
            got = outs[b][t]
            exact += got == want[b]
            assert got in _near_picks(rows[b], draws[3 * t + b], cfg), (t, b, got, want[b])
    assert exact >= 0.9 * 3 * steps, exact
    assert list(smp.rng) == [int(x) for x in st]


def _near_picks(x, u, cfg):
    """Sampler.pick's token for the draw u over logits x, and every token a
    perturbation of x within the logit tolerance (1e-3 of max |logit|) can
    give instead: near-equal logits that may sort either way, and the
    neighbours of a cumulative boundary the draw lies within the tolerance
    of."""
    tol = 1e-3 * float(np.abs(x).max())
    order = np.argsort(-x.astype(np.float64), kind="stable")[:cfg["top_k"]]
    vals = x[order]
    p = np.exp((vals - vals[0]).astype(np.float64) / cfg["temperature"])
    cs = np.cumsum(p)
    kept = int(np.searchsorted(cs, cfg["top_p"] * cs[-1], side="left")) + 1
    r = u * cs[kept - 1]
    i = min(int(np.searchsorted(cs[:kept], r, side="left")), kept - 1)
    near = {int(order[i])}
    near |= {int(order[j]) for j in range(len(order)) if abs(float(vals[j]) - float(vals[i])) <= 2 * tol}
    slack = 4 * tol / cfg["temperature"] * cs[kept - 1]
    for j in (i - 1, i + 1):
        if 0 <= j < len(order) and (abs(cs[i] - r) <= slack or (i > 0 and abs(cs[i - 1] - r) <= slack)):
            near.add(int(order[j]))
    return near
