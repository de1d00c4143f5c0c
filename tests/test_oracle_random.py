"""Pins of the oracle's restatement of the random stream the reference draws
from: Zig's std.Random.DefaultPrng (Xoshiro256++ seeded by SplitMix64),
Random.float(f64) and Random.floatNorm (the 256-layer ziggurat), used by
randomizedSvd (abliterate.zig:473-479), Sketch.init (directions.zig:65-67)
and Sampler.pick (model.zig:5208-5263).

- SplitMix64 and Xoshiro256++ against the sequences of Zig's own std tests
  (lib/std/Random/SplitMix64.zig and Xoshiro256.zig, test "sequence"); the
  same numbers are Vigna's published generators' outputs for those seeds.
- Xoshiro256++'s state transition against its published jump polynomial
  (xoshiro256plusplus.c's JUMP, equivalent to 2^128 steps), checked by
  raising the transition's GF(2) matrix to 2^128 by repeated squaring.
- float(f64) by what it must be: every value in [0, 1), its mantissa the
  draw's low 52 bits, its exponent the draw's leading zeros, uniform.
- The ziggurat's tables by the closed forms its constants satisfy: the base
  layer's area r f(r) + integral of f beyond r equals v (scipy's erfc), every
  layer's rectangle has area v, and the 255th closes the top (area v up to
  f = 1); its draws by the normal distribution (Kolmogorov-Smirnov, tail
  mass beyond r).
- Sampler.pick on the reference's own sampler test (model.zig:5270-5286).

The rule that extends a float(f64) draw whose top 12 bits are zero (one
draw in 4096) follows Zig 0.16's Random.zig as published; no Zig toolchain
is here to run it, so that rule's stream position is parity unpinned."""
import numpy as np
import pytest
from scipy import special, stats

# Zig std: lib/std/Random/SplitMix64.zig test "splitmix64 sequence"
SPLITMIX_SEED = 0xaeecf86f7878dd75
SPLITMIX_SEQ = [0x5dbd39db0178eb44, 0xa9900fb66b397da3, 0x5c1a28b1aeebcf5c, 0x64a963238f776912,
                0xc6d4177b21d1c0ab, 0xb2cbdbdb5ea35394]
# Zig std: lib/std/Random/Xoshiro256.zig test "sequence" (init(0))
XOSHIRO_SEQ0 = [0x53175d61490b23df, 0x61da6f3dc380d507, 0x5c0fdf91ec9a7bfc, 0x02eebf8c3bbe5e1a,
                0x7eca04ebaf4a5eea, 0x0543c37757f08d9a]
# xoshiro256plusplus.c (Blackman & Vigna): JUMP, 2^128 calls of next()
JUMP = [0x180ec6d33cfd0aba, 0xd5a61266f0c9392c, 0xa9582618e03fc9aa, 0x39abdc4529b1661c]

NORM_R, NORM_V = 3.6541528853610088, 0.00492867323399
M64 = (1 << 64) - 1


def test_splitmix_seeding_matches_zig(ref):
    """init(seed) fills the state with SplitMix64's first four outputs."""
    st = ref.sampler_init(SPLITMIX_SEED)
    assert [int(x) for x in st] == SPLITMIX_SEQ[:4]


def test_xoshiro_sequence_matches_zig(ref):
    got = ref.zig_draws(6, 0, "u64")
    assert [int(x) for x in got] == XOSHIRO_SEQ0


def _transition_matrix():
    """Xoshiro256's state update as a 256 x 256 GF(2) matrix (rows of Python
    ints, bit j of row i = coefficient of input bit j in output bit i),
    built by applying the oracle-independent update to unit vectors."""
    def step(s):
        s = list(s)
        t = (s[1] << 17) & M64
        s[2] ^= s[0]
        s[3] ^= s[1]
        s[1] ^= s[2]
        s[0] ^= s[3]
        s[2] ^= t
        s[3] = ((s[3] << 45) | (s[3] >> 19)) & M64
        return s
    cols = []
    for j in range(256):
        s = [0, 0, 0, 0]
        s[j // 64] = 1 << (j % 64)
        out = step(s)
        cols.append(out[0] | out[1] << 64 | out[2] << 128 | out[3] << 192)
    return cols  # column j = image of unit vector j


def _apply(cols, v):
    r = 0
    j = 0
    while v:
        if v & 1:
            r ^= cols[j]
        v >>= 1
        j += 1
    return r


def _compose(a, b):
    """columns of A * B"""
    return [_apply(a, c) for c in b]


def test_xoshiro_transition_meets_the_published_jump(ref):
    """T^(2^128) s equals the JUMP polynomial's combination of T^i s: a wrong
    shift or rotation in the transition fails it. The oracle's stream is
    then tied to the transition: its outputs are rotl(s0 + s3, 23) + s0 of
    the states T^i s0, checked on the first draws."""
    cols = _transition_matrix()
    st0 = [int(x) for x in ref.sampler_init(12345)]
    vec = st0[0] | st0[1] << 64 | st0[2] << 128 | st0[3] << 192
    # the jump as published: accumulate the states at the polynomial's terms
    acc, cur = 0, vec
    for word in JUMP:
        for b in range(64):
            if (word >> b) & 1:
                acc ^= cur
            cur = _apply(cols, cur)
    # T^(2^128) by 128 squarings
    p = cols
    for _ in range(128):
        p = _compose(p, p)
    assert _apply(p, vec) == acc
    # the oracle's outputs follow the transition
    draws = [int(x) for x in ref.zig_draws(8, 12345, "u64")]
    cur = vec
    for d in draws:
        s0, s3 = cur & M64, (cur >> 192) & M64
        x = (s0 + s3) & M64
        assert d == ((((x << 23) | (x >> 41)) & M64) + s0) & M64
        cur = _apply(cols, cur)


def test_float64_is_built_from_one_draw(ref):
    """With a draw's top 12 bits not all zero, float(f64) is that draw read
    as 2^-(1 + clz) (1 + low52 / 2^52), one draw per value; values are
    uniform on [0, 1)."""
    n = 20000
    u64 = ref.zig_draws(n + 64, 99, "u64")
    f = ref.zig_draws(n, 99, "f64")
    assert ((f >= 0) & (f < 1)).all()
    i = 0
    for val in f[:2000]:
        d = int(u64[i])
        if d >> 52 == 0:  # top 12 bits zero: further draws decide the exponent
            break
        lz = 64 - d.bit_length()
        mant = d & ((1 << 52) - 1)
        assert val == np.ldexp(1.0 + mant / 2.0 ** 52, -(1 + lz))
        i += 1
    big = ref.zig_draws(200000, 5, "f64")
    assert stats.kstest(big, "uniform").pvalue > 1e-3
    assert abs((big < 2.0 ** -8).mean() - 2.0 ** -8) < 5e-4


def test_ziggurat_tables_close_form(ref):
    x, f = ref.zig_norm_tables()
    base = NORM_R * np.exp(-NORM_R ** 2 / 2) + np.sqrt(np.pi / 2) * special.erfc(NORM_R / np.sqrt(2))
    assert abs(base - NORM_V) < 1e-9 * NORM_V
    assert x[1] == NORM_R and x[256] == 0.0
    assert abs(x[0] * f[1] - NORM_V) < 1e-12  # x0 f(r) = v
    areas = x[1:256] * (f[2:257] - f[1:256])  # layer i's rectangle: x_i (f_{i+1} - f_i)
    np.testing.assert_allclose(areas[:-1], NORM_V, rtol=1e-9)
    # the top layer: x_255 (1 - f(x_255)) is v to the constants' precision
    assert abs(x[255] * (1 - f[255]) - NORM_V) < 1e-6 * NORM_V
    assert np.all(np.diff(x[1:]) < 0)


def test_norm_draws_are_standard_normal(ref):
    z = ref.zig_draws(400000, 42, "norm")
    assert stats.kstest(z, "norm").pvalue > 1e-3
    tail = (np.abs(z) > NORM_R).mean()
    assert abs(tail - special.erfc(NORM_R / np.sqrt(2))) < 3e-4
    g = ref.edit_gaussian(1000, 42)
    np.testing.assert_array_equal(g, z[:1000].astype(np.float32))
    assert not np.array_equal(ref.edit_gaussian(1000, 43), g)


def test_sampler_reference_test_on_the_oracle(ref):
    """model.zig:5270-5286 on the oracle's Sampler."""
    logits = np.array([[0.0, 2.0, 1.0, -1.0, 2.0 + np.log(np.float32(3.0))]], dtype=np.float32)
    st = ref.sampler_init(1)
    assert ref.sampler_pick(logits, st, 0.0, 50, 1.0)[0] == 4
    st = ref.sampler_init(1)
    assert (ref.sampler_pick(np.tile(logits, (20, 1)), st, 1.0, 1, 1.0) == 4).all()
    st = ref.sampler_init(7)
    n = 20000
    got = ref.sampler_pick(np.tile(logits, (n, 1)), st, 1.0, 2, 1.0)
    counts = np.bincount(got, minlength=5)
    assert counts[0] + counts[2] + counts[3] == 0
    assert abs(counts[4] / n - 0.75) < 0.02
    st = ref.sampler_init(7)
    assert (ref.sampler_pick(np.tile(logits, (200, 1)), st, 1.0, 50, 0.5) == 4).all()


def test_sampler_pick_draws_in_row_order(ref):
    """One float(f64) per sampled row, in order: picking rows one call at a
    time or all at once gives the same tokens and the same final state."""
    rng = np.random.default_rng(3)
    logits = (rng.standard_normal((40, 300)) * 2).astype(np.float32)
    a = ref.sampler_init(11)
    all_at_once = ref.sampler_pick(logits, a, 0.8, 20, 0.9)
    b = ref.sampler_init(11)
    one_by_one = np.concatenate([ref.sampler_pick(logits[i:i + 1], b, 0.8, 20, 0.9) for i in range(40)])
    np.testing.assert_array_equal(all_at_once, one_by_one)
    np.testing.assert_array_equal(a, b)
    # greedy picks draw nothing
    g = ref.sampler_init(11)
    ref.sampler_pick(logits, g, 0.0, 20, 0.9)
    np.testing.assert_array_equal(g, ref.sampler_init(11))


RANDOM_MUTANTS = {
    "xoshiro shift 17 -> 18": ("uint64_t t = st[1] << 17;", "uint64_t t = st[1] << 18;"),
    "xoshiro rotation 45 -> 44": ("st[3] = zig_rotl(st[3], 45);", "st[3] = zig_rotl(st[3], 44);"),
    "float64 exponent bias": ("uint64_t bits = ((1022 - lz) << 52)", "uint64_t bits = ((1023 - lz) << 52)"),
    "ziggurat v": ("const double r = 3.6541528853610088, v = 0.00492867323399;",
                   "const double r = 3.6541528853610088, v = 0.00492867323499;"),
    "ziggurat u range [0, 2)": ("u -= 3.0; /* [-1, 1) */", "u -= 2.0; /* [-1, 1) */"),
    "sampler draw not scaled by the kept mass": ("double r = ref_zig_float64(st) * mass;",
                                                 "double r = ref_zig_float64(st);"),
}


def test_planted_mistakes_fail_the_random_pins():
    import tempfile
    from oracle.ref import Ref
    from test_oracle_pins import _build_mutant
    with tempfile.TemporaryDirectory() as tmp:
        survivors = []
        for name, (old, new) in RANDOM_MUTANTS.items():
            r = Ref(path=_build_mutant(tmp, name, old, new))
            try:
                test_splitmix_seeding_matches_zig(r)
                test_xoshiro_sequence_matches_zig(r)
                test_float64_is_built_from_one_draw(r)
                test_ziggurat_tables_close_form(r)
                test_norm_draws_are_standard_normal(r)
                test_sampler_reference_test_on_the_oracle(r)
                survivors.append(name)
            except AssertionError:
                pass
        assert not survivors, f"mistakes the pins do not catch: {survivors}"
