"""HIP kernels against the CPU oracle, through the C ABI (needs an MI355X).

Bars: decoded weights bit-exact; matrix products within the reference's
device-contract tolerance (selftest.zig:34-41: abs 1e-4 or rel 1e-3 per
element for matmul, abs 1e-5 / rel 1e-4 element-wise, abs/rel 1e-4 for
reductions).
"""
import ctypes
import zlib

import numpy as np
import pytest

import weights_gen as wg
from ditch_amd import abi

pytestmark = pytest.mark.gpu

TOL_MATMUL = dict(atol=1e-4, rtol=1e-3)
TOL_ELEM = dict(atol=1e-5, rtol=1e-4)
TOL_RED = dict(atol=1e-4, rtol=1e-4)


def close(got, want, atol, rtol):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    bad = np.abs(got - want) > atol + rtol * np.abs(want)
    assert not bad.any(), f"{bad.sum()} of {bad.size} outside tolerance; worst {np.abs(got - want).max():.3e}"


def same_bits(got, want):
    """Bit equality; NaN positions must match (payloads of x86-quieted NaNs
    are compared too)."""
    got, want = np.asarray(got), np.asarray(want)
    assert got.dtype == want.dtype and got.shape == want.shape
    neq = got != want
    assert not neq.any(), f"{neq.sum()} of {neq.size} differ; first at {np.argwhere(neq)[0]}: {got[neq][0]:#x} vs {want[neq][0]:#x}"


# -- decode --------------------------------------------------------------------

DEQUANT_CASES = [
    ("f32", lambda r: wg.float_random("f32", 33, 70, r)),
    ("f16", lambda r: wg.float_random("f16", 33, 70, r)),
    ("bf16", lambda r: wg.float_random("bf16", 33, 70, r)),
    ("q8_0", lambda r: wg.gguf_random(abi.Q8_0, 37, 96, r)),
    ("q4_0", lambda r: wg.gguf_random(abi.Q4_0, 21, 64, r)),
    ("q4_1", lambda r: wg.gguf_random(abi.Q4_1, 21, 64, r)),
    ("q5_0", lambda r: wg.gguf_random(abi.Q5_0, 21, 64, r)),
    ("q5_1", lambda r: wg.gguf_random(abi.Q5_1, 21, 64, r)),
    ("q4_k", lambda r: wg.gguf_random(abi.Q4_K, 9, 512, r)),
    ("q6_k", lambda r: wg.gguf_random(abi.Q6_K, 9, 512, r)),
    ("q8_k", lambda r: wg.gguf_random(abi.Q8_K, 9, 512, r)),
    ("fp8_e4m3_all_codes", lambda r: wg.fp8_random(256, 256, r, all_codes=True)),
    ("fp8_e5m2_all_codes", lambda r: wg.fp8_random(256, 256, r, e5m2=True, all_codes=True)),
    ("fp8_16x8_bf16_scale", lambda r: wg.fp8_random(48, 40, r, block=(16, 8), scale_kind="bf16")),
    ("fp8_f16_scale", lambda r: wg.fp8_random(130, 200, r, scale_kind="f16")),
    ("fp8_e8m0_scale", lambda r: wg.fp8_random(64, 96, r, block=(1, 32), scale_kind="e8m0", all_codes=True)),
    ("fp8_row_shard", lambda r: wg.fp8_random(96, 64, r, block=(16, 16), row_shard=48)),
    ("mxfp4_all_scales", lambda r: wg.mxfp4_random(256, 64, r, scale_lo=0, scale_hi=256)),
    ("mxfp4", lambda r: wg.mxfp4_random(40, 256, r)),
    ("mxfp4_t", lambda r: wg.mxfp4_t_random(64, 48, r)),
    ("int4_g128", lambda r: wg.int_random(37, 256, r)),
    ("int4_g16_bf16", lambda r: wg.int_random(37, 48, r, group=16, scale_kind="bf16")),
    ("int4_sym", lambda r: wg.int_random(20, 128, r, zero=False, scale_kind="f32")),
    ("int4_actorder", lambda r: wg.int_random(32, 64, r, group=16, actorder=True)),
    ("int3", lambda r: wg.int_random(33, 40, r, bits=3, group=8)),
    ("int8", lambda r: wg.int_random(17, 64, r, bits=8, group=32)),
]


@pytest.mark.parametrize("name,gen", DEQUANT_CASES, ids=[c[0] for c in DEQUANT_CASES])
def test_dequant_bit_exact(dev, ref, name, gen):
    from ditch_amd.hipmem import Buffer
    w = gen(np.random.default_rng(zlib.crc32(name.encode())))
    want = ref.dequant(w)
    got = dev.dequant(w)  # raw-layout decode
    same_bits(got.view(np.uint32) if got.dtype == np.float32 else got,
              want.view(np.uint32) if want.dtype == np.float32 else want)
    # the re-tiled HBM layout decodes to the same bits
    t = dev.upload(w)
    try:
        buf = Buffer(want.nbytes)
        t.dequant_device(buf.ptr, buf.nbytes, 0, w.rows)
        dev.sync()
        tiled = buf.download(want.dtype, want.shape)
        buf.free()
    finally:
        t.free()
    same_bits(tiled.view(np.uint32) if tiled.dtype == np.float32 else tiled,
              want.view(np.uint32) if want.dtype == np.float32 else want)


# -- matmulT -------------------------------------------------------------------

MM_KINDS = ["f32", "f16", "bf16", "q8_0", "q4_0", "q4_k", "q6_k", "fp8", "fp8_16x8", "mxfp4", "mxfp4_t", "int4",
            "int4_g16", "int4_sym", "int4_actorder", "int8"]
MM_SHAPES = [(1, 48, 256), (3, 100, 384), (16, 64, 512), (17, 80, 256), (64, 200, 512), (100, 96, 1024)]


@pytest.mark.parametrize("kind", MM_KINDS)
@pytest.mark.parametrize("n,rows,cols", MM_SHAPES)
def test_matmulT_matches_oracle(dev, ref, kind, n, rows, cols):
    rng = np.random.default_rng(n * 7919 + rows * 31 + cols)
    if kind.startswith(("q4_k", "q6_k")) and cols % 256:
        pytest.skip("k-quants need 256-column rows")
    w = wg.make(kind, rows, cols, rng)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    want = ref.matmulT(x, w)
    got = dev.matmulT(x, w)
    close(got, want, **TOL_MATMUL)


@pytest.mark.parametrize("kind", MM_KINDS)
@pytest.mark.parametrize("n,rows,cols", [(1, 40, 4096), (7, 33, 2880), (16, 50, 1536)])
def test_gemv_long_rows_matches_oracle(dev, ref, kind, n, rows, cols):
    """The GEMV regime over long rows: each wave's share of K runs through
    its ring of in-flight units several times, with a ragged last round and
    a ragged last row group."""
    rng = np.random.default_rng(n * 131 + cols)
    if kind.startswith(("q4_k", "q6_k")) and cols % 256:
        pytest.skip("k-quants need 256-column rows")
    w = wg.make(kind, rows, cols, rng)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    close(dev.matmulT(x, w), ref.matmulT(x, w), **TOL_MATMUL)


@pytest.mark.parametrize("kind", ["bf16", "f32", "f16"])
def test_matmulT_odd_k(dev, ref, kind):
    """K not a multiple of 8 (or of 4) takes the guarded activation loads."""
    rng = np.random.default_rng(11)
    for n, rows, cols in [(1, 5, 12), (20, 7, 20), (70, 33, 44), (33, 40, 301)]:
        w = wg.float_random(kind, rows, cols, rng)
        x = rng.standard_normal((n, cols)).astype(np.float32)
        close(dev.matmulT(x, w), ref.matmulT(x, w), **TOL_MATMUL)


@pytest.mark.parametrize("kind", ["f32", "f16"])
@pytest.mark.parametrize("n,rows,cols", [(17, 896, 896), (1024, 128, 896), (300, 520, 4864), (64, 33, 96)])
def test_float_weight_product_bias_accumulate(dev, ref, kind, n, rows, cols):
    """f32 / f16 weights above the GEMV regime (exact products on the fp32
    MFMA, k slices added in LDS when the tiles are few), with the bias and
    accumulate epilogue, at the C1 projection shapes and ragged ones."""
    from ditch_amd import hipmem
    rng = np.random.default_rng(n + rows + cols)
    w = wg.float_random(kind, rows, cols, rng)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    bias = rng.standard_normal(rows).astype(np.float32)
    prior = rng.standard_normal((n, rows)).astype(np.float32)
    t = dev.upload(w)
    try:
        bx, bb, bo = hipmem.Buffer.from_array(x), hipmem.Buffer.from_array(bias), hipmem.Buffer.from_array(prior)
        t.matmul_device(bo.ptr, bx.ptr, n, d_bias=bb.ptr, accumulate=True)
        dev.sync()
        got = bo.download(np.float32, (n, rows))
    finally:
        t.free()
    want = prior.astype(np.float64) + ref.matmulT(x, w).astype(np.float64) + bias
    close(got, want, **TOL_MATMUL)


# -- VTable element-wise ops ------------------------------------------------------

def test_rmsnorm_layernorm_softmax(dev, ref):
    rng = np.random.default_rng(12)
    x = rng.standard_normal((7, 300)).astype(np.float32)
    w = rng.standard_normal(300).astype(np.float32)
    close(dev.rmsnormRows(x, w, 1e-6), ref.rmsnorm_rows(x, w, 1e-6), **TOL_ELEM)
    close(dev.rmsnormRows(x, None, 1e-5), ref.rmsnorm_rows(x, None, 1e-5), **TOL_ELEM)
    close(dev.softmaxRows(x * 4), ref.softmax_rows(x * 4), **TOL_ELEM)
    close(dev.logSoftmaxRows(x * 4), ref.log_softmax_rows(x * 4), **TOL_ELEM)


@pytest.mark.parametrize("length", [512, 1024, 2048, 4096])
def test_rmsnorm_rows_held_in_registers(dev, ref, length):
    """Rows of 512-4096 columns take the wave-per-row kernel (the row held in
    registers, one read): with and without a weight, gemma's (1 + w), and a
    row count that leaves the last workgroup partly empty."""
    rng = np.random.default_rng(length)
    x = (rng.standard_normal((7, length)) * 3).astype(np.float32)
    w = rng.standard_normal(length).astype(np.float32)
    close(dev.rmsnormRows(x, w, 1e-6), ref.rmsnorm_rows(x, w, 1e-6), **TOL_ELEM)
    close(dev.rmsnormRows(x, None, 1e-5), ref.rmsnorm_rows(x, None, 1e-5), **TOL_ELEM)
    close(dev.rmsnormRows(x, w, 1e-6, gemma_style=True), ref.rmsnorm_rows(x, w, 1e-6, gemma=True), **TOL_ELEM)


@pytest.mark.parametrize("act", range(6))
def test_gated_activation(dev, ref, act):
    rng = np.random.default_rng(13 + act)
    n, length, stride = 5, 70, 80
    g = rng.standard_normal(n * stride).astype(np.float32) * 3
    u = rng.standard_normal(n * stride).astype(np.float32)
    close(dev.gatedActivation(act, g, u, n, length, stride, length),
          ref.gated(act, g, u, n, length, stride, length), **TOL_ELEM)


def test_rope_rows(dev, ref):
    rng = np.random.default_rng(14)
    ang = rng.uniform(0, 6, (10, 8))
    cos_t, sin_t = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    x = rng.standard_normal((6, 16)).astype(np.float32)
    pos = [0, 3, 9, 2, 2, 5]
    for style in (0, 1):
        close(dev.ropeRows(x, cos_t, sin_t, pos, style), ref.rope_rows(x, cos_t, sin_t, pos, style), **TOL_ELEM)


def test_attention_scores_values(dev, ref):
    rng = np.random.default_rng(15)
    hd, stride, nk = 64, 128, 37
    q = rng.standard_normal(hd).astype(np.float32)
    k = rng.standard_normal(nk * stride).astype(np.float32)
    s = dev.attentionScores(q, k, nk, stride, 0.125)
    want = np.array([np.dot(q.astype(np.float64), k[p * stride:p * stride + hd]) for p in range(nk)]) * 0.125
    close(s, want, **TOL_RED)
    p = np.exp(want - want.max()).astype(np.float32)
    p /= p.sum()
    out = dev.attentionValues(p, k, hd, stride)
    wv = sum(p[i] * k[i * stride:i * stride + hd].astype(np.float64) for i in range(nk))
    close(out, wv, **TOL_RED)


def test_rownorms_matvecT(dev, ref):
    rng = np.random.default_rng(16)
    for kind in ("bf16", "q8_0", "mxfp4", "int4", "fp8"):
        w = wg.make(kind, 70, 256, rng)
        close(dev.rowNorms(w), ref.rowNorms(w), **TOL_RED)
        y = rng.standard_normal((2, 70)).astype(np.float32)
        close(dev.matvecTMulti(w, y), ref.matvecTMulti(w, y), **TOL_MATMUL)


@pytest.mark.parametrize("kind,rows", [("bf16", 8200), ("q8_0", 16411)])
def test_matvecT_tall_row_chunks(dev, ref, kind, rows):
    """matvecTMulti over more than 256 x 32 rows: row chunks taller than 32
    (64 and 96 rows here, the last one ragged), five vectors."""
    rng = np.random.default_rng(rows)
    w = wg.make(kind, rows, 256, rng)
    y = rng.standard_normal((5, rows)).astype(np.float32)
    close(dev.matvecTMulti(w, y), ref.matvecTMulti(w, y), **TOL_MATMUL)


@pytest.mark.parametrize("kind", ["f32", "f16", "bf16", "q8_0", "fp8", "fp8_16x8", "mxfp4", "int4", "int4_g16",
                                  "int4_sym", "int8"])
@pytest.mark.parametrize("rows,cols,q", [(2048, 768, 2), (203, 1024, 9)])
def test_matvecT_formats_and_shapes(dev, ref, kind, rows, cols, q):
    """W^T y over every tile format, with the side-word decode (FP8 128 x 128,
    MXFP4, INT4 group 128) and the element decode (FP8 16 x 8, INT4 group
    16, INT8, symmetric INT4 ...): C4's expert down_proj shape with the
    rank-2 edit's q, and a ragged matrix with q = 9 (three passes of the
    accumulators); a row whose y is 0 in every direction contributes
    nothing."""
    rng = np.random.default_rng(rows + cols + q)
    w = wg.make(kind, rows, cols, rng)
    y = rng.standard_normal((q, rows)).astype(np.float32)
    y[:, 5] = 0.0
    close(dev.matvecTMulti(w, y), ref.matvecTMulti(w, y), **TOL_MATMUL)


def test_matvecT_skips_zero_rows_of_non_finite_weights(dev, ref):
    """A row of NaN / infinite weights (MXFP4 scale byte 255) whose y is 0
    in every direction is skipped, as tensor.matvecTMulti skips it
    (tensor.zig:1056-1094): the product stays finite; with y non-zero there
    it is not finite."""
    rng = np.random.default_rng(31)
    rows, cols = 96, 256
    w = wg.mxfp4_random(rows, cols, rng)
    w.arrays[1][7, 2] = 255
    y = rng.standard_normal((2, rows)).astype(np.float32)
    y[:, 7] = 0.0
    got = dev.matvecTMulti(w, y)
    assert np.isfinite(got).all()
    close(got, ref.matvecTMulti(w, y), **TOL_MATMUL)
    y[1, 7] = 1.0
    assert not np.isfinite(dev.matvecTMulti(w, y)[1]).all()


def test_kl_rows(dev, ref):
    rng = np.random.default_rng(17)
    base = rng.standard_normal((4, 5000)).astype(np.float32) * 2
    lb = ref.log_softmax_rows(base)
    trial = base + rng.standard_normal(base.shape).astype(np.float32) * 0.05
    close(dev.klRows(lb, trial), ref.kl_rows(lb, trial), atol=1e-9, rtol=1e-5)
    assert np.abs(dev.klRows(lb, base)).max() < 1e-6


def test_edit_delta(dev, ref):
    rng = np.random.default_rng(18)
    for kind in ("bf16", "int4", "mxfp4"):
        w = wg.make(kind, 96, 256, rng)
        v, _ = np.linalg.qr(rng.standard_normal((96, 2)))
        v = v.T.astype(np.float32)
        a, b = dev.edit_delta(w, v, 1.0)
        ra, rb = ref.edit_delta(w, v, 1.0)
        close(a, ra, **TOL_MATMUL)
        np.testing.assert_array_equal(b, rb)


def test_errors_are_reported_not_raised(dev):
    """Bad arguments come back as status codes with a message."""
    from ditch_amd.hip import DeviceError
    from ditch_amd.weights import HostWeight
    bad = HostWeight.fp8(np.zeros((64, 64), np.uint8), np.ones((1, 1), np.float32), 128, 128)
    bad.struct.scale_rows = 0
    with pytest.raises(DeviceError):
        dev.matmulT(np.zeros((1, 64), np.float32), bad)


# the reference's device-contract sweep (selftest.zig:121-134, 159-177):
# N(0,1) weights stored as f32/f16/bf16, N(0,1) activations
SELFTEST_SHAPES = [(1, 1, 1), (1, 1, 16), (1, 3, 17), (1, 16, 16), (1, 64, 128), (2, 17, 33), (4, 32, 64),
                   (5, 65, 31), (8, 128, 256), (13, 37, 48)]


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_selftest_matmul_sweep(dev, ref, dtype):
    rng = np.random.default_rng(99)
    for n, rows, cols in SELFTEST_SHAPES:
        w = wg.float_random(dtype, rows, cols, rng, scale=1.0)
        x = rng.standard_normal((n, cols)).astype(np.float32)
        close(dev.matmulT(x, w), ref.matmulT(x, w), **TOL_MATMUL)


def test_tensor_dequant_refuses_a_short_buffer(dev):
    """The decode of plain bf16 weights writes f32: a buffer sized for bf16
    output is refused on the host before any kernel runs."""
    from ditch_amd.hip import DeviceError
    from ditch_amd.hipmem import Buffer
    w = wg.float_random("bf16", 64, 128, np.random.default_rng(1))
    t = dev.upload(w)
    short = Buffer(64 * 128 * 2)
    try:
        with pytest.raises(DeviceError):
            t.dequant_device(short.ptr, short.nbytes, 0, 64)
    finally:
        short.free()
        t.free()


# -- the large-batch tiled product (n >= 128): split activations + LDS-staged MFMA ----------

TILE_KINDS = ["bf16", "fp8", "mxfp4", "int4", "int4_sym", "mxfp4_t", "int8", "fp8_16x8", "q8_0", "f32"]
# (257, 48, 1024), (40, 600, 2048) and (64, 520, 3072) split K over blocks
# (partial sums added by a second kernel); 40 and 64 tokens fill part of one
# 64-token tile
TILE_SHAPES = [(128, 256, 512), (200, 300, 640), (257, 48, 1024), (130, 1000, 384), (300, 17, 128),
               (40, 600, 2048), (64, 520, 3072)]


@pytest.mark.parametrize("kind", TILE_KINDS)
@pytest.mark.parametrize("n,rows,cols", TILE_SHAPES)
def test_matmulT_large_batch_matches_oracle(dev, ref, kind, n, rows, cols):
    """Shapes that reach the tiled kernel (ragged tokens, rows and k stages
    included); formats it does not take run on the small-batch kernels."""
    rng = np.random.default_rng(n * 131 + rows * 7 + cols)
    w = wg.make(kind, rows, cols, rng)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    close(dev.matmulT(x, w), ref.matmulT(x, w), **TOL_MATMUL)


def split_bound(kind, x, wf):
    """Bound on |product - exact product| from the activation split of the
    large-batch products: two bf16 terms leave |x - t0 - t1| <= 2^-18 |x|
    per activation (bounded with a factor 4 of margin: 2^-16 sum_k |x||w|);
    four fp6 terms over E8M0 block scales (MXFP4) leave at most 15^-4 of the
    block's max |x| (bounded by 2^-15 sum_blocks max|x| sum_k |w|)."""
    x64, w64 = np.abs(x).astype(np.float64), np.abs(wf).astype(np.float64)
    if kind != "mxfp4":
        return 2.0 ** -16 * (x64 @ w64.T)
    n, cols = x.shape
    pad = -cols % 32
    xm = np.pad(x64, ((0, 0), (0, pad))).reshape(n, -1, 32).max(-1)
    ws = np.pad(w64, ((0, 0), (0, pad))).reshape(w64.shape[0], -1, 32).sum(-1)
    return 2.0 ** -15 * (xm @ ws.T)


def dequant_f32(ref, w):
    wd = ref.dequant(w)
    return (wd.astype(np.uint32) << 16).view(np.float32) if wd.dtype == np.uint16 else wd


@pytest.mark.parametrize("kind", ["bf16", "fp8", "mxfp4", "int4"])
def test_matmul_device_two_term_bias_accumulate(dev, ref, kind):
    """The forward's product (activations split into two bf16 terms, or four
    fp6 terms for MXFP4 weights) on a resident tensor, with the bias and
    accumulate epilogue, against the oracle."""
    from ditch_amd import hipmem
    rng = np.random.default_rng(77)
    n, rows, cols = 384, 520, 1024
    w = wg.make(kind, rows, cols, rng)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    bias = rng.standard_normal(rows).astype(np.float32)
    prior = rng.standard_normal((n, rows)).astype(np.float32)
    t = dev.upload(w)
    try:
        bx, bb, bo = hipmem.Buffer.from_array(x), hipmem.Buffer.from_array(bias), hipmem.Buffer.from_array(prior)
        t.matmul_device(bo.ptr, bx.ptr, n, d_bias=bb.ptr, accumulate=True)
        dev.sync()
        got = bo.download(np.float32, (n, rows))
    finally:
        t.free()
    want = (prior.astype(np.float64) + ref.matmulT(x, w).astype(np.float64) + bias)
    split = split_bound(kind, x, dequant_f32(ref, w))
    bad = np.abs(got - want) > TOL_MATMUL["atol"] + TOL_MATMUL["rtol"] * np.abs(want) + split
    assert not bad.any(), f"{bad.sum()} outside the split bound"
    assert np.abs(got - want).max() < 1e-3 * np.abs(want).max()


@pytest.mark.parametrize("exp_field", [246, 248])
def test_int4_bf16_scales_at_the_fast_decode_bound(dev, ref, exp_field):
    """INT4 with bf16 scales of magnitude 2^119 (the tiled product's decode,
    q s - z s in one fused multiply-add, still takes them) and 2^121 (past
    its 2^120 bound: the exact decoder's product), activations scaled down
    to keep the sums finite, against the oracle."""
    from ditch_amd import hipmem
    rng = np.random.default_rng(exp_field)
    n, rows, cols = 64, 136, 512
    w = wg.int_random(rows, cols, rng, scale_kind="bf16")
    sc = w.arrays[1]  # the bf16 scale bits (the weight points at this array)
    sc[...] = (sc & 0x807F) | (exp_field << 7)
    x = (rng.standard_normal((n, cols)) * 2.0 ** (127 - exp_field)).astype(np.float32)
    t = dev.upload(w)
    try:
        bx, bo = hipmem.Buffer.from_array(x), hipmem.Buffer.from_array(np.zeros((n, rows), np.float32))
        t.matmul_device(bo.ptr, bx.ptr, n)
        dev.sync()
        got = bo.download(np.float32, (n, rows))
    finally:
        t.free()
    want = ref.matmulT(x, w).astype(np.float64)
    assert np.isfinite(got).all()
    split = split_bound("int4", x, dequant_f32(ref, w))
    bad = np.abs(got - want) > TOL_MATMUL["atol"] + TOL_MATMUL["rtol"] * np.abs(want) + split
    assert not bad.any(), f"{bad.sum()} outside the split bound"


@pytest.mark.parametrize("n,rows,cols", [(1, 72, 512), (2, 1000, 2880), (3, 33, 4096), (4, 520, 8192), (4, 17, 256),
                                         (32, 72, 512), (33, 1000, 2880), (64, 520, 3072), (65, 136, 576),
                                         (128, 64, 4096), (129, 520, 1024), (200, 300, 640), (256, 1040, 2048)])
def test_q8_0_few_and_mid_batch_product_bias_accumulate(dev, ref, n, rows, cols):
    """The few-token Q8_0 product (1..4 tokens, the GEMV) and the mid-batch
    one (32..256 tokens: one workgroup per 64 weight rows and every token, K
    split over its waves and added in LDS):
    ragged tokens, rows, columns and k slices, with the bias and accumulate
    epilogue, against the oracle within the two-term split bound."""
    from ditch_amd import hipmem
    rng = np.random.default_rng(n * 17 + rows + cols)
    w = wg.make("q8_0", rows, cols, rng)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    bias = rng.standard_normal(rows).astype(np.float32)
    prior = rng.standard_normal((n, rows)).astype(np.float32)
    t = dev.upload(w)
    try:
        bx, bb, bo = hipmem.Buffer.from_array(x), hipmem.Buffer.from_array(bias), hipmem.Buffer.from_array(prior)
        t.matmul_device(bo.ptr, bx.ptr, n, d_bias=bb.ptr, accumulate=True)
        dev.sync()
        got = bo.download(np.float32, (n, rows))
    finally:
        t.free()
    want = (prior.astype(np.float64) + ref.matmulT(x, w).astype(np.float64) + bias)
    split = split_bound("q8_0", x, dequant_f32(ref, w))
    bad = np.abs(got - want) > TOL_MATMUL["atol"] + TOL_MATMUL["rtol"] * np.abs(want) + split
    assert not bad.any(), f"{bad.sum()} outside the split bound"
    assert np.abs(got - want).max() < 1e-3 * np.abs(want).max()


@pytest.mark.parametrize("kind,n,rows,cols", [("bf16", 200, 136, 576), ("fp8", 130, 520, 576),
                                               ("mxfp4", 256, 520, 640), ("int4", 321, 72, 1024)])
def test_matmul_frags_device_matches_matmul_device(dev, kind, n, rows, cols):
    """ditch_hip_split_device + ditch_hip_matmulT_frags_device run the same
    large-batch product as ditch_hip_matmulT_device: bit-identical outputs,
    bias and accumulate included (K padded past the product's own stage
    count, ragged token count); the fragment size follows the tensor's
    format (bf16 terms, or fp6 terms for MXFP4)."""
    from ditch_amd import hipmem
    from ditch_amd.hip import DeviceError
    rng = np.random.default_rng(13)
    w = wg.make(kind, rows, cols, rng)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    bias = rng.standard_normal(rows).astype(np.float32)
    prior = rng.standard_normal((n, rows)).astype(np.float32)
    t = dev.upload(w)
    try:
        fb = t.frag_bytes(n)
        if kind == "mxfp4":  # [n/16][cols/128] x 6400 B (four fp6 terms + scales)
            assert fb == -(-n // 16) * -(-cols // 128) * 6400
        else:  # [n/16][cols/128 * 4 k tiles][2 terms] x 1 KiB
            assert fb == -(-n // 16) * (-(-cols // 128) * 4) * 2 * 1024
        assert t.frag_bytes(16) == 0
        bx, bb = hipmem.Buffer.from_array(x), hipmem.Buffer.from_array(bias)
        o1, o2 = hipmem.Buffer.from_array(prior), hipmem.Buffer.from_array(prior)
        xs = hipmem.Buffer(fb)
        t.matmul_device(o1.ptr, bx.ptr, n, d_bias=bb.ptr, accumulate=True)
        t.split_device(xs.ptr, fb, bx.ptr, n)
        t.matmul_frags_device(o2.ptr, xs.ptr, n, d_bias=bb.ptr, accumulate=True)
        dev.sync()
        a, b = o1.download(np.float32, (n, rows)), o2.download(np.float32, (n, rows))
        with pytest.raises(DeviceError, match="too small"):
            t.split_device(xs.ptr, fb - 1, bx.ptr, n)
        with pytest.raises(DeviceError, match="Unsupported"):
            t.split_device(xs.ptr, fb, bx.ptr, 16)
        with pytest.raises(DeviceError, match="Unsupported"):
            t.matmul_frags_device(o2.ptr, xs.ptr, 16)
    finally:
        t.free()
    assert np.array_equal(a, b)


MX_CASES = {
    # n, rows, cols, activation generator
    "ragged": (131, 72, 576, lambda rng, n, c: rng.standard_normal((n, c))),
    "outliers": (256, 136, 1024, lambda rng, n, c: rng.standard_normal((n, c)) * np.where(
        rng.random((n, c)) < 0.01, 300.0, 1.0)),
    "wide_range": (128, 64, 512, lambda rng, n, c: rng.standard_normal((n, c)) * 2.0 ** rng.integers(-60, 60, (n, c))),
    "zero_blocks": (160, 48, 384, lambda rng, n, c: rng.standard_normal((n, c)) * (np.arange(c) // 32 % 3 != 0)),
}


@pytest.mark.parametrize("case", sorted(MX_CASES))
def test_mxfp4_scaled_mfma_product(dev, ref, case):
    """MXFP4 on the scaled MFMA (fp6 activation terms x the fp4 codes with
    both E8M0 scales) against the oracle, within the four-term split bound:
    ragged tokens and K, outlier channels, activations over 2^+-60, all-zero
    32-blocks."""
    from ditch_amd import hipmem
    n, rows, cols, gen = MX_CASES[case]
    rng = np.random.default_rng(sum(map(ord, case)))
    w = wg.make("mxfp4", rows, cols, rng)
    x = gen(rng, n, cols).astype(np.float32)
    t = dev.upload(w)
    try:
        assert t.frag_bytes(n) > 0
        bx, bo = hipmem.Buffer.from_array(x), hipmem.Buffer(n * rows * 4)
        t.matmul_device(bo.ptr, bx.ptr, n)
        dev.sync()
        got = bo.download(np.float32, (n, rows))
    finally:
        t.free()
    want = ref.matmulT(x, w).astype(np.float64)
    wf = dequant_f32(ref, w)
    bound = split_bound("mxfp4", x, wf) + 1e-5 * (np.abs(x).astype(np.float64) @ np.abs(wf).astype(np.float64).T)
    bad = np.abs(got - want) > bound + 1e-30
    assert not bad.any(), f"{bad.sum()} outside the MX split bound (max excess {(np.abs(got - want) - bound).max():.3g})"


def test_mxfp4_scaled_mfma_non_finite_activation_gives_nan_rows(dev, ref):
    """A NaN or infinity among an activation block's 32 values makes that
    token's outputs NaN on the scaled-MFMA path (E8M0 255); other tokens are
    unaffected."""
    from ditch_amd import hipmem
    rng = np.random.default_rng(3)
    n, rows, cols = 128, 32, 256
    w = wg.make("mxfp4", rows, cols, rng)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    x[5, 77] = np.nan
    x[9, 200] = np.inf
    t = dev.upload(w)
    try:
        bx, bo = hipmem.Buffer.from_array(x), hipmem.Buffer(n * rows * 4)
        t.matmul_device(bo.ptr, bx.ptr, n)
        dev.sync()
        got = bo.download(np.float32, (n, rows))
    finally:
        t.free()
    assert np.isnan(got[5]).all() and np.isnan(got[9]).all()
    keep = np.ones(n, bool)
    keep[[5, 9]] = False
    assert np.isfinite(got[keep]).all()


def test_matmulT_large_batch_nan_scale_takes_the_exact_decoder(dev, ref):
    """An E8M0 scale byte 255 (NaN block, dequant.zig:259-261) keeps the
    tensor off the conversion instructions; the NaN rows match the oracle."""
    rng = np.random.default_rng(5)
    w = wg.mxfp4_random(64, 256, rng)
    w.arrays[1][3, 2] = 255  # the scale array the weight struct points at
    x = rng.standard_normal((160, 256)).astype(np.float32)
    got, want = dev.matmulT(x, w), ref.matmulT(x, w)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    close(got[fin], want[fin], **TOL_MATMUL)
