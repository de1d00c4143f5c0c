"""The products at the benchmark configurations' full shapes, through the
C ABI, against the CPU oracle (needs an MI355X).

C2 (Q8_0 14336 x 4096 at M = 1, 4, 16, 64, 256) is compared whole; the C3
FFN product (MXFP4 14336 x 4096 on 8192 tokens) on a sample of tokens that
falls in every 96-token tile row of the scaled-MFMA product, its first and
last tokens included. Bound per element: the reference's matmul tolerance
(selftest.zig:34-41, abs 1e-4 or rel 1e-3) plus the activation split's own
(two bf16 terms: 2^-16 sum_k |x||w|; four fp6 terms over E8M0 block scales:
2^-15 sum_blocks max|x| sum_k |w|).
"""
import numpy as np
import pytest
import torch

import weights_gen as wg
from ditch_amd import synth

pytestmark = pytest.mark.gpu

TOL = dict(atol=1e-4, rtol=1e-3)


def dequant_f32(ref, w):
    wd = ref.dequant(w)
    return (wd.astype(np.uint32) << 16).view(np.float32) if wd.dtype == np.uint16 else wd


def split_bound(mx, x, wf):
    x64, w64 = np.abs(x).astype(np.float64), np.abs(wf).astype(np.float64)
    if not mx:
        return 2.0 ** -16 * (x64 @ w64.T)
    n, cols = x.shape
    xm = x64.reshape(n, cols // 32, 32).max(-1)
    ws = w64.reshape(w64.shape[0], cols // 32, 32).sum(-1)
    return 2.0 ** -15 * (xm @ ws.T)


def device_product(dev, t, x, rows):
    from ditch_amd import hipmem
    n = x.shape[0]
    bx, bo = hipmem.Buffer.from_array(x), hipmem.Buffer(n * rows * 4)
    t.matmul_device(bo.ptr, bx.ptr, n)
    dev.sync()
    return bo.download(np.float32, (n, rows))


def check(got, want, bound):
    err = np.abs(got.astype(np.float64) - want)
    bad = err > TOL["atol"] + TOL["rtol"] * np.abs(want) + bound
    assert not bad.any(), f"{bad.sum()} of {bad.size} outside the bound; worst {err.max():.3e}"
    assert err.max() < 1e-3 * np.abs(want).max()


@pytest.fixture(scope="module")
def c2(dev, ref):
    w = synth.q8_0_random(14336, 4096, torch.Generator().manual_seed(5))
    t = dev.upload(w)
    yield w, t, dequant_f32(ref, w)
    t.free()


@pytest.mark.parametrize("m", [1, 4, 16, 64, 256])
def test_c2_q8_0_full_shape(dev, ref, c2, m):
    """GEMV (M <= 16), tiled product with split-K (64, 256)."""
    w, t, wf = c2
    x = np.random.default_rng(m).standard_normal((m, 4096)).astype(np.float32)
    got = device_product(dev, t, x, 14336)
    want = ref.matmulT(x, w).astype(np.float64)
    check(got, want, split_bound(False, x, wf))


def test_c3_mxfp4_ffn_full_shape_sampled_tokens(dev, ref):
    """8192 tokens x 14336 rows x K 4096 on the scaled MFMA; tokens sampled
    in every 96-token tile row (offsets 0, 47, 95 within it, rotating)."""
    rng = np.random.default_rng(31)
    w = wg.mxfp4_random(14336, 4096, rng)
    x = rng.standard_normal((8192, 4096)).astype(np.float32)
    t = dev.upload(w)
    try:
        got = device_product(dev, t, x, 14336)
    finally:
        t.free()
    tiles = (8192 + 95) // 96
    sample = np.unique(np.clip([96 * i + (0, 47, 95)[i % 3] for i in range(tiles)] + [8191], 0, 8191))
    xs = x[sample]
    want = ref.matmulT(xs, w).astype(np.float64)
    check(got[sample], want, split_bound(True, xs, dequant_f32(ref, w)))
