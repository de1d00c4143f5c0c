"""ditch_hip_matmulT_device_noalloc (scratch in the library's static device
array, no allocation) against ditch_hip_matmulT_device on the same inputs:
two calls in a row, the second smaller, over the product's paths (GEMV with
and without term staging, the generic GEMM, the tiled product with split-K,
the scaled-MFMA product, and a product whose split-K partial sums do not fit
the scratch, which then runs unsplit). The bar is the product tolerance of
the VTable products (abs 1e-4, rel 1e-3 of the output scale); where the two
calls pick the same kernels the outputs are identical. Calls on two streams
are ordered through the one scratch array, and calls captured into a HIP
graph (global capture mode: an allocation would end the capture with an
error) give, on every replay, the allocating product's outputs."""
import ctypes

import numpy as np
import pytest
import torch

from ditch_amd import hipmem, synth
from ditch_amd.hip import DeviceError

pytestmark = pytest.mark.gpu

CASES = {
    # name: (format, rows, cols, n first call, n second call, identical)
    "gemv_bf16": ("bf16", 1000, 2048, 12, 3, True),
    "gemm_fp8": ("fp8", 520, 1024, 24, 17, True),
    "tiled_splitk_fp8": ("fp8", 4096, 4096, 64, 48, True),
    "mx_mxfp4": ("mxfp4", 2048, 4096, 256, 160, True),
    "tiled_int4": ("int4", 1536, 2048, 200, 33, True),
    "unsplit_q8_0": ("q8_0", 14336, 4096, 256, 128, False),
}


def _weight(fmt, rows, cols, seed):
    gen = torch.Generator().manual_seed(seed)
    if fmt == "q8_0":
        return synth.q8_0_random(rows, cols, gen)
    return synth.QUANTIZERS[fmt](torch.randn(rows, cols, generator=gen) * 0.02)


@pytest.mark.parametrize("name", list(CASES))
def test_noalloc_matches_matmul_device(dev, name):
    fmt, rows, cols, n1, n2, identical = CASES[name]
    t = dev.upload(_weight(fmt, rows, cols, len(name)))
    try:
        rng = np.random.default_rng(len(name) + 1)
        bias = hipmem.Buffer.from_array(rng.standard_normal(rows).astype(np.float32))
        for n in (n1, n2):
            x = rng.standard_normal((n, cols)).astype(np.float32)
            bx = hipmem.Buffer.from_array(x)
            o1, o2 = hipmem.Buffer(n * rows * 4), hipmem.Buffer(n * rows * 4)
            init = rng.standard_normal((n, rows)).astype(np.float32)
            o1.upload(init)
            o2.upload(init)
            t.matmul_device(o1.ptr, bx.ptr, n, d_bias=bias.ptr, accumulate=True)
            t.matmul_device_noalloc(o2.ptr, bx.ptr, n, d_bias=bias.ptr, accumulate=True)
            dev.sync()
            a = o1.download(np.float32, (n, rows))
            b = o2.download(np.float32, (n, rows))
            if identical:
                np.testing.assert_array_equal(b, a)
            else:
                # the same sums in another order: f32 rounding only
                assert np.abs(b - a).max() <= 1e-4 * max(1.0, float(np.abs(a).max())), name
    finally:
        t.free()


def test_noalloc_refuses_more_than_the_scratch(dev):
    """A batch whose activation fragments alone exceed the static scratch is
    refused before any launch; the next call still works."""
    cap = dev.lib.ditch_hip_static_scratch_bytes()
    assert cap == 64 << 20
    rows, cols = 256, 4096
    t = dev.upload(_weight("bf16", rows, cols, 3))
    try:
        n = 8192  # two bf16 terms of 8192 x 4096: 128 MiB of fragments
        bx, bo = hipmem.Buffer(n * cols * 4), hipmem.Buffer(n * rows * 4)
        with pytest.raises(DeviceError, match="static scratch holds"):
            t.matmul_device_noalloc(bo.ptr, bx.ptr, n)
        x = np.random.default_rng(4).standard_normal((40, cols)).astype(np.float32)
        bx2, o1, o2 = hipmem.Buffer.from_array(x), hipmem.Buffer(40 * rows * 4), hipmem.Buffer(40 * rows * 4)
        t.matmul_device(o1.ptr, bx2.ptr, 40)
        t.matmul_device_noalloc(o2.ptr, bx2.ptr, 40)
        dev.sync()
        np.testing.assert_array_equal(o2.download(np.float32, (40, rows)), o1.download(np.float32, (40, rows)))
    finally:
        t.free()


def test_noalloc_calls_on_two_streams_are_ordered(dev):
    """Calls alternating between two streams with different inputs (and
    different weights) share the one scratch array: each call's stream waits
    for the previous call's kernels, so every output equals the allocating
    product's on the same inputs."""
    from ditch_amd.hipmem import hip
    lib = hip()
    streams = []
    for _ in range(2):
        s = ctypes.c_void_p()
        assert lib.hipStreamCreateWithFlags(ctypes.byref(s), 1) == 0  # non-blocking, default priority
        streams.append(s)
    ts = [dev.upload(_weight("fp8", 4096, 4096, 11)), dev.upload(_weight("int4", 1536, 2048, 12))]
    try:
        rng = np.random.default_rng(13)
        jobs = []
        for i in range(6):
            t = ts[i % 2]
            rows, cols = (4096, 4096) if i % 2 == 0 else (1536, 2048)
            n = (64, 200, 48, 33, 96, 130)[i]
            x = rng.standard_normal((n, cols)).astype(np.float32)
            bx = hipmem.Buffer.from_array(x)
            want, got = hipmem.Buffer(n * rows * 4), hipmem.Buffer(n * rows * 4)
            jobs.append((t, n, rows, bx, want, got, streams[i % 2]))
        for t, n, rows, bx, want, got, s in jobs:
            t.matmul_device_noalloc(got.ptr, bx.ptr, n, stream=s.value)
        for s in streams:
            assert lib.hipStreamSynchronize(s) == 0
        for t, n, rows, bx, want, got, s in jobs:
            t.matmul_device(want.ptr, bx.ptr, n)
        dev.sync()
        for t, n, rows, bx, want, got, s in jobs:
            np.testing.assert_array_equal(got.download(np.float32, (n, rows)), want.download(np.float32, (n, rows)))
    finally:
        for t in ts:
            t.free()
        for s in streams:
            lib.hipStreamDestroy(s)


# (format, rows, cols, n): the tiled product with split-K partial sums in the
# scratch, the scaled-MFMA product, the GEMV with term staging
GRAPH_CASES = [("fp8", 4096, 4096, 64), ("mxfp4", 2048, 4096, 256), ("bf16", 1000, 2048, 12)]


@pytest.mark.parametrize("first,second", [(0, 1), (1, 2)])
def test_noalloc_products_replayed_from_a_graph(dev, first, second):
    """Two products (different weights, inputs and paths) captured on one
    stream, the graph replayed three times with new inputs uploaded between
    the replays: every replay equals the allocating product on its inputs."""
    from ditch_amd.hipmem import hip
    lib = hip()
    P = ctypes.c_void_p
    for name, args in {"hipStreamBeginCapture": [P, ctypes.c_int], "hipStreamEndCapture": [P, ctypes.POINTER(P)],
                       "hipGraphInstantiate": [ctypes.POINTER(P), P, P, P, ctypes.c_size_t],
                       "hipGraphLaunch": [P, P], "hipGraphExecDestroy": [P], "hipGraphDestroy": [P]}.items():
        getattr(lib, name).argtypes = args
        getattr(lib, name).restype = ctypes.c_int
    stream = ctypes.c_void_p()
    assert lib.hipStreamCreateWithFlags(ctypes.byref(stream), 1) == 0  # non-blocking, default priority
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    cases = [GRAPH_CASES[first], GRAPH_CASES[second]]
    ts = [dev.upload(_weight(f, r, c, 20 + i)) for i, (f, r, c, n) in enumerate(cases)]
    try:
        rng = np.random.default_rng(21)
        bufs = []
        for (f, r, c, n) in cases:
            bx = hipmem.Buffer(n * c * 4)
            bx.upload(rng.standard_normal((n, c)).astype(np.float32))
            bias = hipmem.Buffer.from_array(rng.standard_normal(r).astype(np.float32))
            bufs.append((bx, bias, hipmem.Buffer(n * r * 4), hipmem.Buffer(n * r * 4)))
        dev.sync()
        assert lib.hipStreamBeginCapture(stream, 0) == 0  # hipStreamCaptureModeGlobal
        for t, (f, r, c, n), (bx, bias, got, want) in zip(ts, cases, bufs):
            t.matmul_device_noalloc(got.ptr, bx.ptr, n, d_bias=bias.ptr, stream=stream.value)
        assert lib.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
        assert lib.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for replay in range(3):
            # new inputs (eager, on the library stream), then the graph
            for (f, r, c, n), (bx, bias, got, want) in zip(cases, bufs):
                bx.upload(rng.standard_normal((n, c)).astype(np.float32))
                got.zero()
            assert lib.hipDeviceSynchronize() == 0
            assert lib.hipGraphLaunch(exe, stream) == 0
            assert lib.hipStreamSynchronize(stream) == 0
            for t, (f, r, c, n), (bx, bias, got, want) in zip(ts, cases, bufs):
                t.matmul_device(want.ptr, bx.ptr, n, d_bias=bias.ptr)
            dev.sync()
            for (f, r, c, n), (bx, bias, got, want) in zip(cases, bufs):
                np.testing.assert_array_equal(got.download(np.float32, (n, r)), want.download(np.float32, (n, r)),
                                              err_msg=f"{f} {r}x{c} n={n}, replay {replay}")
    finally:
        if exe.value:
            lib.hipGraphExecDestroy(exe)
        if graph.value:
            lib.hipGraphDestroy(graph)
        for t in ts:
            t.free()
        lib.hipStreamDestroy(stream)
