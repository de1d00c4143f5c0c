"""The device decoders on the closed-form cases of test_oracle_pins.py: the
raw-layout decode and the re-tiled HBM layout give the encoder's target
bits directly (no oracle in between) for MXFP4 (natural, several blocks a
row, and the gpt-oss transposed layout), FP8 with every scale-grid dtype
and row shards, and pack-quantized INT at 2, 3, 5 and 8 bits."""
import numpy as np
import pytest

from ditch_amd.hipmem import Buffer
from test_oracle_pins import (INT_CASES, fp8_grid_case, fp8_shard_case, int_case, mxfp4_natural_case,
                              mxfp4_transposed_case)

pytestmark = pytest.mark.gpu

CASES = [("mxfp4_natural", lambda r: mxfp4_natural_case(r)),
         ("mxfp4_transposed", lambda r: mxfp4_transposed_case(r)),
         ("mxfp4_natural_wide", lambda r: mxfp4_natural_case(r, rows=37, cols=1024))]
CASES += [(f"fp8_{k}{'_e5m2' if e else ''}", (lambda k, e: lambda r: fp8_grid_case(r, k, e5m2=e))(k, e))
          for k in ("f32", "bf16", "f16", "e8m0") for e in (False, True)]
CASES += [("fp8_row_shard", lambda r: fp8_shard_case(r))]
CASES += [(f"int_{i}_{kw['bits']}b", (lambda kw: lambda r: int_case(r, **kw))(kw)) for i, kw in enumerate(INT_CASES)]


@pytest.mark.parametrize("name,make", CASES, ids=[c[0] for c in CASES])
def test_device_decode_equals_closed_form(dev, name, make):
    w, want = make(np.random.default_rng(len(name) * 31 + 7))
    np.testing.assert_array_equal(dev.dequant(w), want)
    t = dev.upload(w)
    try:
        buf = Buffer(want.nbytes)
        t.dequant_device(buf.ptr, buf.nbytes, 0, w.rows)
        dev.sync()
        np.testing.assert_array_equal(buf.download(want.dtype, want.shape), want)
        buf.free()
    finally:
        t.free()
