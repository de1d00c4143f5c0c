"""Closed-form pins of the oracle's quantised-safetensors decoders on the
layouts the reference's own tests do not reach (dequant.zig:471-673).

Each check builds the packed tensor with an independent ENCODER written from
the format's definition (numpy bit streams, torch's float8 and bfloat16
casts), from a known target matrix, and requires the oracle to decode it
back bit for bit:

  * MXFP4 natural layout (dequant.zig:643-673): several 32-column blocks per
    row, a distinct E8M0 byte for every (row, block);
  * MXFP4 gpt-oss layout (dequant.zig:603-637): `_blocks` [src_rows]
    [src_cols/32][16] of the transposed matrix, scales [src_rows][src_cols/32];
  * FP8 (dequant.zig:471-514): f32, bf16, f16 and E8M0 scale grids with
    partial edge blocks, and `row_shard` (every shard its own scale grid);
  * pack-quantized INT (dequant.zig:313-321, 518-597) at 2, 3, 5 and 8 bits,
    zero points packed along rows, f16/bf16/f32 scales, and actorder g_idx.

test_planted_mistakes_fail_the_pins compiles copies of the oracle with one
plausible mistake each (an index or a layout misread) and requires the pins
to reject every copy.
"""
import os
import shutil
import subprocess
import tempfile

import numpy as np
import pytest
import torch

from ditch_amd.weights import HostWeight

E2M1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], dtype=np.float64)
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def bf16_bits(x64):
    """Round-to-nearest-even bfloat16 bit patterns of float64 values (torch)."""
    t = torch.from_numpy(np.ascontiguousarray(x64, dtype=np.float64)).to(torch.float32).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def bitstream_words(fields, bits):
    """pack_to_int32: fields of `bits` bits laid one after the other from bit 0
    of a little-endian stream of 32-bit words (zero padded)."""
    fields = np.asarray(fields, dtype=np.uint64)
    bit_idx = np.arange(bits, dtype=np.uint64)
    stream = ((fields[:, None] >> bit_idx[None, :]) & 1).astype(np.uint8).reshape(-1)
    nwords = -(-stream.size // 32)
    stream = np.concatenate([stream, np.zeros(nwords * 32 - stream.size, dtype=np.uint8)])
    return np.packbits(stream, bitorder="little").view("<u4").astype(np.uint32)


# ---------------------------------------------------------------------------
# MXFP4


def mxfp4_natural_case(rng, rows=6, cols=256):
    codes = rng.integers(0, 16, size=(rows, cols))
    nblk = cols // 32
    # distinct for up to 150 blocks, always finite (byte 255 is a NaN scale)
    sc = (60 + rng.permutation(rows * nblk) % 150).astype(np.uint8).reshape(rows, nblk)
    target = E2M1[codes] * np.exp2(np.repeat(sc.astype(np.float64), 32, axis=1) - 127)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)  # low nibble = even column
    return HostWeight.mxfp4(packed, sc), bf16_bits(target)


def mxfp4_transposed_case(rng, rows=96, cols=40):
    """View [rows][cols] = the transpose of the stored source [cols][rows]."""
    src = rng.integers(0, 16, size=(cols, rows))  # source codes [src_rows][src_cols]
    nblk = rows // 32
    sc = (60 + rng.permutation(cols * nblk) % 150).astype(np.uint8).reshape(cols, nblk)
    src_vals = E2M1[src] * np.exp2(np.repeat(sc.astype(np.float64), 32, axis=1) - 127)
    pairs = (src[:, 0::2] | (src[:, 1::2] << 4)).astype(np.uint8)  # [src_rows][src_cols/2]
    blocks = pairs.reshape(cols, nblk, 16)
    return HostWeight.mxfp4_t(blocks, sc), bf16_bits(src_vals.T)


def check_mxfp4(ref, rng):
    for case in (mxfp4_natural_case, mxfp4_transposed_case):
        w, want = case(rng)
        np.testing.assert_array_equal(ref.dequant(w), want, err_msg=case.__name__)


def test_mxfp4_natural_multiblock(ref):
    w, want = mxfp4_natural_case(np.random.default_rng(1))
    np.testing.assert_array_equal(ref.dequant(w), want)
    # a row range decodes just its rows (readMxfp4Packed's row chunks)
    np.testing.assert_array_equal(ref.dequant(w, 2, 3), want[2:5])


def test_mxfp4_transposed_layout(ref):
    w, want = mxfp4_transposed_case(np.random.default_rng(2))
    assert (w.rows, w.cols) == want.shape
    np.testing.assert_array_equal(ref.dequant(w), want)
    np.testing.assert_array_equal(ref.dequant(w, 33, 10), want[33:43])


# ---------------------------------------------------------------------------
# FP8


def _fp8_codes(rng, rows, cols, e5m2=False):
    """Finite codes and their values by torch's float8 cast."""
    codes = rng.integers(0, 256, size=(rows, cols)).astype(np.uint8)
    dt = torch.float8_e5m2 if e5m2 else torch.float8_e4m3fn
    vals = torch.from_numpy(codes).view(dt).to(torch.float64).numpy()
    bad = ~np.isfinite(vals)
    codes[bad] = 0x30
    vals[bad] = torch.tensor([0x30], dtype=torch.uint8).view(dt).to(torch.float64).item()
    return codes, vals


def _grid_values(rng, kind, shape):
    """A scale grid whose entries are exact in `kind`: (stored array, f64 values)."""
    if kind == "e8m0":
        b = (110 + rng.permutation(np.prod(shape)) % 30).astype(np.uint8).reshape(shape)
        return ("e8m0", b), np.exp2(b.astype(np.float64) - 127)
    v = rng.uniform(0.5, 2.0, size=shape) * np.exp2(rng.integers(-12, -4, size=shape))
    if kind == "f16":
        a = v.astype(np.float16)
        return a, a.astype(np.float64)
    if kind == "bf16":
        bits = bf16_bits(v)
        return ("bf16", bits), (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    a = v.astype(np.float32)
    return a, a.astype(np.float64)


def fp8_grid_case(rng, kind, rows=40, cols=52, br=16, bc=8, e5m2=False):
    codes, vals = _fp8_codes(rng, rows, cols, e5m2)
    gshape = (-(-rows // br), -(-cols // bc))
    stored, g = _grid_values(rng, kind, gshape)
    full = np.repeat(np.repeat(g, br, axis=0), bc, axis=1)[:rows, :cols]
    want = bf16_bits((vals * full).astype(np.float32).astype(np.float64))
    return HostWeight.fp8(codes, stored, br, bc, e5m2=e5m2), want


def fp8_shard_case(rng, shards=3, rs=20, cols=24, br=16, bc=8):
    """A row-sharded matrix (fused projections): shard i is rows [i*rs, (i+1)*rs)
    with its own grid of ceil(rs/br) scale rows; the grids are stacked."""
    codes, vals = _fp8_codes(rng, shards * rs, cols)
    per = -(-rs // br)
    grids, fulls = [], []
    for _ in range(shards):
        stored, g = _grid_values(rng, "f32", (per, -(-cols // bc)))
        grids.append(stored)
        fulls.append(np.repeat(np.repeat(g, br, axis=0), bc, axis=1)[:rs, :cols])
    scale = np.vstack(grids)
    want = bf16_bits((vals * np.vstack(fulls)).astype(np.float32).astype(np.float64))
    return HostWeight.fp8(codes, scale, br, bc, row_shard=rs), want


def check_fp8(ref, rng):
    for kind in ("f32", "bf16", "f16", "e8m0"):
        w, want = fp8_grid_case(rng, kind)
        np.testing.assert_array_equal(ref.dequant(w), want, err_msg=kind)
    w, want = fp8_shard_case(rng)
    np.testing.assert_array_equal(ref.dequant(w), want, err_msg="row_shard")


@pytest.mark.parametrize("kind", ["f32", "bf16", "f16", "e8m0"])
@pytest.mark.parametrize("e5m2", [False, True])
def test_fp8_scale_grids(ref, kind, e5m2):
    w, want = fp8_grid_case(np.random.default_rng(3), kind, e5m2=e5m2)
    np.testing.assert_array_equal(ref.dequant(w), want)
    np.testing.assert_array_equal(ref.dequant(w, 15, 9), want[15:24])


def test_fp8_row_shard(ref):
    w, want = fp8_shard_case(np.random.default_rng(4))
    np.testing.assert_array_equal(ref.dequant(w), want)


# ---------------------------------------------------------------------------
# pack-quantized INT


def int_case(rng, bits, rows=13, cols=96, group=32, zero=True, scale_kind="f16", actorder=False):
    nf = 1 << bits
    off = nf >> 1
    fields = rng.integers(0, nf, size=(rows, cols))
    groups = -(-cols // group)
    g_idx = rng.integers(0, groups, size=cols).astype(np.int32) if actorder else None
    col_group = g_idx if actorder else np.arange(cols) // group
    zf = rng.integers(0, nf, size=(rows, groups)) if zero else np.full((rows, groups), off)
    stored, sv = _grid_values(rng, scale_kind, (rows, groups))
    words = np.stack([bitstream_words(fields[r], bits) for r in range(rows)])
    zw = np.stack([bitstream_words(zf[:, g], bits) for g in range(groups)], axis=1) if zero else None
    q = fields.astype(np.int64) - off
    zp = zf.astype(np.int64)[:, col_group] - off
    want = bf16_bits(((q - zp) * sv[:, col_group]).astype(np.float32).astype(np.float64))
    w = HostWeight.int_packed(words.view(np.int32), stored, rows, cols, bits, group,
                              zero=None if zw is None else zw.view(np.int32), g_idx=g_idx)
    return w, want


INT_CASES = [dict(bits=2), dict(bits=3), dict(bits=5), dict(bits=8), dict(bits=3, zero=False),
             dict(bits=5, scale_kind="bf16"), dict(bits=8, scale_kind="f32"), dict(bits=3, actorder=True),
             dict(bits=4, actorder=True, scale_kind="bf16")]


def check_int(ref, rng):
    for kw in INT_CASES:
        w, want = int_case(rng, **kw)
        np.testing.assert_array_equal(ref.dequant(w), want, err_msg=str(kw))


@pytest.mark.parametrize("kw", INT_CASES, ids=[str(k) for k in INT_CASES])
def test_int_packed_widths(ref, kw):
    w, want = int_case(np.random.default_rng(5), **kw)
    np.testing.assert_array_equal(ref.dequant(w), want)
    np.testing.assert_array_equal(ref.dequant(w, 4, 6), want[4:10])


def test_bitstream_packer_matches_the_reference_known_answers():
    """The encoder above against unpackField's own test (dequant.zig:1301-1310):
    4-bit fields 0..15 fill 0x76543210, 0xfedcba98; a 3-bit field 10 spans
    bits 30..32."""
    np.testing.assert_array_equal(bitstream_words(np.arange(16), 4), [0x76543210, 0xFEDCBA98])
    f = np.zeros(11, dtype=np.uint64)
    f[10] = 0b101
    np.testing.assert_array_equal(bitstream_words(f, 3), [0b01 << 30, 1])


# ---------------------------------------------------------------------------
# The pins reject plausible mistakes (planted in copies of the oracle, CPU only)

MUTANTS = {
    "mxfp4 scale row stride dropped":
        ("const uint8_t *srow = (const uint8_t *)w->scale + r * nblk;",
         "const uint8_t *srow = (const uint8_t *)w->scale + r;"),
    "mxfp4 nibble order swapped":
        ("dst[k * 32 + 2 * j] = ref_f32_to_bf16(e2m1_table[b & 0x0f] * sc);",
         "dst[k * 32 + 2 * j] = ref_f32_to_bf16(e2m1_table[b >> 4] * sc);"),
    "mxfp4_t scales read transposed":
        ("float sc = ref_e8m0_scale(scales[j * nblk + k]);",
         "float sc = ref_e8m0_scale(scales[k * src_rows + j]);"),
    "fp8 row shards ignored":
        ("if (w->row_shard == 0) return r / w->block_rows;", "return r / w->block_rows;"),
    "fp8 grid column by block_rows":
        ("srow * w->scale_cols + c / w->block_cols", "srow * w->scale_cols + c / w->block_rows"),
    "bf16 scales widened as f16":
        ("case DITCH_BF16: return ref_bf16_to_f32(((const uint16_t *)base)[idx]);",
         "case DITCH_BF16: return ref_f16_to_f32(((const uint16_t *)base)[idx]);"),
    "int offset fixed at 4 bits":
        ("int offset = 1 << (bits - 1);", "int offset = 8;"),
    "int zero point straddle word":
        ("if (lo < bits) v |= (zw[(wi + 1) * groups + g] & field_mask(bits - lo)) << lo;",
         "if (lo < bits) v |= (zw[wi * groups + g + 1] & field_mask(bits - lo)) << lo;"),
}


def _build_mutant(tmp, name, old, new):
    src = open(os.path.join(ROOT, "oracle", "cpu_ref.c")).read()
    assert src.count(old) == 1, f"mutant '{name}': the oracle text it changes is gone"
    d = os.path.join(tmp, name.replace(" ", "_"))
    os.makedirs(os.path.join(d, "oracle"))
    os.makedirs(os.path.join(d, "include"))
    open(os.path.join(d, "oracle", "cpu_ref.c"), "w").write(src.replace(old, new))
    shutil.copy(os.path.join(ROOT, "oracle", "cpu_ref.h"), os.path.join(d, "oracle"))
    shutil.copy(os.path.join(ROOT, "include", "ditch_hip.h"), os.path.join(d, "include"))
    so = os.path.join(d, "mutant.so")
    subprocess.run(["gcc", "-O1", "-fPIC", "-shared", "-std=c11", "-ffp-contract=off", "-o", so,
                    os.path.join(d, "oracle", "cpu_ref.c"), "-lm", "-lpthread"], check=True)
    return so


def test_planted_mistakes_fail_the_pins():
    from oracle.ref import Ref
    with tempfile.TemporaryDirectory() as tmp:
        survivors = []
        for name, (old, new) in MUTANTS.items():
            r = Ref(path=_build_mutant(tmp, name, old, new))
            caught = False
            for check in (check_mxfp4, check_fp8, check_int):
                try:
                    check(r, np.random.default_rng(7))
                except AssertionError:
                    caught = True
            if not caught:
                survivors.append(name)
        assert not survivors, f"mistakes the pins do not catch: {survivors}"
