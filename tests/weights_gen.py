"""Random weights of every storage format for the parity tests (seeded)."""
import numpy as np

from ditch_amd import abi
from ditch_amd.weights import HostWeight

GGUF_BLOCK = {abi.Q8_0: (32, 34), abi.Q4_0: (32, 18), abi.Q4_1: (32, 20), abi.Q5_0: (32, 22),
              abi.Q5_1: (32, 24), abi.Q4_K: (256, 144), abi.Q6_K: (256, 210), abi.Q8_K: (256, 292)}


def _f16_bytes(vals):
    return np.asarray(vals, dtype=np.float16).view(np.uint8).reshape(-1, 2)


def gguf_random(dt, rows, cols, rng, scale=0.02):
    if dt in (abi.Q4_K, abi.Q6_K):
        scale = 0.002  # k-quant sub-block scales multiply d by up to 63
    bs, bb = GGUF_BLOCK[dt]
    nb = rows * cols // bs
    raw = rng.integers(0, 256, (nb, bb), dtype=np.uint8)
    if dt == abi.Q8_K:
        raw[:, 0:4] = np.asarray(rng.uniform(0.001, 0.01, nb), dtype=np.float32).view(np.uint8).reshape(-1, 4)
    elif dt == abi.Q6_K:
        raw[:, 208:210] = _f16_bytes(rng.uniform(-scale, scale, nb))
    else:
        raw[:, 0:2] = _f16_bytes(rng.uniform(-scale, scale, nb))
        if dt in (abi.Q4_1, abi.Q5_1, abi.Q4_K):
            raw[:, 2:4] = _f16_bytes(rng.uniform(-scale, scale, nb))
    return HostWeight.gguf(dt, raw.reshape(-1), rows, cols)


def fp8_random(rows, cols, rng, block=(128, 128), scale_kind="f32", e5m2=False, all_codes=False, row_shard=0):
    codes = rng.integers(0, 256, (rows, cols), dtype=np.uint8)
    if not all_codes:  # keep NaN codes out of matmul inputs
        bad = (codes & 0x7F) == (0x7C if e5m2 else 0x7F)
        if e5m2:
            bad = (codes & 0x7C) == 0x7C
        codes[bad] = 0
    br, bc = block
    if row_shard:
        per = -(-row_shard // br)
        sr = (rows // row_shard) * per
    else:
        sr = -(-rows // br)
    sc = -(-cols // bc)
    s = rng.uniform(1e-4, 1e-2, (sr, sc)).astype(np.float32)
    if scale_kind == "f32":
        scale = s
    elif scale_kind == "f16":
        scale = s.astype(np.float16)
    elif scale_kind == "bf16":
        scale = ("bf16", (s.view(np.uint32) >> 16).astype(np.uint16))
    else:
        scale = ("e8m0", rng.integers(110, 130, (sr, sc), dtype=np.uint8))
    return HostWeight.fp8(codes, scale, br, bc, e5m2=e5m2, row_shard=row_shard)


def mxfp4_random(rows, cols, rng, scale_lo=118, scale_hi=126):
    packed = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
    scales = rng.integers(scale_lo, scale_hi, (rows, cols // 32), dtype=np.uint8)
    return HostWeight.mxfp4(packed, scales)


def mxfp4_t_random(rows, cols, rng):
    """view [rows][cols] stored transposed: blocks [cols][rows/32][16]."""
    blocks = rng.integers(0, 256, (cols, rows // 32, 16), dtype=np.uint8)
    scales = rng.integers(118, 126, (cols, rows // 32), dtype=np.uint8)
    return HostWeight.mxfp4_t(blocks, scales)


def int_random(rows, cols, rng, bits=4, group=128, zero=True, actorder=False, scale_kind="f16"):
    groups = -(-cols // group)
    fields = rng.integers(0, 1 << bits, (rows, cols), dtype=np.uint64)
    wpr = -(-cols * bits // 32)
    words = np.zeros((rows, wpr), dtype=np.uint64)
    for c in range(cols):
        start = c * bits
        w, off = start // 32, start % 32
        words[:, w] |= (fields[:, c] << off) & 0xFFFFFFFF
        if off + bits > 32:
            words[:, w + 1] |= fields[:, c] >> (32 - off)
    words = words.astype(np.uint32).view(np.int32)
    s = rng.uniform(1e-3, 2e-2, (rows, groups)).astype(np.float32)
    scale = s.astype(np.float16) if scale_kind == "f16" else (("bf16", (s.view(np.uint32) >> 16).astype(np.uint16)) if scale_kind == "bf16" else s)
    zw = None
    if zero:
        zf = rng.integers(0, 1 << bits, (rows, groups), dtype=np.uint64)
        zrows = -(-rows * bits // 32)
        zwords = np.zeros((zrows, groups), dtype=np.uint64)
        for r in range(rows):
            start = r * bits
            w, off = start // 32, start % 32
            zwords[w] |= (zf[r] << off) & 0xFFFFFFFF
            if off + bits > 32:
                zwords[w + 1] |= zf[r] >> (32 - off)
        zw = zwords.astype(np.uint32).view(np.int32)
    g_idx = None
    if actorder:
        g_idx = rng.permutation(np.arange(cols) // group).astype(np.int32)
    return HostWeight.int_packed(words, scale, rows, cols, bits, group, zero=zw, g_idx=g_idx)


def float_random(kind, rows, cols, rng, scale=0.05):
    w = (rng.standard_normal((rows, cols)) * scale).astype(np.float32)
    if kind == "f32":
        return HostWeight.f32(w)
    if kind == "f16":
        return HostWeight.f16(w.astype(np.float16))
    bits = (w.view(np.uint32) + 0x7FFF + ((w.view(np.uint32) >> 16) & 1)) >> 16
    return HostWeight.bf16(bits.astype(np.uint16))


def make(kind, rows, cols, rng):
    """A weight of `kind` for matmul parity (finite values only)."""
    if kind in ("f32", "f16", "bf16"):
        return float_random(kind, rows, cols, rng)
    if kind == "q8_0":
        return gguf_random(abi.Q8_0, rows, cols, rng)
    if kind in ("q4_0", "q4_1", "q5_0", "q5_1", "q4_k", "q6_k", "q8_k"):
        return gguf_random(getattr(abi, kind.upper()), rows, cols, rng)
    if kind == "fp8":
        return fp8_random(rows, cols, rng)
    if kind == "fp8_16x8":
        return fp8_random(rows, cols, rng, block=(16, 8))
    if kind == "mxfp4":
        return mxfp4_random(rows, cols, rng)
    if kind == "mxfp4_t":
        return mxfp4_t_random(rows, cols, rng)
    if kind == "int4":
        return int_random(rows, cols, rng)
    if kind == "int4_g16":
        return int_random(rows, cols, rng, group=16)
    if kind == "int4_sym":
        return int_random(rows, cols, rng, zero=False)
    if kind == "int4_actorder":
        return int_random(rows, cols, rng, group=16, actorder=True)
    if kind == "int8":
        return int_random(rows, cols, rng, bits=8, group=32)
    raise ValueError(kind)
