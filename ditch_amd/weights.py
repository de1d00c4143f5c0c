"""Host-side weight descriptors: numpy arrays -> `ditch_weight` structs.

A `HostWeight` keeps the numpy buffers alive for as long as the struct that
points at them is in use (the C ABI never takes ownership).
"""
import ctypes

import numpy as np

from . import abi

_SCALE_DTYPES = {
    np.dtype(np.float32): abi.F32,
    np.dtype(np.float16): abi.F16,
}


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class HostWeight:
    """One `ditch_weight` over numpy storage.

    kind: "f32" | "f16" | "bf16" | "gguf" | "fp8" | "mxfp4" | "mxfp4_t" | "int"
    """

    def __init__(self, dtype, rows, cols, data, scale=None, scale_dtype=abi.F32, scale_rows=0,
                 scale_cols=0, block_rows=0, block_cols=0, row_shard=0, e5m2=False, bits=0,
                 group=0, zero=None, g_idx=None):
        self.arrays = [np.ascontiguousarray(a) if a is not None else None
                       for a in (data, scale, zero, g_idx)]
        data, scale, zero, g_idx = self.arrays
        w = abi.Weight()
        w.data = _ptr(data)
        w.dtype = dtype
        w.scale_dtype = scale_dtype
        w.rows = rows
        w.cols = cols
        w.scale = _ptr(scale)
        w.scale_rows = scale_rows
        w.scale_cols = scale_cols
        w.block_rows = block_rows
        w.block_cols = block_cols
        w.row_shard = row_shard
        w.fp8_e5m2 = 1 if e5m2 else 0
        w.bits = bits
        w.group = group
        w.zero = _ptr(zero)
        w.g_idx = _ptr(g_idx)
        self.struct = w
        self.dtype = dtype
        self.rows = rows
        self.cols = cols

    def ref(self):
        return ctypes.byref(self.struct)

    # constructors -----------------------------------------------------------

    @staticmethod
    def f32(a):
        a = np.ascontiguousarray(a, dtype=np.float32)
        return HostWeight(abi.F32, a.shape[0], a.shape[1], a)

    @staticmethod
    def bf16(bits):
        """bits: uint16 array [rows][cols] of bf16 patterns."""
        bits = np.ascontiguousarray(bits, dtype=np.uint16)
        return HostWeight(abi.BF16, bits.shape[0], bits.shape[1], bits)

    @staticmethod
    def f16(a):
        a = np.ascontiguousarray(a, dtype=np.float16)
        return HostWeight(abi.F16, a.shape[0], a.shape[1], a.view(np.uint16))

    @staticmethod
    def gguf(dtype, raw, rows, cols):
        """raw: uint8 bytes of `rows` rows of GGUF blocks."""
        return HostWeight(dtype, rows, cols, np.ascontiguousarray(raw, dtype=np.uint8))

    @staticmethod
    def fp8(codes, scale, block_rows, block_cols, e5m2=False, row_shard=0):
        """codes: uint8 [rows][cols]; scale: [scale_rows][scale_cols] f32/f16
        array, or ('bf16', uint16 array) / ('e8m0', uint8 array)."""
        sdt, sarr = _scale_kind(scale)
        codes = np.ascontiguousarray(codes, dtype=np.uint8)
        return HostWeight(abi.FP8, codes.shape[0], codes.shape[1], codes, scale=sarr,
                          scale_dtype=sdt, scale_rows=sarr.shape[0], scale_cols=sarr.shape[1],
                          block_rows=block_rows, block_cols=block_cols, row_shard=row_shard,
                          e5m2=e5m2)

    @staticmethod
    def mxfp4(packed, scales):
        """packed: uint8 [rows][cols/2] (low nibble first); scales: uint8 [rows][cols/32]."""
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        rows, half = packed.shape
        return HostWeight(abi.MXFP4, rows, half * 2, packed, scale=np.ascontiguousarray(scales, dtype=np.uint8),
                          scale_dtype=abi.E8M0)

    @staticmethod
    def mxfp4_t(blocks, scales):
        """gpt-oss layout: blocks uint8 [src_rows][src_cols/32][16], scales
        uint8 [src_rows][src_cols/32]; the view is [src_cols][src_rows]."""
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        src_rows, nblk = blocks.shape[0], blocks.shape[1]
        return HostWeight(abi.MXFP4_T, nblk * 32, src_rows, blocks,
                          scale=np.ascontiguousarray(scales, dtype=np.uint8), scale_dtype=abi.E8M0)

    @staticmethod
    def int_packed(words, scale, rows, cols, bits, group, zero=None, g_idx=None):
        """compressed-tensors pack-quantized: words int32 [rows][ceil(cols*bits/32)];
        scale [rows][groups] (f32/f16 array or ('bf16', uint16)); zero int32
        [ceil(rows*bits/32)][groups] or None; g_idx int32 [cols] or None."""
        sdt, sarr = _scale_kind(scale)
        return HostWeight(abi.INT_PACKED, rows, cols, np.ascontiguousarray(words).view(np.int32), scale=sarr,
                          scale_dtype=sdt, scale_rows=rows, scale_cols=sarr.shape[1], bits=bits, group=group,
                          zero=None if zero is None else np.ascontiguousarray(zero).view(np.int32),
                          g_idx=None if g_idx is None else np.ascontiguousarray(g_idx, dtype=np.int32))


def _scale_kind(scale):
    if isinstance(scale, tuple):
        kind, arr = scale
        if kind == "bf16":
            return abi.BF16, np.ascontiguousarray(arr, dtype=np.uint16)
        if kind == "e8m0":
            return abi.E8M0, np.ascontiguousarray(arr, dtype=np.uint8)
        raise ValueError(kind)
    arr = np.ascontiguousarray(scale)
    if arr.dtype == np.float16:
        return abi.F16, arr.view(np.uint16)
    return abi.F32, np.ascontiguousarray(arr, dtype=np.float32)


def vector(a):
    """A norm or bias vector as a 1-row f32 weight."""
    a = np.ascontiguousarray(a, dtype=np.float32).reshape(1, -1)
    return HostWeight(abi.F32, 1, a.shape[1], a)
