"""Synthetic weights in the benchmark configurations' formats.

Quantisers here are this build's own (the decoders are what must match the
reference; any encoder's output is decoded by the closed forms the tests
pin). They run in torch on whatever device the input lives on, so the
large configurations can be quantised on the GPU and only the packed codes
cross to host memory.
"""
import numpy as np
import torch

from .weights import HostWeight

E2M1 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def _np(t):
    return t.detach().cpu().contiguous().numpy()


def bf16_weight(w: torch.Tensor) -> HostWeight:
    return HostWeight.bf16(_np(w.to(torch.bfloat16).view(torch.int16)).view(np.uint16))


def f32_weight(w: torch.Tensor) -> HostWeight:
    return HostWeight.f32(_np(w.float()))


def q8_0_random(rows, cols, gen: torch.Generator, device="cpu") -> HostWeight:
    """Config C2: int8 codes uniform in [-127, 127], block scales |N(0,1)| * 0.01 in f16."""
    nb = cols // 32
    q = torch.randint(-127, 128, (rows, nb, 32), generator=gen, device=device, dtype=torch.int32).to(torch.int8)
    d = (torch.randn(rows, nb, 1, generator=gen, device=device).abs() * 0.01).to(torch.float16)
    blocks = torch.cat([d.view(torch.uint8).view(rows, nb, 2), q.view(torch.uint8)], dim=2)
    return HostWeight.gguf(5, _np(blocks).reshape(-1), rows, cols)


def q8_0_quantize(w: torch.Tensor) -> HostWeight:
    """ggml's Q8_0 quantiser (quant.zig:245-255 semantics: amax/127, round)."""
    rows, cols = w.shape
    x = w.float().reshape(rows, cols // 32, 32)
    amax = x.abs().amax(dim=2, keepdim=True)
    d = amax / 127.0
    idv = torch.where(d != 0, 1.0 / d, torch.zeros_like(d))
    q = torch.round(x * idv).clamp(-128, 127).to(torch.int8)
    dh = d.to(torch.float16)
    blocks = torch.cat([dh.view(torch.uint8).view(rows, cols // 32, 2), q.view(torch.uint8)], dim=2)
    return HostWeight.gguf(5, _np(blocks).reshape(-1), rows, cols)


def mxfp4_quantize(w: torch.Tensor) -> HostWeight:
    """E2M1 codes with one E8M0 exponent per 32 columns (natural layout)."""
    rows, cols = w.shape
    x = w.float().reshape(rows, cols // 32, 32)
    amax = x.abs().amax(dim=2, keepdim=True).clamp_min(1e-30)
    e = torch.ceil(torch.log2(amax / 6.0)).clamp(-127, 127)
    y = x / torch.exp2(e)
    # nearest E2M1 magnitude through the midpoints between grid values
    mids = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], device=w.device)
    idx = torch.bucketize(y.abs(), mids)
    code = idx | ((y < 0).to(torch.int64) << 3)
    code = code.reshape(rows, cols // 2, 2)
    packed = (code[..., 0] | (code[..., 1] << 4)).to(torch.uint8)
    scales = (e.reshape(rows, cols // 32) + 127).to(torch.uint8)
    return HostWeight.mxfp4(_np(packed), _np(scales))


def fp8_quantize(w: torch.Tensor, block=128) -> HostWeight:
    """E4M3 codes with an f32 scale per block x block (DeepSeek layout,
    `weight_scale_inv`)."""
    rows, cols = w.shape
    sr, sc = -(-rows // block), -(-cols // block)
    pad = torch.zeros(sr * block, sc * block, device=w.device)
    pad[:rows, :cols] = w.float()
    blocks = pad.reshape(sr, block, sc, block)
    amax = blocks.abs().amax(dim=(1, 3)).clamp_min(1e-12)
    s = amax / 448.0
    q = (blocks / s[:, None, :, None]).to(torch.float8_e4m3fn).reshape(sr * block, sc * block)[:rows, :cols]
    return HostWeight.fp8(_np(q.view(torch.uint8)), _np(s.float()), block, block)


def int4_quantize(w: torch.Tensor, group=128) -> HostWeight:
    """compressed-tensors pack-quantized, 4-bit asymmetric groups: f16 scale,
    zero points packed along rows (dequant.zig:518-597 layout)."""
    rows, cols = w.shape
    g = cols // group
    x = w.float().reshape(rows, g, group)
    lo, hi = x.amin(dim=2, keepdim=True), x.amax(dim=2, keepdim=True)
    s = ((hi - lo) / 15.0).clamp_min(1e-8).to(torch.float16)
    sf = s.float()
    zf = torch.round(-lo / sf).clamp(0, 15)
    field = (torch.round(x / sf) + zf).clamp(0, 15).to(torch.int64).reshape(rows, cols)
    shifts = (torch.arange(8, device=w.device) * 4)
    words = (field.reshape(rows, cols // 8, 8) << shifts).sum(dim=2).to(torch.int64)
    words = (words & 0xFFFFFFFF).to(torch.int64)
    words32 = _np(words).astype(np.uint32).view(np.int32)
    zfield = zf.reshape(rows, g).to(torch.int64)
    zrows = -(-rows * 4 // 32)
    zpad = torch.zeros(zrows * 8, g, dtype=torch.int64, device=w.device)
    zpad[:rows] = zfield
    zw = (zpad.reshape(zrows, 8, g) << shifts.reshape(1, 8, 1)).sum(dim=1)
    zw32 = _np(zw & 0xFFFFFFFF).astype(np.uint32).view(np.int32)
    return HostWeight.int_packed(words32, _np(s.reshape(rows, g)), rows, cols, 4, group, zero=zw32)


def int4_random(rows, cols, rng: np.random.Generator, group=128, std=0.02) -> HostWeight:
    """Random compressed-tensors pack-quantized 4-bit weights drawn in the
    packed domain (no source matrix: fast at the MoE configurations' sizes):
    fields uniform in 0..15, zero points in 6..9 packed along rows, f16 group
    scales around std / 4.6 (the spread of a uniform field about its zero)."""
    g = -(-cols // group)
    words = rng.integers(0, 1 << 32, size=(rows, -(-cols * 4 // 32)), dtype=np.uint64).astype(np.uint32)
    s = (std / 4.6 * rng.uniform(0.5, 1.5, size=(rows, g))).astype(np.float16)
    zf = rng.integers(6, 10, size=(rows, g), dtype=np.int64)
    zrows = -(-rows * 4 // 32)
    zpad = np.zeros((zrows * 8, g), dtype=np.int64)
    zpad[:rows] = zf
    zw = (zpad.reshape(zrows, 8, g) << (np.arange(8, dtype=np.int64) * 4).reshape(1, 8, 1)).sum(axis=1)
    zw32 = (zw & 0xFFFFFFFF).astype(np.uint32).view(np.int32)
    return HostWeight.int_packed(words.view(np.int32), s, rows, cols, 4, group, zero=zw32)


def fp8_random(rows, cols, rng: np.random.Generator, block=128, std=0.02) -> HostWeight:
    """Random E4M3 codes drawn in the code domain (uniform bytes, the two NaN
    codes replaced by the largest finite ones) with an f32 scale per block x
    block around std / 100 (the codes' RMS is about 100): fast at the MoE
    configurations' sizes."""
    codes = np.frombuffer(rng.bytes(rows * cols), dtype=np.uint8).reshape(rows, cols).copy()
    codes -= ((codes & 0x7f) == 0x7f).view(np.uint8)
    sr, sc = -(-rows // block), -(-cols // block)
    s = (std / 100.0 * rng.uniform(0.5, 1.5, size=(sr, sc))).astype(np.float32)
    return HostWeight.fp8(codes, s, block, block)


QUANTIZERS = {
    "f32": f32_weight,
    "bf16": bf16_weight,
    "q8_0": q8_0_quantize,
    "mxfp4": mxfp4_quantize,
    "fp8": fp8_quantize,
    "int4": int4_quantize,
}
