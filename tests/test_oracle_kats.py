"""Known answers and closed forms that pin the oracle's decoders and kernels.

Every check here comes from the reference's own unit tests (cited) or from
mathematics / an independent library (numpy, torch's float8 and bfloat16
casts), never from retyping the oracle's formula.
"""
import ctypes

import numpy as np
import pytest
import torch

from ditch_amd import abi
from ditch_amd.weights import HostWeight


def f32bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# -- fp8 tables: dequant.zig:1290-1299 and torch's float8 casts --------------

def test_fp8_known_values(ref):
    v = ref.lib.ref_fp8_value
    assert v(0x7E, 0) == 448.0 and v(0xFE, 0) == -448.0
    assert np.isnan(v(0x7F, 0))
    assert v(0x38, 0) == 1.0
    assert v(0x01, 0) == 0.001953125
    assert v(0x7B, 1) == 57344.0
    assert np.isinf(v(0x7C, 1))
    assert v(0x3C, 1) == 1.0


@pytest.mark.parametrize("e5m2", [False, True])
def test_fp8_table_equals_torch_float8(ref, e5m2):
    codes = torch.arange(256, dtype=torch.uint8)
    tdt = torch.float8_e5m2 if e5m2 else torch.float8_e4m3fn
    want = codes.view(tdt).to(torch.float32).numpy()
    got = np.array([ref.lib.ref_fp8_value(c, int(e5m2)) for c in range(256)], dtype=np.float32)
    nan = np.isnan(want)
    assert (np.isnan(got) == nan).all()
    np.testing.assert_array_equal(got[~nan], want[~nan])
    # the sign of the NaN codes follows the code's sign bit (dequant.zig:302)
    assert (np.signbit(got[nan]) == (np.arange(256)[nan] >= 128)).all()


# -- e8m0 x e2m1: exhaustive exactness, dequant.zig:263-268 -------------------

def test_e8m0_times_e2m1_is_exact(ref):
    e2m1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6])
    for b in range(255):
        sc = ref.lib.ref_e8m0_scale(b)
        exact = np.float32(e2m1 * 2.0 ** (b - 127))
        assert np.array_equal(f32bits(np.float32(e2m1 * np.float64(sc))), f32bits(exact)), b


def test_mxfp4_decode_exhaustive_codes_and_scales(ref):
    """All 16 codes x 256 scale bytes through the packed decoder, against
    the closed form 2^(b-127) * e2m1 rounded by torch to bfloat16."""
    rows = 256
    packed = np.tile(np.array([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE] * 2, dtype=np.uint8), (rows, 1))
    scales = np.arange(256, dtype=np.uint8).reshape(rows, 1)
    w = HostWeight.mxfp4(packed, scales)
    got = ref.dequant(w)
    e2m1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], dtype=np.float64)
    codes = np.tile(np.arange(16), 2)
    for b in range(255):
        val = torch.tensor(e2m1[codes] * 2.0 ** (b - 127), dtype=torch.float64).to(torch.bfloat16)
        assert np.array_equal(got[b], val.view(torch.int16).numpy().view(np.uint16)), b
    # byte 255 is an infinite scale: 0 * inf is NaN, the rest +-inf
    assert np.isnan((got[255].astype(np.uint32) << 16).view(np.float32)[codes % 8 == 0]).all()
    assert np.isinf((got[255].astype(np.uint32) << 16).view(np.float32)[codes % 8 != 0]).all()


# -- bf16 / f16 conversions ----------------------------------------------------

def test_bf16_rne_equals_torch(ref):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10 ** rng.uniform(-40, 38, 20000).astype(np.float32),
                        np.array([0, -0., 1e-45, -1e-45, 3.4e38, np.inf, -np.inf, 1.0039062, 1.0117188], dtype=np.float32),
                        # exact ties (round to even) and the carry into the exponent
                        (np.array([0x3F808000, 0x3F818000, 0x3F7FFFFF, 0x7F7FFFFF], dtype=np.uint32)).view(np.float32)])
    x = x[np.isfinite(x) | np.isinf(x)]
    got = ref.f32_to_bf16(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, want)
    # NaN: (bits >> 16) | 0x40 (tensor.zig:425)
    nan = np.array([0x7F800001, 0xFFC01234], dtype=np.uint32).view(np.float32)
    np.testing.assert_array_equal(ref.f32_to_bf16(nan), np.array([0x7FC0, 0xFFC0], dtype=np.uint16))


def test_f16_widening_exhaustive(ref):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([ref.lib.ref_f16_to_f32(int(v)) for v in h], dtype=np.float32)
    nan = np.isnan(want)
    assert (np.isnan(got) == nan).all()
    np.testing.assert_array_equal(f32bits(got[~nan]), f32bits(want[~nan]))


def test_f16_narrowing_equals_numpy(ref):
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(5000) * 10 ** rng.uniform(-9, 5, 5000)).astype(np.float32)
    got = np.array([ref.lib.ref_f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    np.testing.assert_array_equal(got, x.astype(np.float16).view(np.uint16))


# -- pack-quantized fields: dequant.zig:1301-1310 -------------------------------

def test_unpack_field_known_answers(ref):
    f = ref.lib.ref_unpack_field if hasattr(ref.lib, "ref_unpack_field") else None
    lib = ref.lib
    lib.ref_unpack_field.restype = ctypes.c_uint32
    lib.ref_unpack_field.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    words = np.array([0x76543210, 0xFEDCBA98], dtype=np.uint32)
    for i in range(16):
        assert lib.ref_unpack_field(words.ctypes.data, i, 4) == i
    words = np.array([1 << 30, 1], dtype=np.uint32)
    assert lib.ref_unpack_field(words.ctypes.data, 10, 3) == 0b101


def test_int4_decode_closed_form(ref):
    """(q - zp) * s rounded to bf16 for every 4-bit field and zero point."""
    rows, cols, group = 16, 16, 16
    fields = np.tile(np.arange(16, dtype=np.uint32), (rows, 1))
    words = np.zeros((rows, 2), dtype=np.uint32)
    for c in range(cols):
        words[:, c // 8] |= fields[:, c] << (4 * (c % 8))
    zfield = np.arange(rows, dtype=np.uint32) % 16
    zw = np.zeros((2, 1), dtype=np.uint32)
    for r in range(rows):
        zw[(r * 4) // 32, 0] |= zfield[r] << ((r * 4) % 32)
    scale = np.linspace(0.01, 0.3, rows, dtype=np.float32).reshape(rows, 1).astype(np.float16)
    w = HostWeight.int_packed(words, scale, rows, cols, 4, group, zero=zw)
    got = ref.dequant(w)
    q = fields.astype(np.int64) - 8
    zp = zfield.astype(np.int64)[:, None] - 8
    val = np.float32((q - zp).astype(np.float32) * scale.astype(np.float32))
    want = torch.from_numpy(val).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, want)


# -- GGUF blocks: quant.zig:367-482 ----------------------------------------------

def test_q8_0_round_trip(ref):
    rng = np.random.default_rng(7)
    x = ((rng.random(64, dtype=np.float32) * 2 - 1) * 2).astype(np.float32)
    x[0], x[5], x[17] = 0, 2.5, -2.5
    blocks = ref.quantize_q8_0(x)
    y = ref.gguf_dequant(abi.Q8_0, blocks, 64)
    for blk in range(2):
        xb = x[blk * 32:(blk + 1) * 32]
        amax = np.abs(xb).max()
        d = np.float32(np.float16(amax / 127))
        assert (np.abs(xb - y[blk * 32:(blk + 1) * 32]) <= d * 0.5 + amax * 1e-3).all()
    assert abs(y[5] - 2.5) <= 2.5e-3
    assert blocks[2 + 5] == 127


def _wf16(b, off, v):
    b[off:off + 2] = np.frombuffer(np.float16(v).tobytes(), dtype=np.uint8)


def test_q4_k_hand_built_block(ref):
    b = np.zeros(144, dtype=np.uint8)
    _wf16(b, 0, 0.5)
    _wf16(b, 2, 0.25)
    b[4 + 0], b[4 + 4], b[4 + 1], b[4 + 5] = 4, 2, 8, 1
    b[4 + 8] = 0x35
    b[4 + 0] |= 0x40
    b[16 + 0] = 0x3 | (0x9 << 4)
    b[16 + 64] = 0x7
    y = ref.gguf_dequant(abi.Q4_K, b, 256)
    assert abs(y[0] - (0.5 * 4 * 3 - 0.25 * 2)) < 1e-6
    assert abs(y[32] - (0.5 * 8 * 9 - 0.25 * 1)) < 1e-6
    assert abs(y[1] - (-0.25 * 2)) < 1e-6
    assert abs(y[128] - (0.5 * 21 * 7 - 0.25 * 3)) < 1e-6


def test_q6_k_hand_built_block(ref):
    b = np.zeros(210, dtype=np.uint8)
    _wf16(b, 208, 0.125)
    b[192 + 0] = 3
    b[192 + 2] = np.uint8(np.int8(-2).view(np.uint8))
    b[0] = 0xA
    b[128] = 0x2
    b[32] = 0x1
    b[128] |= 0x1 << 2
    y = ref.gguf_dequant(abi.Q6_K, b, 256)
    assert abs(y[0] - 0.125 * 3 * 10) < 1e-6
    assert abs(y[32] - 0.125 * -2 * -15) < 1e-6
    assert abs(y[1] - 0.125 * 3 * -32) < 1e-6


def test_q8_k_block(ref):
    b = np.zeros(292, dtype=np.uint8)
    b[0:4] = np.frombuffer(np.float32(0.75).tobytes(), dtype=np.uint8)
    b[4 + 3] = np.uint8(np.int8(-100).view(np.uint8))
    b[4 + 255] = 64
    y = ref.gguf_dequant(abi.Q8_K, b, 256)
    assert abs(y[3] + 75) < 1e-6 and abs(y[255] - 48) < 1e-6 and y[0] == 0


@pytest.mark.parametrize("dt", [abi.Q4_0, abi.Q4_1, abi.Q5_0, abi.Q5_1])
def test_small_block_formats_closed_form(ref, dt):
    """Q4_0/Q4_1/Q5_0/Q5_1 element formulas written from the ggml block
    definitions with numpy (independent unpacking code)."""
    rng = np.random.default_rng(dt)
    nb = 8
    bb = {abi.Q4_0: 18, abi.Q4_1: 20, abi.Q5_0: 22, abi.Q5_1: 24}[dt]
    raw = rng.integers(0, 256, nb * bb, dtype=np.uint8)
    for i in range(nb):  # finite scales
        _wf16(raw, i * bb, rng.uniform(-1, 1))
        if dt in (abi.Q4_1, abi.Q5_1):
            _wf16(raw, i * bb + 2, rng.uniform(-1, 1))
    y = ref.gguf_dequant(dt, raw, nb * 32)
    for i in range(nb):
        blk = raw[i * bb:(i + 1) * bb]
        d = np.float32(blk[0:2].view(np.float16)[0])
        if dt == abi.Q4_0:
            qs = blk[2:18]
            q = np.concatenate([(qs & 15).astype(np.int32) - 8, (qs >> 4).astype(np.int32) - 8])
            want = q.astype(np.float32) * d
        elif dt == abi.Q4_1:
            m = np.float32(blk[2:4].view(np.float16)[0])
            qs = blk[4:20]
            q = np.concatenate([qs & 15, qs >> 4]).astype(np.float32)
            want = (q * d).astype(np.float32) + m
        else:
            off = 2 if dt == abi.Q5_0 else 4
            m = np.float32(blk[2:4].view(np.float16)[0]) if dt == abi.Q5_1 else None
            qh = int(blk[off:off + 4].view(np.uint32)[0])
            qs = blk[off + 4:off + 20]
            hb = np.array([(qh >> j) & 1 for j in range(32)])
            q = np.concatenate([qs & 15, qs >> 4]).astype(np.int32) | (hb << 4)
            want = ((q - 16).astype(np.float32) * d) if dt == abi.Q5_0 else (q.astype(np.float32) * d + m)
        np.testing.assert_array_equal(y[i * 32:(i + 1) * 32], want.astype(np.float32))


# -- kernels ---------------------------------------------------------------------

def test_matmul_with_delta_known_answer(ref):
    """tensor.zig:1400-1421."""
    w = HostWeight.f32(np.array([[1, 2], [3, 4], [5, 6]], dtype=np.float32))
    out = ref.matmulT(np.array([[1, 1]], dtype=np.float32), w,
                      delta=(np.array([[1, 0]], np.float32), np.array([[1], [1], [1]], np.float32)))
    np.testing.assert_array_equal(out[0], [4, 8, 12])
    np.testing.assert_array_equal(ref.matvecTMulti(w, np.array([[1, 1, 1]], np.float32))[0], [9, 12])


def test_matmul_against_float64(ref):
    rng = np.random.default_rng(3)
    for n, rows, cols in [(1, 7, 33), (5, 40, 100), (17, 65, 257)]:
        x = rng.standard_normal((n, cols)).astype(np.float32)
        wf = rng.standard_normal((rows, cols)).astype(np.float32)
        got = ref.matmulT(x, HostWeight.f32(wf))
        want = x.astype(np.float64) @ wf.astype(np.float64).T
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-4)


def test_cephes_exp_within_two_ulp(ref):
    x = np.linspace(-87, 88, 20001, dtype=np.float32)
    got = np.array([ref.lib.ref_exp_cephes(float(v)) for v in x], dtype=np.float32)
    want = np.exp(x.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32))
    assert (np.abs(got - want) <= 2 * np.abs(ulp)).all()


def test_log_softmax_and_kl_closed_form(ref):
    from scipy.special import log_softmax
    rng = np.random.default_rng(4)
    base = rng.standard_normal((3, 1000)).astype(np.float32) * 3
    lb = ref.log_softmax_rows(base)
    np.testing.assert_allclose(lb, log_softmax(base.astype(np.float64), axis=1), atol=2e-6)
    assert np.abs(ref.kl_rows(lb, base)).max() < 1e-6  # KL of identical logits (scorers.zig:911)
    trial = base + rng.standard_normal(base.shape).astype(np.float32) * 0.1
    lt = log_softmax(trial.astype(np.float64), axis=1)
    p = np.exp(lb.astype(np.float64))
    want = (p * (lb.astype(np.float64) - lt)).sum(axis=1)
    np.testing.assert_allclose(ref.kl_rows(lb, trial), want, rtol=1e-4)
    assert (ref.kl_rows(lb, trial) > 0).all()


def test_rope_preserves_pair_norms_and_is_identity_at_zero(ref):
    rng = np.random.default_rng(5)
    half = 8
    ang = rng.uniform(0, 6, (4, half))
    cos_t, sin_t = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    cos_t[0], sin_t[0] = 1, 0
    x = rng.standard_normal((4, 16)).astype(np.float32)
    for style in (abi.ROPE_NEOX, abi.ROPE_GPTJ):
        y = ref.rope_rows(x, cos_t, sin_t, [0, 1, 2, 3], style)
        np.testing.assert_array_equal(y[0], x[0])
        if style == abi.ROPE_NEOX:
            pn = lambda a: a[:, :half] ** 2 + a[:, half:] ** 2
        else:
            pn = lambda a: a[:, 0::2] ** 2 + a[:, 1::2] ** 2
        np.testing.assert_allclose(pn(y), pn(x), rtol=1e-5)


def test_edit_removes_the_directions(ref):
    """abliterate.zig:580-591: after the none-mode edit with weight 1, V^T W' ~ 0."""
    rng = np.random.default_rng(6)
    rows, cols, k = 48, 40, 2
    wf = rng.standard_normal((rows, cols)).astype(np.float32)
    v, _ = np.linalg.qr(rng.standard_normal((rows, k)))
    v = v.T.astype(np.float32)
    a, b = ref.edit_delta(HostWeight.f32(wf), v, 1.0)
    wp = wf.astype(np.float64) + b.astype(np.float64) @ a.astype(np.float64)
    assert np.abs(v.astype(np.float64) @ wp).max() < 1e-4


# -- closed forms for the per-op kernels (float64 / torch restatements) ----------

def test_matvecT_and_row_norms_against_float64(ref):
    rng = np.random.default_rng(7)
    for q, rows, cols in [(1, 9, 31), (3, 70, 129), (8, 300, 64)]:
        wf = rng.standard_normal((rows, cols)).astype(np.float32)
        y = rng.standard_normal((q, rows)).astype(np.float32)
        y[0, ::3] = 0  # zero entries are skipped by the reference (tensor.zig:1056-1094)
        w = HostWeight.f32(wf)
        want = y.astype(np.float64) @ wf.astype(np.float64)
        np.testing.assert_allclose(ref.matvecTMulti(w, y), want, rtol=1e-5, atol=1e-4)
        np.testing.assert_allclose(ref.rowNorms(w), np.linalg.norm(wf.astype(np.float64), axis=1), rtol=1e-6)


def test_attention_scores_and_values_against_float64(ref):
    rng = np.random.default_rng(8)
    hd, n_keys, stride = 64, 37, 96
    q = rng.standard_normal(hd).astype(np.float32)
    kv = rng.standard_normal(n_keys * stride).astype(np.float32)
    scores = np.empty(n_keys, np.float32)
    ref.lib.ref_attention_scores(scores.ctypes.data, n_keys, q.ctypes.data, hd, kv.ctypes.data, stride, 0.125)
    kmat = kv.reshape(n_keys, stride)[:, :hd].astype(np.float64)
    np.testing.assert_allclose(scores, 0.125 * (kmat @ q.astype(np.float64)), rtol=1e-5, atol=1e-5)
    p = rng.random(n_keys).astype(np.float32)
    vd = 48
    out = np.empty(vd, np.float32)
    ref.lib.ref_attention_values(out.ctypes.data, vd, p.ctypes.data, n_keys, kv.ctypes.data, stride)
    want = p.astype(np.float64) @ kv.reshape(n_keys, stride)[:, :vd].astype(np.float64)
    np.testing.assert_allclose(out, want, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("one_plus", [0, 1])
def test_layernorm_and_gemma_rmsnorm_against_float64(ref, one_plus):
    rng = np.random.default_rng(9)
    n = 200
    x = (rng.standard_normal(n) * 3 + 1).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    out = np.empty(n, np.float32)
    ref.lib.ref_layernorm(out.ctypes.data, x.ctypes.data, w.ctypes.data, n, b.ctypes.data, n, 1e-5, one_plus)
    xd = x.astype(np.float64)
    scale = (1 + w.astype(np.float64)) if one_plus else w.astype(np.float64)
    want = (xd - xd.mean()) / np.sqrt(xd.var() + 1e-5) * scale + b
    np.testing.assert_allclose(out, want, rtol=1e-5, atol=1e-5)
    got = ref.rmsnorm_rows(x[None], w, 1e-6, gemma=bool(one_plus))[0]
    want = xd / np.sqrt((xd * xd).mean() + 1e-6) * scale
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_gated_activations_against_torch(ref):
    """Activation order of tensor.Activation (compute.zig:81-83): silu,
    gelu_tanh, gelu (erf), relu, relu2, quick_gelu (x * sigmoid(1.702 x))."""
    import torch.nn.functional as F
    g = torch.linspace(-9, 9, 601, dtype=torch.float64)
    u = torch.linspace(2, -1, 601, dtype=torch.float64)
    want = [F.silu(g), F.gelu(g, approximate="tanh"), F.gelu(g), F.relu(g), F.relu(g) ** 2,
            g * torch.sigmoid(1.702 * g)]
    for act, a in enumerate(want):
        got = ref.gated(act, g.float().numpy(), u.float().numpy(), 1, g.numel(), g.numel(), g.numel())
        np.testing.assert_allclose(got, (a * u).numpy(), rtol=2e-5, atol=2e-6, err_msg=f"act {act}")


def test_softmax_against_scipy(ref):
    from scipy.special import softmax
    rng = np.random.default_rng(10)
    x = (rng.standard_normal((4, 77)) * 5).astype(np.float32)
    np.testing.assert_allclose(ref.softmax_rows(x), softmax(x.astype(np.float64), axis=1), rtol=2e-6, atol=1e-9)
