"""The CPU oracle against the reference's committed goldens.

Each fixture under tests/golden/fixtures is a tiny checkpoint with the
reference's NumPy forward outputs (reference.json): last-position logits,
every layer entry's last-token residual and the greedy argmax. The reference
checks its Zig forward against them within 2e-3 absolute
(model_test.zig:58-75); the oracle is held to the same bar.
"""
import numpy as np
import pytest

import fixture_io as fx
from oracle.ref import RefModel

HF = ["qwen2", "llama", "qwen2_fp8", "qwen2_int4", "qwen2_int4_actorder", "qwen3_moe", "qwen3_moe_fused",
      "qwen3_moe_fused_t", "qwen3_moe_big", "deepseek_v3"]
GGUF = ["qwen2_gguf", "llama_gguf"]
TOL = 2e-3  # model_test.zig:62


def spec_of(name):
    return fx.spec_from_gguf(name) if name in GGUF else fx.spec_from_hf(name)


@pytest.mark.parametrize("name", HF + GGUF)
def test_oracle_matches_reference_goldens(name):
    spec = spec_of(name)
    model = RefModel(spec)
    g = fx.golden(name)
    for case in g["cases"]:
        ids = case["ids"]
        n = len(ids)
        res, logits = model.forward(ids, fx.case_rows(ids), capture_rows=[n - 1], logit_rows=[n - 1])
        want = np.asarray(case["last_logits"], dtype=np.float32)
        np.testing.assert_allclose(logits[0], want, atol=TOL, rtol=0)
        assert int(np.argmax(logits[0])) == case["argmax"]
        hidden = np.asarray(case["last_hidden"], dtype=np.float32)
        assert hidden.shape[0] == spec.config["layers"] + 1
        np.testing.assert_allclose(res[:, 0, :], hidden, atol=TOL, rtol=0)


def test_plant_a_mistake_in_the_oracle_fails():
    """A wrong sign in one weight row (planted on the CPU, in the oracle's
    input) moves the logits past the golden tolerance: the golden check has
    teeth."""
    spec = spec_of("qwen2")
    w = spec.get("O", 1)
    bits = w.arrays[0].copy()
    bits[:4] ^= 0x8000  # flip the sign of four rows of o_proj in layer 1
    from ditch_amd.weights import HostWeight
    spec.set("O", HostWeight.bf16(bits), 1)
    model = RefModel(spec)
    case = fx.golden("qwen2")["cases"][0]
    ids = case["ids"]
    _, logits = model.forward(ids, fx.case_rows(ids), logit_rows=[len(ids) - 1])
    assert np.abs(logits[0] - np.asarray(case["last_logits"])).max() > TOL


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4", "int4"])
def test_packed_mode_matches_decoded_mode(fmt):
    """The oracle's streamed mode (packed weights decoded row by row at use,
    dequant.zig:427-456) gives the same forward, bit for bit, as its mapped
    mode (each weight decoded to bf16 once)."""
    import model_gen as mg
    spec = mg.moe(fmt, hidden=128, layers=2, heads=2, kv_heads=1, head_dim=64, vocab=300, experts=8, top_k=2,
                  moe_inter=128, seed=5)
    tokens, rows, last = mg.batch(2, [9, 5], 300, seed=6)
    outs = []
    for packed in (False, True):
        m = RefModel(spec, keep_packed=packed)
        try:
            outs.append(m.forward(tokens, rows, capture_rows=last, logit_rows=last))
        finally:
            m.free()
    np.testing.assert_array_equal(outs[0][0], outs[1][0])
    np.testing.assert_array_equal(outs[0][1], outs[1][1])


def test_oracle_routes_repeated_selections():
    """Group-limited routing that keeps 2 experts for top-4 makes every
    token select expert 0 more than once (moe.zig:971-985 returns index 0
    when nothing is above -inf): the expert then takes more pairs than
    there are tokens, and the oracle's per-expert buffers must hold them
    (buffers sized by the token count were overrun); two runs agree bit for
    bit and stay finite."""
    import model_gen as mg
    spec = mg.moe("int4", hidden=128, layers=1, heads=2, kv_heads=1, head_dim=64, vocab=300, experts=8, top_k=4,
                  moe_inter=128, sigmoid=True, n_group=4, topk_group=1, seed=9)
    tokens, rows, last = mg.batch(3, [20, 7, 33], 300, seed=10)
    m = RefModel(spec)
    try:
        r1 = m.forward(tokens, rows, capture_rows=last, logit_rows=last)
        r2 = m.forward(tokens, rows, capture_rows=last, logit_rows=last)
    finally:
        m.free()
    assert np.isfinite(r1[1]).all()
    np.testing.assert_array_equal(r1[1], r2[1])
