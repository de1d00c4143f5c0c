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

HF = ["qwen2", "llama", "qwen2_fp8", "qwen2_int4", "qwen2_int4_actorder", "qwen3_moe", "deepseek_v3"]
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
