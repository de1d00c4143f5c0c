"""Configuration C5 at its own workload on the GPU (needs an MI355X and about
25 GB of host memory): a DeepSeek-V3-shaped dense layer and routed layer
(d 7168, MLA over 128 heads, dense FFN 18432, all 256 routed experts of FFN
2048, top-8 of 8 groups keeping 4, sigmoid router, scaling 2.5, one shared
expert, FP8 E4M3 with 128 x 128 block scales), 16 prompts x 256 tokens
(about 128 tokens per expert), with the routed experts streamed through a
device cache smaller than the layer (moe.zig:998-1228,
expert_cache.zig:352-425), against the oracle.

The oracle keeps the FP8 experts packed and decodes rows at use (the
reference's streamed mode, dequant.zig:427-456) and runs the first two
prompts: prompts are independent (per-prompt KV rows, per-token routing),
so their rows of the 16-prompt GPU batch are held to the parity bars
(logits within 1e-3 of max |logit|, KL <= 1e-4, residuals within 1e-3).
"""
import time

import numpy as np
import pytest

import model_gen as mg
from ditch_amd.hip import Model
from oracle.ref import RefModel
from test_gpu_forward import check_parity

pytestmark = pytest.mark.gpu

EXPERTS, PROMPTS, TOKENS = 256, 16, 256
EXPERT_BYTES = 3 * (2048 * 7168 + 16 * 56 * 4)  # gate, up, down codes + f32 block scales


def _log(msg):
    print(f"[c5] {msg}", flush=True)


def test_c5_routed_layer_at_workload_streamed(dev, ref):
    t0 = time.time()
    spec = mg.mla_c5(experts=EXPERTS, seed=21)
    tokens, rows, last = mg.batch(PROMPTS, [TOKENS], spec.config["vocab"], seed=22)
    assert len(tokens) == PROMPTS * TOKENS
    _log(f"spec of {EXPERTS} experts in {time.time() - t0:.1f}s")
    # three quarters of the layer's experts fit: the layer runs in chunks
    budget = 3 * EXPERTS // 4 * EXPERT_BYTES
    gm = Model(dev, spec, expert_cache_bytes=budget)
    try:
        _log(f"registered (streamed, budget {budget / 1e9:.2f} GB) at {time.time() - t0:.1f}s")
        outs = []
        for it in range(2):
            outs.append(gm.forward(tokens, rows, capture_rows=last, logit_rows=last))
            _log(f"forward {it} at {time.time() - t0:.1f}s")
        st = gm.expert_cache_stats()
    finally:
        gm.free()
    assert 0 < st["slots"] < EXPERTS, st
    assert st["evictions"] > 0 and st["misses"] >= EXPERTS // 2, st
    # the second forward re-streams what the first evicted and gives the same rows
    np.testing.assert_array_equal(outs[0][1], outs[1][1])
    np.testing.assert_array_equal(outs[0][0], outs[1][0])

    sub = 2 * TOKENS  # the first two prompts
    cm = RefModel(spec, threads=16, keep_packed=True)
    try:
        rc, lc = cm.forward(tokens[:sub], rows[:sub], capture_rows=last[:2], logit_rows=last[:2])
    finally:
        cm.free()
    _log(f"oracle (2 prompts) at {time.time() - t0:.1f}s")
    rg, lg = outs[0]
    err, kl = check_parity(ref, rg[:, :2, :], lg[:2], rc, lc, "c5 workload")
    _log(f"logits max err {err:.2e} of max |logit|, KL {kl:.2e}; cache {st}")
    assert np.isfinite(lg).all()
