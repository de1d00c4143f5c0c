"""The resident forward pass on the GPU against the oracle and the
reference's goldens (needs an MI355X).

Bars: logits within 1e-3 relative to the CPU
logits (max |dlogit| <= 1e-3 * max |logit|), per-prompt KL(CPU || GPU) <=
1e-4 with scorers.zig:387-394's formula, residuals within 1e-3 relative;
against the fixture goldens, the reference's own 2e-3 absolute
(model_test.zig:58-75).
"""
import numpy as np
import pytest

import fixture_io as fx
import model_gen as mg
from ditch_amd import abi
from ditch_amd.hip import Model
from oracle.ref import RefModel

pytestmark = pytest.mark.gpu

HF = ["qwen2", "llama", "qwen2_fp8", "qwen2_int4", "qwen2_int4_actorder", "qwen3_moe", "qwen3_moe_fused",
      "qwen3_moe_fused_t", "qwen3_moe_big", "deepseek_v3"]
GGUF = ["qwen2_gguf", "llama_gguf"]


def check_parity(ref, res_g, log_g, res_c, log_c, tag=""):
    scale = np.abs(log_c).max()
    err = np.abs(log_g - log_c).max()
    assert err <= 1e-3 * scale, f"{tag} logits: max err {err:.3e} vs scale {scale:.3e}"
    if res_c.size:
        rs = np.abs(res_c).max(axis=-1, keepdims=True)
        assert (np.abs(res_g - res_c) <= 1e-3 * rs + 1e-6).all(), f"{tag} residuals"
    lb = ref.log_softmax_rows(log_c)
    kl = ref.kl_rows(lb, log_g)
    assert kl.max() <= 1e-4, f"{tag} KL {kl.max():.3e}"
    return err / scale, kl.max()


@pytest.mark.parametrize("name", HF + GGUF)
def test_fixture_forward_matches_goldens_and_oracle(dev, ref, name):
    spec = fx.spec_from_gguf(name) if name in GGUF else fx.spec_from_hf(name)
    gm = Model(dev, spec)
    cm = RefModel(spec)
    try:
        for case in fx.golden(name)["cases"]:
            ids = case["ids"]
            n = len(ids)
            res, logits = gm.forward(ids, fx.case_rows(ids), capture_rows=[n - 1], logit_rows=[n - 1])
            np.testing.assert_allclose(logits[0], case["last_logits"], atol=2e-3, rtol=0)
            np.testing.assert_allclose(res[:, 0, :], case["last_hidden"], atol=2e-3, rtol=0)
            assert int(np.argmax(logits[0])) == case["argmax"]
            rc, lc = cm.forward(ids, fx.case_rows(ids), capture_rows=[n - 1], logit_rows=[n - 1])
            check_parity(ref, res, logits, rc, lc, name)
    finally:
        gm.free()
        cm.free()


def test_fixture_batch_of_prompts(dev, ref):
    """All cases of a fixture as one batch (rows {b, pos}): each prompt's
    logits equal its single-prompt run."""
    spec = fx.spec_from_hf("qwen3_moe")
    cases = fx.golden("qwen3_moe")["cases"]
    tokens, rows, last = [], [], []
    for b, c in enumerate(cases):
        for p, t in enumerate(c["ids"]):
            tokens.append(t)
            rows.append((b, p))
        last.append(len(tokens) - 1)
    gm = Model(dev, spec)
    try:
        res, logits = gm.forward(tokens, rows, capture_rows=last, logit_rows=last)
    finally:
        gm.free()
    for i, c in enumerate(cases):
        np.testing.assert_allclose(logits[i], c["last_logits"], atol=2e-3, rtol=0)
        np.testing.assert_allclose(res[:, i, :], c["last_hidden"], atol=2e-3, rtol=0)


SYNTH = {
    "dense_bf16": lambda: mg.dense("bf16", qkv_bias=True),
    "dense_f32": lambda: mg.dense("f32", embed_fmt="f32"),
    "dense_mxfp4": lambda: mg.dense("mxfp4", tie=False),
    "dense_fp8": lambda: mg.dense("fp8", qk_norm=True),
    "dense_int4": lambda: mg.dense("int4"),
    "dense_q8_0": lambda: mg.dense("q8_0"),
    "moe_int4_softmax": lambda: mg.moe("int4"),
    "moe_fp8_sigmoid_groups": lambda: mg.moe("fp8", sigmoid=True, n_group=4, topk_group=2, shared=128, scaling=2.5,
                                             dense_first=1),
    "mla_fp8": lambda: mg.mla("fp8"),
    # group-limited routing that keeps 2 experts for top-4: every token's
    # last selections repeat expert 0 (moe.zig:971-985 returns index 0 when
    # nothing is above -inf), so the combine must order repeats stably
    # hidden 512 and q_lora 512: the norms take the wave-per-row kernel (the
    # final norm through the logit rows' index, MLA's q_a norm in place)
    "dense_bf16_h512": lambda: mg.dense("bf16", hidden=512, inter=1024, heads=8, kv_heads=2, head_dim=64),
    "mla_fp8_qlora512": lambda: mg.mla("fp8", q_lora=512),
    # head widths that are not multiples of 4 (kv_a 82 rows): the keys and
    # values assembled per head and rotated by the general RoPE kernel, not
    # the float4 cache kernel; head_dim 48 on the per-row attention
    "mla_fp8_odd_widths": lambda: mg.mla("fp8", nope=30, rope=18, v_dim=30),
    "moe_int4_repeated_selections": lambda: mg.moe("int4", experts=8, top_k=4, sigmoid=True, n_group=4,
                                                   topk_group=1),
}


@pytest.mark.parametrize("name", list(SYNTH))
def test_synthetic_forward_matches_oracle(dev, ref, name):
    spec = SYNTH[name]()
    tokens, rows, last = mg.batch(6, [17, 64, 1, 40], spec.config["vocab"], seed=len(name))
    gm = Model(dev, spec)
    cm = RefModel(spec)
    try:
        rg, lg = gm.forward(tokens, rows, capture_rows=last, logit_rows=last)
        rc, lc = cm.forward(tokens, rows, capture_rows=last, logit_rows=last)
    finally:
        gm.free()
        cm.free()
    check_parity(ref, rg, lg, rc, lc, name)


LARGE = ["dense_mxfp4", "dense_fp8", "dense_int4", "dense_bf16"]


@pytest.mark.parametrize("name", LARGE)
def test_synthetic_forward_large_batch_matches_oracle(dev, ref, name):
    """294 rows: every product on the large-batch kernels, with the fused
    producers (RMSNorm and the gate/up epilogue writing the next product's
    fragments; fp6 terms and the scaled MFMA for MXFP4)."""
    spec = SYNTH[name]()
    tokens, rows, last = mg.batch(3, [130, 64, 100], spec.config["vocab"], seed=len(name) + 7)
    gm = Model(dev, spec)
    cm = RefModel(spec)
    try:
        rg, lg = gm.forward(tokens, rows, capture_rows=last, logit_rows=last)
        rc, lc = cm.forward(tokens, rows, capture_rows=last, logit_rows=last)
    finally:
        gm.free()
        cm.free()
    check_parity(ref, rg, lg, rc, lc, name)


def test_edit_then_forward(dev, ref):
    """Rank-2 none-mode edit (abliterate.zig:264-280) of o_proj, down_proj and
    every expert down_proj, applied in the matmul epilogue, against the
    oracle doing the same edit."""
    spec = mg.moe("int4", dense_first=1)
    rng = np.random.default_rng(3)
    v, _ = np.linalg.qr(rng.standard_normal((spec.config["hidden"], 2)))
    v = v.T.astype(np.float32)
    tokens, rows, last = mg.batch(6, [30, 12, 64], spec.config["vocab"], seed=5)  # 212 rows: the tiled product
    gm = Model(dev, spec)
    cm = RefModel(spec)
    try:
        for li in range(spec.config["layers"]):
            for m in (gm, cm):
                m.edit(li, abi.SLOT["O"], -1, v, 1.0)
                if spec.moe_layers[li]:
                    for e in range(spec.config["n_experts"]):
                        m.edit(li, abi.SLOT["EXPERT_DOWN"], e, v, 1.0)
                else:
                    m.edit(li, abi.SLOT["DOWN"], -1, v, 1.0)
        rg, lg = gm.forward(tokens, rows, capture_rows=last, logit_rows=last)
        rc, lc = cm.forward(tokens, rows, capture_rows=last, logit_rows=last)
        check_parity(ref, rg, lg, rc, lc, "edited")
        # the edit changed the model
        gm.reset_deltas()
        _, l0 = gm.forward(tokens, rows, logit_rows=last)
        assert np.abs(l0 - lg).max() > 1e-4
    finally:
        gm.free()
        cm.free()


@pytest.mark.parametrize("lens", [[3, 1], [30, 12, 64]])
def test_high_rank_deltas_then_forward(dev, ref, lens):
    """Deltas of rank 80 and 130 (no cap in the reference's setDelta,
    tensor.zig:588-592) on o_proj, the dense down_proj and every routed
    expert's down_proj, at decode-sized and tiled row counts."""
    spec = mg.moe("int4", dense_first=1)
    c = spec.config
    tokens, rows, last = mg.batch(len(lens), lens, c["vocab"], seed=7)
    gm = Model(dev, spec)
    cm = RefModel(spec)
    rng = np.random.default_rng(sum(lens))
    try:
        for li in range(c["layers"]):
            slots = [(abi.SLOT["O"], -1, c["hidden"], c["heads"] * c["head_dim"], 80)]
            if spec.moe_layers[li]:
                slots += [(abi.SLOT["EXPERT_DOWN"], e, c["hidden"], c["moe_inter"], 130 if e % 2 else 80)
                          for e in range(c["n_experts"])]
            else:
                slots.append((abi.SLOT["DOWN"], -1, c["hidden"], c["inter"], 130))
            for slot, e, r, k, rank in slots:
                a = (rng.standard_normal((rank, k)) * 0.02).astype(np.float32)
                b = (rng.standard_normal((r, rank)) * 0.02).astype(np.float32)
                gm.set_delta(li, slot, e, a, b)
                cm.set_delta(li, slot, e, a, b)
        rg, lg = gm.forward(tokens, rows, capture_rows=last, logit_rows=last)
        rc, lc = cm.forward(tokens, rows, capture_rows=last, logit_rows=last)
    finally:
        gm.free()
        cm.free()
    check_parity(ref, rg, lg, rc, lc, "high_rank")


@pytest.mark.parametrize("lens", [[20, 28], [130, 82]])
def test_edit_split_k_products(dev, ref, lens):
    """Rank-2 edits of o_proj and down_proj on a dense FP8 model whose
    down_proj (K = 1536) splits K over blocks: the delta, residual
    accumulate and the split-K partial sums meet in the second kernel; 48
    rows on the f32-row path, 212 on the fused producers."""
    spec = mg.dense("fp8", hidden=256, inter=1536, seed=9)
    rng = np.random.default_rng(4)
    v, _ = np.linalg.qr(rng.standard_normal((spec.config["hidden"], 2)))
    v = v.T.astype(np.float32)
    tokens, rows, last = mg.batch(2, lens, spec.config["vocab"], seed=11)
    gm = Model(dev, spec)
    cm = RefModel(spec)
    try:
        for li in range(spec.config["layers"]):
            for m in (gm, cm):
                m.edit(li, abi.SLOT["O"], -1, v, 1.0)
                m.edit(li, abi.SLOT["DOWN"], -1, v, 1.0)
        rg, lg = gm.forward(tokens, rows, capture_rows=last, logit_rows=last)
        rc, lc = cm.forward(tokens, rows, capture_rows=last, logit_rows=last)
    finally:
        gm.free()
        cm.free()
    check_parity(ref, rg, lg, rc, lc, "edited_split_k")


# Shapes that take the MFMA attention kernel (head dims 64/128, and MLA's
# 192/128): several 64-key chunks, prompts that share 16-row blocks, GQA
# groups of 4, and one query head per KV head.
ATTN_CASES = {
    "gqa4_hd128": (lambda: mg.dense("bf16", hidden=512, inter=512, heads=8, kv_heads=2, head_dim=128, seed=3),
                   [130, 7, 70, 16]),
    "gqa1_hd64": (lambda: mg.dense("mxfp4", hidden=256, inter=512, heads=4, kv_heads=4, head_dim=64, seed=4),
                  [65, 3, 129]),
    "mla_hd192": (lambda: mg.mla("bf16", hidden=256, heads=2, q_lora=64, kv_lora=64, nope=128, rope=64, v_dim=128,
                                 seed=5), [100, 33]),
}


@pytest.mark.parametrize("name", list(ATTN_CASES))
def test_long_prompt_attention_matches_oracle(dev, ref, name):
    make, lens = ATTN_CASES[name]
    spec = make()
    tokens, rows, last = mg.batch(len(lens), lens, spec.config["vocab"], seed=11)
    # capture every row of the last prompt as well: attention of early positions
    cap = sorted(set(last) | set(range(len(tokens) - lens[-1], len(tokens))))
    gm = Model(dev, spec)
    cm = RefModel(spec)
    try:
        rg, lg = gm.forward(tokens, rows, capture_rows=cap, logit_rows=last)
        rc, lc = cm.forward(tokens, rows, capture_rows=cap, logit_rows=last)
    finally:
        gm.free()
        cm.free()
    check_parity(ref, rg, lg, rc, lc, name)


# Equal-length prompts flattened in order are dense rows (row r = prompt r / T
# at position r % T): the whole-prompt attention kernel's case when T <= 128.
DENSE_CASES = {
    "gqa4_hd128_T128": (lambda: mg.dense("bf16", hidden=512, inter=512, heads=8, kv_heads=2, head_dim=128, seed=3),
                        3, 128),
    "gqa7_hd64_T64": (lambda: mg.dense("f32", hidden=896, inter=512, heads=14, kv_heads=2, head_dim=64,
                                       embed_fmt="f32", seed=6), 4, 64),
    "gqa8_hd128_T100": (lambda: mg.dense("mxfp4", hidden=512, inter=512, heads=16, kv_heads=2, head_dim=128, seed=7),
                        2, 100),
    "gqa1_hd64_T33": (lambda: mg.dense("fp8", hidden=256, inter=512, heads=4, kv_heads=4, head_dim=64, seed=8), 3, 33),
}


@pytest.mark.parametrize("name", list(DENSE_CASES))
def test_dense_prompt_attention_matches_per_block_kernel_and_oracle(dev, ref, name):
    """The dense batch (whole-prompt attention kernel) gives the same bits at
    every row as the same rows shuffled (not dense: the per-block kernel),
    and matches the oracle; T = 100 and 33 leave partial 16-row blocks and
    32-key chunks."""
    make, B, T = DENSE_CASES[name]
    spec = make()
    tokens, rows, last = mg.batch(B, [T], spec.config["vocab"], seed=T)
    n = len(tokens)
    assert rows == [(r // T, r % T) for r in range(n)]
    perm = np.random.default_rng(T).permutation(n)
    inv = np.argsort(perm)
    rows_p = [rows[i] for i in perm]
    gm = Model(dev, spec)
    cm = RefModel(spec)
    try:
        rg, lg = gm.forward(tokens, rows, capture_rows=list(range(n)), logit_rows=last)
        rp, lp = gm.forward(tokens[perm], rows_p, capture_rows=[int(inv[r]) for r in range(n)],
                            logit_rows=[int(inv[r]) for r in last])
        rc, lc = cm.forward(tokens, rows, capture_rows=last, logit_rows=last)
    finally:
        gm.free()
        cm.free()
    np.testing.assert_array_equal(rg, rp)
    np.testing.assert_array_equal(lg, lp)
    check_parity(ref, rg[:, last], lg, rc, lc, name)


# ---------------------------------------------------------------------------
# Routed-expert streaming (expert_cache.zig:108-607)


def _moe_forward(gm, cm, tokens, rows, last):
    rg, lg = gm.forward(tokens, rows, capture_rows=last, logit_rows=last)
    rc, lc = cm.forward(tokens, rows, capture_rows=last, logit_rows=last)
    return rg, lg, rc, lc


def _cache_geometry(dev, spec, tokens, rows, last):
    """(slot bytes, slot count) of a cache whose budget holds every expert."""
    probe = Model(dev, spec, expert_cache_bytes=1 << 40)
    try:
        probe.forward(tokens, rows, logit_rows=last)
        st = probe.expert_cache_stats()
        assert st["misses"] > 0 and st["bytes_read"] > 0 and st["resident"] == st["misses"]
        return st["slot_bytes"], st["slots"]
    finally:
        probe.free()


@pytest.mark.parametrize("fraction", [1.0, 0.4, 0.0])
def test_streamed_experts_match_oracle(dev, ref, fraction):
    """Experts kept in pinned host memory and copied into a device cache that
    holds every expert (fraction 1), 40 % of them (layers run in chunks) or
    exactly one (fraction 0): the forward equals the oracle's, twice in a
    row; a cache as large as the model misses each expert once and then
    only hits."""
    spec = mg.moe("int4", layers=3, dense_first=1, experts=16, top_k=4, seed=21)
    tokens, rows, last = mg.batch(3, [40, 17, 64], spec.config["vocab"], seed=9)
    slot, total = _cache_geometry(dev, spec, tokens, rows, last)
    assert total == 2 * 16
    budget = max(slot, int(fraction * total) * slot)
    gm = Model(dev, spec, expert_cache_bytes=budget)
    cm = RefModel(spec)
    try:
        for it in range(2):
            rg, lg, rc, lc = _moe_forward(gm, cm, tokens, rows, last)
            check_parity(ref, rg, lg, rc, lc, f"streamed {fraction} pass {it}")
        st = gm.expert_cache_stats()
        assert st["slots"] == budget // slot
        if fraction == 1.0:
            assert st["evictions"] == 0 and st["hits"] == st["misses"]  # second pass: every expert resident
        else:
            assert st["evictions"] > 0
    finally:
        gm.free()
        cm.free()


def test_streamed_expert_edit_matches_oracle(dev, ref):
    """The rank-2 edit of streamed experts' down projections (the edit reads a
    device copy of each expert's blob) against the oracle doing the same."""
    spec = mg.moe("int4", dense_first=1, seed=4)
    rng = np.random.default_rng(8)
    v, _ = np.linalg.qr(rng.standard_normal((spec.config["hidden"], 2)))
    v = v.T.astype(np.float32)
    tokens, rows, last = mg.batch(3, [30, 12, 64], spec.config["vocab"], seed=6)
    slot, _ = _cache_geometry(dev, spec, tokens, rows, last)
    gm = Model(dev, spec, expert_cache_bytes=3 * slot)
    cm = RefModel(spec)
    try:
        for li in range(spec.config["layers"]):
            if spec.moe_layers[li]:
                for e in range(spec.config["n_experts"]):
                    for m in (gm, cm):
                        m.edit(li, abi.SLOT["EXPERT_DOWN"], e, v, 1.0)
        rg, lg, rc, lc = _moe_forward(gm, cm, tokens, rows, last)
        check_parity(ref, rg, lg, rc, lc, "streamed edit")
    finally:
        gm.free()
        cm.free()


@pytest.mark.parametrize("streamed", [False, True])
def test_edit_batch_matches_per_matrix_edits_and_oracle(dev, ref, streamed):
    """One ditch_hip_model_edit_batch call over every layer's o_proj (layer
    0's in bf16, the rest INT4: two tile formats in one batch), the dense
    layer's down_proj and every routed expert's down_proj, with a direction
    set and weight per layer (abliterate.apply, abliterate.zig:148-210):
    the same forward, bit for bit, as one ditch_hip_model_edit per matrix,
    and the oracle's forward after the same edits; with the experts
    streamed, their blobs are staged on the device one at a time."""
    spec = mg.moe("int4", dense_first=1, seed=12)
    gen_o = np.random.default_rng(13)
    from ditch_amd import synth
    import torch
    spec.set("O", synth.bf16_weight(torch.from_numpy(gen_o.normal(0, 0.02, (256, 256)).astype(np.float32))), 0)
    rng = np.random.default_rng(14)
    L, E = spec.config["layers"], spec.config["n_experts"]
    targets = []
    for li in range(L):
        v, _ = np.linalg.qr(rng.standard_normal((spec.config["hidden"], 2)))
        v = np.ascontiguousarray(v.T.astype(np.float32))
        targets.append((li, abi.SLOT["O"], -1, v, 0.5 + 0.25 * li))
        if spec.moe_layers[li]:
            targets += [(li, abi.SLOT["EXPERT_DOWN"], e, v, 1.0) for e in range(E)]
        else:
            targets.append((li, abi.SLOT["DOWN"], -1, v, 0.9))
    tokens, rows, last = mg.batch(3, [30, 12, 64], spec.config["vocab"], seed=15)
    budget = 0
    if streamed:
        slot, _ = _cache_geometry(dev, spec, tokens, rows, last)
        budget = 3 * slot
    gm = Model(dev, spec, expert_cache_bytes=budget)
    cm = RefModel(spec)
    try:
        gm.edit_batch(targets, 2)
        rg, lg = gm.forward(tokens, rows, capture_rows=last, logit_rows=last)
        gm.reset_deltas()
        for layer, slot_, e, v, wt in targets:
            gm.edit(layer, slot_, e, v, wt)
            cm.edit(layer, slot_, e, v, wt)
        rg1, lg1 = gm.forward(tokens, rows, capture_rows=last, logit_rows=last)
        rc, lc = cm.forward(tokens, rows, capture_rows=last, logit_rows=last)
    finally:
        gm.free()
        cm.free()
    np.testing.assert_array_equal(lg, lg1)
    np.testing.assert_array_equal(rg, rg1)
    check_parity(ref, rg, lg, rc, lc, "edit batch")


def test_expert_cache_rejects_late_budget_and_tiny_budget(dev):
    from ditch_amd.hip import DeviceError
    spec = mg.moe("int4", dense_first=1, seed=2)
    gm = Model(dev, spec)
    try:
        with pytest.raises(DeviceError, match="registered before"):
            dev.check(dev.lib.ditch_hip_model_set_expert_cache(gm.h, 1 << 30))
    finally:
        gm.free()
    tokens, rows, last = mg.batch(2, [5, 7], spec.config["vocab"], seed=1)
    gm = Model(dev, spec, expert_cache_bytes=1024)
    try:
        with pytest.raises(DeviceError, match="below one expert"):
            gm.forward(tokens, rows, logit_rows=last)
    finally:
        gm.free()


# ---------------------------------------------------------------------------
# Config C4's layer shape (Qwen3-30B-A3B INT4 MoE + rank-2 edit)


def test_c4_shape_moe_forward_edit_and_streaming(dev, ref):
    """Two layers at C4's width (d 2048, 32/4 heads of 128, 128 experts top-8
    of FFN 768, INT4 group 128): the forward, then the rank-2 none-mode edit
    of every o_proj and every expert's down_proj (abliterate.zig:167-188,
    264-280), resident and with the experts streamed through a cache of a
    quarter of them, each against the oracle."""
    spec = mg.moe_c4(layers=2, seed=12)
    tokens, rows, last = mg.batch(4, [32, 20, 48, 28], spec.config["vocab"], seed=3)
    rng = np.random.default_rng(14)
    v, _ = np.linalg.qr(rng.standard_normal((spec.config["hidden"], 2)))
    v = v.T.astype(np.float32)
    cm = RefModel(spec)
    gm = Model(dev, spec)
    gs = None
    try:
        rg, lg, rc, lc = _moe_forward(gm, cm, tokens, rows, last)
        check_parity(ref, rg, lg, rc, lc, "c4 shape")
        for li in range(spec.config["layers"]):
            for m in (gm, cm):
                m.edit(li, abi.SLOT["O"], -1, v, 1.0)
                for e in range(spec.config["n_experts"]):
                    m.edit(li, abi.SLOT["EXPERT_DOWN"], e, v, 1.0)
        rg2, lg2, rc2, lc2 = _moe_forward(gm, cm, tokens, rows, last)
        check_parity(ref, rg2, lg2, rc2, lc2, "c4 shape edited")
        assert np.abs(lc2 - lc).max() > 1e-4  # the edit changed the model
        gm.free()
        slot, _ = _cache_geometry(dev, spec, tokens, rows, last)
        gs = Model(dev, spec, expert_cache_bytes=2 * 128 * slot // 4)
        for li in range(spec.config["layers"]):
            gs.edit(li, abi.SLOT["O"], -1, v, 1.0)
            for e in range(spec.config["n_experts"]):
                gs.edit(li, abi.SLOT["EXPERT_DOWN"], e, v, 1.0)
        rs, ls = gs.forward(tokens, rows, capture_rows=last, logit_rows=last)
        check_parity(ref, rs, ls, rc2, lc2, "c4 shape edited, streamed")
        st = gs.expert_cache_stats()
        assert st["slots"] == 64 and st["evictions"] > 0
    finally:
        gm.free()
        if gs is not None:
            gs.free()
        cm.free()


# ---------------------------------------------------------------------------
# Config C5's layer shapes (DeepSeek-V3 FP8, MLA, group-limited routing)


def test_c5_shape_mla_moe_streamed(dev, ref):
    """A dense and a routed layer at C5's width (d 7168, MLA over 128 heads,
    dense FFN 18432, experts of FFN 2048 top-8 of 8 groups keeping 4,
    shared expert, FP8 128 x 128): resident, and with the routed experts
    streamed through a cache of a quarter of them (the C5 configuration's
    96 GB cache over 101.5 GB of experts, scaled to 64 experts), against the
    oracle."""
    spec = mg.mla_c5(experts=64, seed=5)
    tokens, rows, last = mg.batch(2, [40, 24], spec.config["vocab"], seed=3)
    cm = RefModel(spec, threads=16)
    try:
        rc, lc = cm.forward(tokens, rows, capture_rows=last, logit_rows=last)
        gm = Model(dev, spec)
        try:
            rg, lg = gm.forward(tokens, rows, capture_rows=last, logit_rows=last)
        finally:
            gm.free()
        check_parity(ref, rg, lg, rc, lc, "c5 shape")
        slot, total = _cache_geometry(dev, spec, tokens, rows, last)
        assert total == 64
        gs = Model(dev, spec, expert_cache_bytes=16 * slot)
        try:
            for it in range(2):
                rs, ls = gs.forward(tokens, rows, capture_rows=last, logit_rows=last)
                check_parity(ref, rs, ls, rc, lc, f"c5 shape streamed pass {it}")
            st = gs.expert_cache_stats()
            assert st["slots"] == 16 and st["evictions"] > 0
        finally:
            gs.free()
    finally:
        cm.free()
