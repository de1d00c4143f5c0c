"""The benchmark configurations at their own widths on the GPU, against the
oracle, and the device-resident entry points (forward_device with the KV
cache shape, log-softmax and KL on device memory).

Bars (the same as test_gpu_forward.py): logits
within 1e-3 of max |logit|, per-prompt KL(CPU || GPU) <= 1e-4 with
scorers.zig:387-394's formula, residuals within 1e-3 relative.
"""
import numpy as np
import pytest

import model_gen as mg
from ditch_amd import abi, hipmem, synth
from ditch_amd.hip import DeviceError, Model
from oracle.ref import RefModel
from test_gpu_forward import check_parity

pytestmark = pytest.mark.gpu


def _prompt_kl(ref, log_c, log_g, tails):
    """scorers.zig:378-402: per-prompt mean over its tail rows of
    KL(base || trial), base = the oracle's logits."""
    kl = ref.kl_rows(ref.log_softmax_rows(log_c), log_g)
    out, i = [], 0
    for t in tails:
        out.append(kl[i:i + t].mean())
        i += t
    return np.array(out)


def _run_both(dev, spec, tokens, rows, last, threads=16):
    cm = RefModel(spec, threads=threads)
    try:
        rc, lc = cm.forward(tokens, rows, capture_rows=last, logit_rows=last)
    finally:
        cm.free()
    gm = Model(dev, spec)
    try:
        rg, lg = gm.forward(tokens, rows, capture_rows=last, logit_rows=last)
        stats = gm.path_stats()
    finally:
        gm.free()
    return rg, lg, rc, lc, stats


def test_c1_width_f32_forward(dev, ref):
    """Config C1 at its width: Qwen2.5-0.5B-shaped (d 896, FFN 4864, 14 q /
    2 kv heads of 64, q/k/v bias, tied f32 embedding of 151 936 rows, theta
    1e6), f32 weights N(0, 0.02), two layers, 16 prompts x 64 tokens."""
    spec = mg.dense("f32", hidden=896, inter=4864, layers=2, heads=14, kv_heads=2, head_dim=64, vocab=151936,
                    qkv_bias=True, embed_fmt="f32", tie=True, rope_theta=1e6, seed=31)
    tokens, rows, last = mg.batch(16, [64], spec.config["vocab"], seed=32)
    rg, lg, rc, lc, _ = _run_both(dev, spec, tokens, rows, last)
    check_parity(ref, rg, lg, rc, lc, "c1 width")
    assert _prompt_kl(ref, lc, lg, [1] * 16).max() <= 1e-4


@pytest.mark.parametrize("fmt", ["mxfp4", "fp8"])
def test_c3_width_forward(dev, ref, fmt):
    """Config C3 at its width and batch: Llama-3-8B-shaped (d 4096, FFN
    14336, 32/8 heads of 128, vocab 128 256, theta 5e5, eps 1e-5), linear
    weights MXFP4 or FP8 E4M3 with 128 x 128 block scales, bf16 embedding and
    lm_head, two layers, 64 prompts x 128 tokens: logits, residuals at every
    layer entry and per-prompt KL against the oracle."""
    import torch
    gen = torch.Generator().manual_seed(41 if fmt == "mxfp4" else 42)
    h, ff, nh, nkv, hd, V, L = 4096, 14336, 32, 8, 128, 128256, 2
    from ditch_amd.spec import ModelSpec
    spec = ModelSpec(hidden=h, inter=ff, layers=L, heads=nh, kv_heads=nkv, head_dim=hd, vocab=V, rms_eps=1e-5,
                     rope_theta=5e5, rope_len=8192, tie_embeddings=0)
    q = synth.QUANTIZERS[fmt]
    spec.set("EMBED", synth.bf16_weight(torch.randn(V, h, generator=gen) * 0.02))
    spec.set("LM_HEAD", synth.bf16_weight(torch.randn(V, h, generator=gen) * 0.02))
    spec.set("FINAL_NORM", (1 + torch.randn(h, generator=gen) * 0.02).numpy())
    for li in range(L):
        for name, r, c in (("Q", nh * hd, h), ("K", nkv * hd, h), ("V", nkv * hd, h), ("O", h, nh * hd),
                           ("GATE", ff, h), ("UP", ff, h), ("DOWN", h, ff)):
            spec.set(name, q(torch.randn(r, c, generator=gen) * 0.02), li)
        spec.set("ATTN_NORM", (1 + torch.randn(h, generator=gen) * 0.02).numpy(), li)
        spec.set("FFN_NORM", (1 + torch.randn(h, generator=gen) * 0.02).numpy(), li)
    tokens, rows, last = mg.batch(64, [128], V, seed=43)
    rg, lg, rc, lc, _ = _run_both(dev, spec, tokens, rows, last)
    check_parity(ref, rg, lg, rc, lc, f"c3 width {fmt}")
    assert _prompt_kl(ref, lc, lg, [1] * 64).max() <= 1e-4


def test_c4_layer_at_full_batch_takes_the_device_plan(dev, ref):
    """One layer at C4's width over C4's batch (32 prompts x 128 tokens:
    32 768 token-expert pairs, about 256 per expert, several tile rows per
    expert segment), resident and unedited: the routed products are planned
    on the device (no count read-back) and the forward matches the oracle."""
    spec = mg.moe_c4(layers=1, seed=51)
    tokens, rows, last = mg.batch(32, [128], spec.config["vocab"], seed=52)
    rg, lg, rc, lc, stats = _run_both(dev, spec, tokens, rows, last)
    assert stats["moe_device_planned"] == 1 and stats["moe_host_planned"] == 0, stats
    check_parity(ref, rg, lg, rc, lc, "c4 layer full batch")


def test_c4_layer_edited_in_one_batch_stays_on_the_device_plan(dev, ref):
    """The same layer with the rank-2 none-mode edit of o_proj and all 128
    expert down projections made by one ditch_hip_model_edit_batch call
    (abliterate.apply, abliterate.zig:148-210): the deltas equal those of
    one ditch_hip_model_edit per matrix (the same forward, bit for bit), the
    edited routed layer is still planned on the device (its down deltas in
    the device segment table), and the forward matches the oracle doing the
    same edit."""
    spec = mg.moe_c4(layers=1, seed=51)
    tokens, rows, last = mg.batch(32, [128], spec.config["vocab"], seed=52)
    rng = np.random.default_rng(53)
    v, _ = np.linalg.qr(rng.standard_normal((spec.config["hidden"], 2)))
    v = np.ascontiguousarray(v.T.astype(np.float32))
    E = spec.config["n_experts"]
    targets = [(0, abi.SLOT["O"], -1, v, 0.8)] + [(0, abi.SLOT["EXPERT_DOWN"], e, v, 1.0) for e in range(E)]
    cm = RefModel(spec, threads=16)
    try:
        for layer, slot, e, vv, wt in targets:
            cm.edit(layer, slot, e, vv, wt)
        rc, lc = cm.forward(tokens, rows, capture_rows=last, logit_rows=last)
    finally:
        cm.free()
    gm = Model(dev, spec)
    try:
        gm.edit_batch(targets, 2)
        before = gm.path_stats()
        rg, lg = gm.forward(tokens, rows, capture_rows=last, logit_rows=last)
        after = gm.path_stats()
        assert after["moe_device_planned"] - before["moe_device_planned"] == 1, after
        assert after["moe_host_planned"] == before["moe_host_planned"], after
        gm.reset_deltas()
        for layer, slot, e, vv, wt in targets:
            gm.edit(layer, slot, e, vv, wt)
        rg1, lg1 = gm.forward(tokens, rows, capture_rows=last, logit_rows=last)
        gm.reset_deltas()
        _, l0 = gm.forward(tokens, rows, logit_rows=last)
    finally:
        gm.free()
    np.testing.assert_array_equal(lg, lg1)
    np.testing.assert_array_equal(rg, rg1)
    check_parity(ref, rg, lg, rc, lc, "c4 layer edited in one batch")
    assert np.abs(l0 - lg).max() > 1e-4  # the edit changed the model


def test_mla_attention_256_keys(dev, ref):
    """MLA (head dims 192 / 128) over prompts of C5's 256 tokens: the
    attention kernel's uncached two-pass path (more than 128 keys)."""
    spec = mg.mla("bf16", hidden=256, heads=2, q_lora=64, kv_lora=64, nope=128, rope=64, v_dim=128, seed=61)
    tokens, rows, last = mg.batch(3, [256, 200, 256], spec.config["vocab"], seed=62)
    cap = sorted(set(last) | set(range(len(tokens) - 256, len(tokens), 17)))
    cm = RefModel(spec)
    gm = Model(dev, spec)
    try:
        rg, lg = gm.forward(tokens, rows, capture_rows=cap, logit_rows=last)
        rc, lc = cm.forward(tokens, rows, capture_rows=cap, logit_rows=last)
    finally:
        gm.free()
        cm.free()
    check_parity(ref, rg, lg, rc, lc, "mla 256 keys")


# ---------------------------------------------------------------------------
# Device-resident entry points


def _device_forward(gm, spec, tokens, rows, cap, lr, n_prompts, max_len):
    c = spec.config
    rows_a = np.ascontiguousarray(rows, dtype=np.uint32).reshape(-1, 2)
    cap_a, lr_a = np.asarray(cap, dtype=np.uint64), np.asarray(lr, dtype=np.uint64)
    bt, br = hipmem.Buffer.from_array(np.asarray(tokens, dtype=np.uint32)), hipmem.Buffer.from_array(rows_a)
    bc, bl = hipmem.Buffer.from_array(cap_a), hipmem.Buffer.from_array(lr_a)
    bres = hipmem.Buffer((c["layers"] + 1) * cap_a.size * c["hidden"] * 4)
    blog = hipmem.Buffer(lr_a.size * c["vocab"] * 4)
    gm.forward_device(bt.ptr, br.ptr, len(tokens), n_prompts, max_len, bc.ptr, cap_a.size, bres.ptr, bl.ptr,
                      lr_a.size, blog.ptr)
    return bres, blog


def test_forward_device_matches_forward_and_scores_on_device(dev, ref):
    """forward_device (KV cache shape from the caller, nothing read back) gives
    the host forward's outputs bit for bit; the log-softmax and the KL of its
    logits computed on device memory match the oracle."""
    spec = mg.dense("bf16", qkv_bias=True, vocab=5000, seed=71)
    tokens, rows, last = mg.batch(5, [33, 7, 64, 1, 20], spec.config["vocab"], seed=72)
    gm = Model(dev, spec)
    try:
        rh, lh = gm.forward(tokens, rows, capture_rows=last, logit_rows=last)
        bres, blog = _device_forward(gm, spec, tokens, rows, last, last, 5, 64)
        dev.sync()
        rd = bres.download(np.float32, rh.shape)
        ld = blog.download(np.float32, lh.shape)
        np.testing.assert_array_equal(rd, rh)
        np.testing.assert_array_equal(ld, lh)
        n, V = lh.shape
        bout = hipmem.Buffer(n * V * 4)
        dev.logSoftmaxRows_device(bout.ptr, blog.ptr, n, V)
        base = ref.log_softmax_rows(lh * 1.5)
        bbase = hipmem.Buffer.from_array(base.astype(np.float32))
        bkl = hipmem.Buffer(n * 8)
        dev.klRows_device(bkl.ptr, bbase.ptr, blog.ptr, n, V)
        dev.sync()
        np.testing.assert_allclose(bout.download(np.float32, (n, V)), ref.log_softmax_rows(lh), atol=1e-5, rtol=1e-4)
        np.testing.assert_allclose(bkl.download(np.float64, (n,)), ref.kl_rows(base, lh), atol=1e-9, rtol=1e-5)
        # in place
        dev.logSoftmaxRows_device(blog.ptr, blog.ptr, n, V)
        dev.sync()
        np.testing.assert_allclose(blog.download(np.float32, (n, V)), ref.log_softmax_rows(lh), atol=1e-5, rtol=1e-4)
    finally:
        gm.free()


@pytest.mark.parametrize("n,V", [(1, 7), (3, 128256), (64, 128256), (200, 2049)])
def test_log_softmax_and_kl_device_row_split(dev, ref, n, V):
    """Rows split over several workgroups (a 128 k vocabulary over few rows)
    or one chunk each (short rows): the oracle's log-softmax (f32 max, f64
    sum) and f64 KL."""
    rng = np.random.default_rng(n * 7 + V)
    x = (rng.standard_normal((n, V)) * 3).astype(np.float32)
    x[0, rng.integers(V)] = 40.0  # one dominant logit
    base = ref.log_softmax_rows((x * 0.5 + rng.standard_normal((n, V)).astype(np.float32)).astype(np.float32))
    bx, bb = hipmem.Buffer.from_array(x), hipmem.Buffer.from_array(base.astype(np.float32))
    bo, bk = hipmem.Buffer(n * V * 4), hipmem.Buffer(n * 8)
    dev.logSoftmaxRows_device(bo.ptr, bx.ptr, n, V)
    dev.klRows_device(bk.ptr, bb.ptr, bx.ptr, n, V)
    dev.sync()
    np.testing.assert_allclose(bo.download(np.float32, (n, V)), ref.log_softmax_rows(x), atol=1e-5, rtol=1e-4)
    np.testing.assert_allclose(bk.download(np.float64, (n,)), ref.kl_rows(base, x), atol=1e-9, rtol=1e-5)
    # the host entry points run the same kernels
    np.testing.assert_array_equal(dev.logSoftmaxRows(x), bo.download(np.float32, (n, V)))


def test_forward_device_skips_rows_outside_the_cache(dev, ref):
    """A row whose position is past the caller's KV cache is skipped on the
    device (no access leaves the cache); the other prompts' outputs are those
    of the full forward."""
    spec = mg.dense("bf16", vocab=3000, seed=81)
    tokens, rows, last = mg.batch(2, [16, 40], spec.config["vocab"], seed=82)
    gm = Model(dev, spec)
    try:
        rh, lh = gm.forward(tokens, rows, capture_rows=last, logit_rows=last)
        bres, blog = _device_forward(gm, spec, tokens, rows, last, last, 2, 16)  # prompt 1 runs past 16
        dev.sync()
        rd = bres.download(np.float32, rh.shape)
        ld = blog.download(np.float32, lh.shape)
        np.testing.assert_array_equal(rd[:, 0], rh[:, 0])
        np.testing.assert_array_equal(ld[0], lh[0])
    finally:
        gm.free()


def test_forward_device_refuses_short_outputs(dev):
    spec = mg.dense("bf16", vocab=1000, seed=91)
    tokens, rows, last = mg.batch(2, [8, 8], spec.config["vocab"], seed=92)
    gm = Model(dev, spec)
    try:
        c = spec.config
        bt = hipmem.Buffer.from_array(np.asarray(tokens, dtype=np.uint32))
        br = hipmem.Buffer.from_array(np.asarray(rows, dtype=np.uint32).reshape(-1, 2))
        bl = hipmem.Buffer.from_array(np.asarray(last, dtype=np.uint64))
        blog = hipmem.Buffer(2 * c["vocab"] * 4)
        with pytest.raises(DeviceError, match="logit buffer"):
            gm.forward_device(bt.ptr, br.ptr, 16, 2, 8, None, 0, None, bl.ptr, 2, blog.ptr,
                              logit_bytes=2 * c["vocab"] * 4 - 4)
        with pytest.raises(DeviceError, match="KV cache"):
            gm.forward_device(bt.ptr, br.ptr, 16, 0, 8, None, 0, None, bl.ptr, 2, blog.ptr)
    finally:
        gm.free()


def test_model_set_refuses_misshaped_experts_and_dropped_deltas(dev):
    """A routed expert whose shape differs from the configuration is refused
    at registration (no kernel ever sees it); deltas on slots the forward
    applies none to (embedding, expert gate/up) are refused."""
    spec = mg.moe("int4", dense_first=1, seed=3)
    gm = Model(dev, spec)
    try:
        c = spec.config
        rng = np.random.default_rng(1)
        bad = synth.int4_random(c["hidden"] + 128, c["moe_inter"], rng)
        with pytest.raises(DeviceError, match="expert down"):
            dev.check(dev.lib.ditch_hip_model_set(gm.h, 1, abi.SLOT["EXPERT_DOWN"], 0, bad.ref()))
        bad = synth.int4_random(c["moe_inter"], c["hidden"] + 128, rng)
        with pytest.raises(DeviceError, match="expert gate/up"):
            dev.check(dev.lib.ditch_hip_model_set(gm.h, 1, abi.SLOT["EXPERT_GATE"], 0, bad.ref()))
        v = np.linalg.qr(rng.standard_normal((c["moe_inter"], 1)))[0].T
        for slot in ("EXPERT_GATE", "EXPERT_UP"):
            with pytest.raises(DeviceError, match="not applied"):
                gm.edit(1, abi.SLOT[slot], 0, v, 1.0)
        with pytest.raises(DeviceError, match="not applied"):
            gm.set_delta(-1, abi.SLOT["EMBED"], -1, np.zeros((1, c["hidden"])), np.zeros((c["vocab"], 1)))
        # the model still runs
        tokens, rows, last = mg.batch(2, [5, 9], c["vocab"], seed=2)
        gm.forward(tokens, rows, logit_rows=last)
    finally:
        gm.free()
