"""Benchmark of the MI355X backend on BASELINE.json's headline metric.

Default workload: Llama-3-8B-shaped decoder, 32 layers, d=4096,
FFN 14336, GQA 32/8 x 128, vocab 128256, linear weights MXFP4 (`--workload
c3_fp8` for FP8 E4M3 with 128x128 block scales), bf16 embedding and lm_head.
A step is one resident forward over 64 prompts x 128 random tokens with the
last-token residual captured at every layer entry and the last-token logits,
followed by the log-softmax of those logit rows (the KL scorer's input,
tensor.zig:1203-1210). `value` = prompt tokens/s with inputs already in HBM.

Beside it, in the same JSON line:
  c3_fp8       - the same forward with FP8 128x128 linear weights (the other
                 half of the metric; c3_mxfp4 when the headline is FP8);
  roofline     - the dominant kernel of the headline forward: the fused
                 gate/up/SwiGLU product at the FFN shape, timed with HIP
                 events on the library's stream (roofline_fp8: the same for
                 the FP8 leg);
  gemv         - configs[1]: the Q8_0 14336x4096 dequant-fused product for
                 M in {1, 4, 16, 64, 256}, achieved HBM GB/s vs 8 TB/s
                 (gemv_cpu_baseline: the oracle's product for each M);
  c1           - configs[0]: Qwen2.5-0.5B-shaped f32 forward, 16 x 64 tokens,
                 its CPU baseline, and on the same model the rest of a
                 search trial (`trial`: the residual-mean pass over 400
                 prompts, greedy decode of 16 x 32 tokens, the none / pre /
                 full edit apply) beside the reference's published figures;
  c4           - configs[3]: Qwen3-30B-A3B-shaped INT4 MoE, 48 layers, 32 x
                 128 tokens, then the rank-2 edit of every o_proj and expert
                 down_proj (one batch call: its apply time) and the edited
                 forward, with its CPU baseline (a layer sample, scaled);
  c5           - configs[4] (`--no-c5` skips it; skipped with the reason when
                 host memory is short): DeepSeek-V3-shaped FP8, 12 layers,
                 256 experts streamed through a 96 GB HBM cache, 16 x 256
                 tokens, with its CPU baseline (a one-prompt sample of the
                 dense and the first routed layer, scaled);
  cpu_baseline - the CPU oracle (oracle/cpu_ref.c, built -march=native on
                 this host) on a sample of the benchmark's prompts at the
                 full depth, with the GPU's logits compared on that sample.
Only rank 0 / one GPU: `--gpus N` with N > 1 exits with a message.
"""
import argparse
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "prompt tokens/s (8B MXFP4/FP8 forward) + dequant-GEMV HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0
FP6_FP4_PEAK_TFLOPS = 10100.0  # dense MFMA, fp6 and fp4 operands
MX_TERMS = 4  # fp6 terms per activation on the scaled-MFMA (MXFP4) path
BF16_TERMS = 2  # bf16 terms per activation on the tiled bf16-MFMA path

C3 = dict(hidden=4096, inter=14336, layers=32, heads=32, kv_heads=8, head_dim=128, vocab=128256,
          rope_theta=500000.0, rms_eps=1e-5, prompts=64, tokens=128)
C1 = dict(hidden=896, inter=4864, layers=24, heads=14, kv_heads=2, head_dim=64, vocab=151936, rope_theta=1e6,
          rms_eps=1e-6, prompts=16, tokens=64)
C4 = dict(hidden=2048, layers=48, heads=32, kv_heads=4, head_dim=128, experts=128, top_k=8, moe_inter=768,
          vocab=151936, prompts=32, tokens=128)
C5 = dict(hidden=7168, layers=12, dense_layers=3, heads=128, q_lora=1536, kv_lora=512, nope=128, rope=64, v_dim=128,
          dense_ff=18432, experts=256, top_k=8, moe_inter=2048, vocab=129280, prompts=16, tokens=256,
          cache_bytes=96 * 10**9)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_share():
    """Cores this process may use, capped at the GPU box's share of 16 per GPU."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


# host bytes the C5 leg needs: 2 304 routed expert blobs of ~44 MB each plus
# the trunk, with room for the rest of the process
C5_HOST_BYTES = 120 * 10**9


def host_mem_available():
    try:
        for line in open("/proc/meminfo"):
            if line.startswith("MemAvailable:"):
                return int(line.split()[1]) * 1024
    except OSError:
        pass
    return None


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---------------------------------------------------------------------------
# synthetic models


def build_spec(fmt, cfg, layers=None, distinct=4, seed=0):
    """Llama-3-8B-shaped ModelSpec: N(0, 0.02) linear weights quantised to
    `fmt`; norms 1 + N(0, 0.02); bf16 embedding and lm_head. `distinct`
    random layers are generated and cycled over the layers (every layer is
    registered, so each has its own copy in HBM)."""
    import torch
    from ditch_amd import synth
    from ditch_amd.spec import ModelSpec

    torch.set_num_threads(cpu_share())
    L = cfg["layers"] if layers is None else layers
    h, ff, nh, nkv, hd, V = cfg["hidden"], cfg["inter"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["vocab"]
    spec = ModelSpec(hidden=h, inter=ff, layers=L, heads=nh, kv_heads=nkv, head_dim=hd, vocab=V,
                     rms_eps=cfg["rms_eps"], rope_theta=cfg["rope_theta"], rope_len=8192, tie_embeddings=0)
    gen = torch.Generator().manual_seed(seed)
    q = synth.QUANTIZERS[fmt]
    spec.set("EMBED", synth.bf16_weight(torch.randn(V, h, generator=gen) * 0.02))
    spec.set("LM_HEAD", synth.bf16_weight(torch.randn(V, h, generator=gen) * 0.02))
    spec.set("FINAL_NORM", (1 + torch.randn(h, generator=gen) * 0.02).numpy())
    pool = []
    for d in range(min(distinct, L)):
        t0 = time.time()
        lw = {}
        for name, r, c in (("Q", nh * hd, h), ("K", nkv * hd, h), ("V", nkv * hd, h), ("O", h, nh * hd),
                           ("GATE", ff, h), ("UP", ff, h), ("DOWN", h, ff)):
            lw[name] = q(torch.randn(r, c, generator=gen) * 0.02)
        lw["ATTN_NORM"] = (1 + torch.randn(h, generator=gen) * 0.02).numpy()
        lw["FFN_NORM"] = (1 + torch.randn(h, generator=gen) * 0.02).numpy()
        pool.append(lw)
        log(f"  synthetic layer {d} ({fmt}) in {time.time() - t0:.1f}s")
    for li in range(L):
        for name, w in pool[li % len(pool)].items():
            spec.set(name, w, li)
    return spec


def c1_spec(seed=0):
    """Qwen2.5-0.5B-shaped, f32 weights N(0, 0.02), norms
    1 + N(0, 0.02), q/k/v biases, tied f32 embedding, theta 1e6."""
    import torch
    from ditch_amd import synth
    from ditch_amd.spec import ModelSpec
    c = C1
    gen = torch.Generator().manual_seed(seed)
    h, ff, nh, nkv, hd, V = c["hidden"], c["inter"], c["heads"], c["kv_heads"], c["head_dim"], c["vocab"]
    spec = ModelSpec(hidden=h, inter=ff, layers=c["layers"], heads=nh, kv_heads=nkv, head_dim=hd, vocab=V,
                     rms_eps=c["rms_eps"], rope_theta=c["rope_theta"], rope_len=8192, qkv_bias=1, tie_embeddings=1)
    f32 = lambda r, cc: synth.f32_weight(torch.randn(r, cc, generator=gen) * 0.02)
    vec = lambda n, one: ((1 if one else 0) + torch.randn(n, generator=gen) * 0.02).numpy()
    spec.set("EMBED", f32(V, h))
    spec.set("FINAL_NORM", vec(h, True))
    for li in range(c["layers"]):
        for name, r, cc in (("Q", nh * hd, h), ("K", nkv * hd, h), ("V", nkv * hd, h), ("O", h, nh * hd),
                            ("GATE", ff, h), ("UP", ff, h), ("DOWN", h, ff)):
            spec.set(name, f32(r, cc), li)
        spec.set("Q_BIAS", vec(nh * hd, False), li)
        spec.set("K_BIAS", vec(nkv * hd, False), li)
        spec.set("V_BIAS", vec(nkv * hd, False), li)
        spec.set("ATTN_NORM", vec(h, True), li)
        spec.set("FFN_NORM", vec(h, True), li)
    return spec


def c4_spec(layers, distinct=4, seed=21):
    """Qwen3-30B-A3B-shaped (d 2048, 32/4 heads of 128 with q/k
    head norm, 128 experts top-8 of FFN 768, softmax router with renorm),
    INT4 group-128 asymmetric linear weights drawn in the packed domain,
    router N(0, 0.02), bf16 embedding and lm_head (vocab 151 936). `distinct` random
    layers cycled over the layers (each layer registered: its own HBM copy)."""
    import torch
    from ditch_amd import abi, synth
    from ditch_amd.spec import ModelSpec
    c = C4
    rng = np.random.default_rng(seed)
    h, nh, nkv, hd, E, mi, V = c["hidden"], c["heads"], c["kv_heads"], c["head_dim"], c["experts"], c["moe_inter"], \
        c["vocab"]
    spec = ModelSpec(hidden=h, inter=4 * h, layers=layers, heads=nh, kv_heads=nkv, head_dim=hd, vocab=V, rms_eps=1e-6,
                     qk_norm=1, tie_embeddings=0, rope_theta=1e6, rope_len=8192, n_experts=E, top_k=c["top_k"],
                     moe_inter=mi, norm_topk_prob=1, scoring=abi.SCORING_SOFTMAX, moe_layers=[1] * layers)
    spec.set("EMBED", synth.bf16_weight(torch.from_numpy(rng.normal(0, 0.02, (V, h)).astype(np.float32))))
    spec.set("LM_HEAD", synth.bf16_weight(torch.from_numpy(rng.normal(0, 0.02, (V, h)).astype(np.float32))))
    spec.set("FINAL_NORM", 1 + rng.normal(0, 0.02, h))
    pool = []
    for d in range(min(distinct, layers)):
        lw = {("ATTN_NORM", -1): 1 + rng.normal(0, 0.02, h), ("FFN_NORM", -1): 1 + rng.normal(0, 0.02, h),
              ("Q_NORM", -1): 1 + rng.normal(0, 0.02, hd), ("K_NORM", -1): 1 + rng.normal(0, 0.02, hd)}
        for name, r, cc in (("Q", nh * hd, h), ("K", nkv * hd, h), ("V", nkv * hd, h), ("O", h, nh * hd)):
            lw[(name, -1)] = synth.int4_random(r, cc, rng)
        lw[("ROUTER", -1)] = synth.bf16_weight(torch.from_numpy(rng.normal(0, 0.02, (E, h)).astype(np.float32)))
        for e in range(E):
            lw[("EXPERT_GATE", e)] = synth.int4_random(mi, h, rng)
            lw[("EXPERT_UP", e)] = synth.int4_random(mi, h, rng)
            lw[("EXPERT_DOWN", e)] = synth.int4_random(h, mi, rng)
        pool.append(lw)
    for li in range(layers):
        for (name, e), w in pool[li % len(pool)].items():
            spec.set(name, w, li, e)
    return spec


def c5_spec(distinct_experts=8, seed=5, layers=None):
    """DeepSeek-V3-shaped first 12 layers (d 7168, MLA q_lora
    1536 / kv_lora 512 / nope 128 / rope 64 / v 128 over 128 heads, 3 dense
    layers of FFN 18432, then 256 routed experts of FFN 2048 top-8 of 8
    groups keeping 4, sigmoid router with zero correction bias, scaling 2.5,
    one shared expert), FP8 E4M3 with 128 x 128 f32 block scales drawn in the
    code domain; `distinct_experts` expert triples cycled over the 256 x 9
    routed experts (each registered separately)."""
    import torch
    from ditch_amd import abi, synth
    from ditch_amd.spec import ModelSpec
    c = C5
    rng = np.random.default_rng(seed)
    h, nh, hd = c["hidden"], c["heads"], c["nope"] + c["rope"]
    E, mi, V, L = c["experts"], c["moe_inter"], c["vocab"], layers or c["layers"]
    moe = [0] * c["dense_layers"] + [1] * (L - c["dense_layers"])
    spec = ModelSpec(hidden=h, inter=c["dense_ff"], layers=L, heads=nh, kv_heads=nh, head_dim=hd,
                     v_head_dim=c["v_dim"], vocab=V, rms_eps=1e-6, tie_embeddings=0, rope_theta=10000.0,
                     rope_len=8192, rope_style=abi.ROPE_GPTJ, mla=1, q_lora_rank=c["q_lora"],
                     kv_lora_rank=c["kv_lora"], qk_nope_dim=c["nope"], qk_rope_dim=c["rope"],
                     attn_scale=float(np.float32(1) / np.sqrt(np.float32(hd))), n_experts=E, top_k=c["top_k"],
                     moe_inter=mi, norm_topk_prob=1, scoring=abi.SCORING_SIGMOID, group_limited=1, n_group=8,
                     topk_group=4, routed_scaling=2.5, shared_inter=mi, moe_layers=moe)
    f8 = lambda r, cc: synth.fp8_random(r, cc, rng)
    bf = lambda r, cc: synth.bf16_weight(torch.from_numpy(rng.normal(0, 0.02, (r, cc)).astype(np.float32)))
    spec.set("EMBED", bf(V, h))
    spec.set("LM_HEAD", bf(V, h))
    spec.set("FINAL_NORM", 1 + rng.normal(0, 0.02, h))
    trunk = {"MLA_Q_A": f8(c["q_lora"], h), "MLA_Q_B": f8(nh * hd, c["q_lora"]),
             "MLA_KV_A": f8(c["kv_lora"] + c["rope"], h), "MLA_KV_B": f8(nh * (c["nope"] + c["v_dim"]), c["kv_lora"]),
             "O": f8(h, nh * c["v_dim"])}
    dense = {"GATE": f8(c["dense_ff"], h), "UP": f8(c["dense_ff"], h), "DOWN": f8(h, c["dense_ff"])}
    shared = {"SHARED_GATE": f8(mi, h), "SHARED_UP": f8(mi, h), "SHARED_DOWN": f8(h, mi)}
    experts = [(f8(mi, h), f8(mi, h), f8(h, mi)) for _ in range(distinct_experts)]
    router = synth.f32_weight(torch.from_numpy(rng.normal(0, 0.02, (E, h)).astype(np.float32)))
    for li in range(L):
        spec.set("ATTN_NORM", 1 + rng.normal(0, 0.02, h), li)
        spec.set("FFN_NORM", 1 + rng.normal(0, 0.02, h), li)
        spec.set("MLA_Q_A_NORM", 1 + rng.normal(0, 0.02, c["q_lora"]), li)
        spec.set("MLA_KV_A_NORM", 1 + rng.normal(0, 0.02, c["kv_lora"]), li)
        for name, w in trunk.items():
            spec.set(name, w, li)
        if not moe[li]:
            for name, w in dense.items():
                spec.set(name, w, li)
            continue
        spec.set("ROUTER", router, li)
        spec.set("ROUTER_CORRECTION", np.zeros(E), li)
        for name, w in shared.items():
            spec.set(name, w, li)
        for e in range(E):
            g, u, d = experts[(e + li) % distinct_experts]
            spec.set("EXPERT_GATE", g, li, e)
            spec.set("EXPERT_UP", u, li, e)
            spec.set("EXPERT_DOWN", d, li, e)
    return spec


def make_batch(cfg, seed=1):
    rng = np.random.default_rng(seed)
    P, T = cfg["prompts"], cfg["tokens"]
    tokens = rng.integers(0, cfg["vocab"], P * T).astype(np.uint32)
    rows = np.array([(b, p) for b in range(P) for p in range(T)], dtype=np.uint32)
    last = np.array([b * T + T - 1 for b in range(P)], dtype=np.uint64)
    return tokens, rows, last


# ---------------------------------------------------------------------------
# GPU legs


def time_forward(dev, model, cfg, steps, warmup, batch=None):
    """One step = forward_device (residual capture at every layer entry, the
    last-token logits) + the log-softmax of those logit rows, both enqueued
    on the library stream; timed with HIP events on that stream."""
    from ditch_amd import hipmem
    tokens, rows, last = make_batch(cfg) if batch is None else batch
    n = tokens.size
    P, T = cfg["prompts"], cfg["tokens"]
    L, hidden, V = cfg["layers"], cfg["hidden"], cfg["vocab"]
    bt, br = hipmem.Buffer.from_array(tokens), hipmem.Buffer.from_array(rows)
    bc, bl = hipmem.Buffer.from_array(last), hipmem.Buffer.from_array(last)
    bres = hipmem.Buffer((L + 1) * last.size * hidden * 4)
    blog = hipmem.Buffer(last.size * V * 4)
    blp = hipmem.Buffer(last.size * V * 4)

    def step():
        model.forward_device(bt.ptr, br.ptr, n, P, T, bc.ptr, last.size, bres.ptr, bl.ptr, last.size, blog.ptr)
        dev.logSoftmaxRows_device(blp.ptr, blog.ptr, last.size, V)

    for _ in range(warmup):
        step()
    dev.sync()
    e0, e1 = hipmem.Event(), hipmem.Event()
    t0 = time.perf_counter()
    e0.record(dev.stream)
    for _ in range(steps):
        step()
    e1.record(dev.stream)
    e1.synchronize()
    hipmem.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_ms(e1) / steps
    res = bres.download(np.float32, (L + 1, last.size, hidden))
    logits = blog.download(np.float32, (last.size, V))
    logprobs = blp.download(np.float32, (last.size, V))
    return dict(ms=ms, wall=wall, res=res, logits=logits, logprobs=logprobs, batch=(tokens, rows, last))


def time_launches(dev, launch, reps):
    from ditch_amd import hipmem
    for _ in range(3):
        launch()
    dev.sync()
    e0, e1 = hipmem.Event(), hipmem.Event()
    e0.record(dev.stream)
    for _ in range(reps):
        launch()
    e1.record(dev.stream)
    e1.synchronize()
    return e0.elapsed_ms(e1) / reps


def time_matmul(dev, tensor, n, k, reps):
    """Average launch time of the tensor's product on n x k f32 activations
    (events on the context stream, which the kernel is launched on)."""
    from ditch_amd import hipmem
    rng = np.random.default_rng(3)
    x = hipmem.Buffer.from_array(rng.standard_normal((n, k)).astype(np.float32))
    out = hipmem.Buffer(n * tensor.rows * 4)
    return time_launches(dev, lambda: tensor.matmul_device(out.ptr, x.ptr, n), reps)


def roofline_leg(dev, fmt, cfg, reps):
    """The dominant kernel of the forward: the fused gate/up/SwiGLU product
    (the MLP's first launch, N = 2 x 14336 rows over K = 4096) on the
    forward's 8192 tokens, its input fragments split once before the timed
    region and its output written as the down projection's fragments,
    exactly as the forward launches it."""
    import torch
    from ditch_amd import hipmem, synth
    gen = torch.Generator().manual_seed(7)
    q = synth.QUANTIZERS[fmt]
    n, ff, h = cfg["prompts"] * cfg["tokens"], cfg["inter"], cfg["hidden"]
    gate = dev.upload(q(torch.randn(ff, h, generator=gen) * 0.02))
    up = dev.upload(q(torch.randn(ff, h, generator=gen) * 0.02))
    x = hipmem.Buffer.from_array(np.random.default_rng(3).standard_normal((n, h)).astype(np.float32))
    fb, ob = gate.frag_bytes(n), gate.glu_frag_bytes(up, n)
    assert fb and ob, "the fused product does not take the FFN shape"
    xs, act = hipmem.Buffer(fb), hipmem.Buffer(ob)
    gate.split_device(xs.ptr, fb, x.ptr, n)
    ms = time_launches(dev, lambda: gate.glu_device(up, act.ptr, ob, xs.ptr, fb, n), reps)
    gate.free()
    up.free()
    flops = 2.0 * n * (2 * ff) * h
    achieved = flops / (ms * 1e-3) / 1e12
    common = {"bound": "mfma", "achieved": round(achieved, 2), "unit": "TFLOP/s",
              "traffic": traffic_for(f"glu_{fmt}"), "avg_launch_ms": round(ms, 4),
              "algorithmic_flops_per_launch": flops,
              "per_unit": "2 flops per weight element per token (x 2 matrices: gate and up)"}
    if fmt == "mxfp4":
        # fp6 (activation terms) x fp4 (codes) scaled MFMA: the published
        # fp6/fp4 dense peak; the four terms make the MFMA work four times
        # the algorithmic flops, so the split's own ceiling is peak / 4
        return {**common, "peak": FP6_FP4_PEAK_TFLOPS, "frac": round(achieved / FP6_FP4_PEAK_TFLOPS, 4),
                "kernel": f"mx_gemm_kernel<GLU> (v_mfma_scale_f32_16x16x128_f8f6f4, fp6 x fp4) "
                          f"{n}x(2x{ff})x{h}",
                "mfma_flops_per_algorithmic_flop": MX_TERMS,
                "frac_of_fp8_peak": round(achieved / FP8_PEAK_TFLOPS, 4),
                "frac_of_split_ceiling": round(achieved / (FP6_FP4_PEAK_TFLOPS / MX_TERMS), 4)}
    return {**common, "peak": BF16_PEAK_TFLOPS, "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
            "kernel": f"tile_gemm_kernel<{fmt}, GLU> (bf16 MFMA, two bf16 activation terms) {n}x(2x{ff})x{h}",
            "mfma_flops_per_algorithmic_flop": BF16_TERMS,
            "frac_of_fp8_peak": round(achieved / FP8_PEAK_TFLOPS, 4),
            "frac_of_split_ceiling": round(achieved / (BF16_PEAK_TFLOPS / BF16_TERMS), 4)}


def forward_leg(dev, fmt, cfg, steps, warmup):
    from ditch_amd.hip import Model
    t0 = time.time()
    spec = build_spec(fmt, cfg)
    log(f"synthetic c3_{fmt} spec in {time.time() - t0:.1f}s; uploading")
    t0 = time.time()
    model = Model(dev, spec)
    log(f"uploaded {model.nbytes / 1e9:.2f} GB in {time.time() - t0:.1f}s")
    r = time_forward(dev, model, cfg, steps, warmup)
    model.free()
    r["spec"] = spec
    r["tokens_per_s"] = cfg["prompts"] * cfg["tokens"] / (r["ms"] * 1e-3)
    log(f"c3_{fmt} forward: {r['ms']:.2f} ms/step, {r['tokens_per_s']:.0f} tokens/s "
        f"(wall {r['wall']:.2f}s for {steps} steps)")
    return r


def gemm_leg(dev, fmt, cfg, reps):
    """The forward's plain large-batch product at the FFN gate shape (N =
    14336 rows over K = 4096) on the forward's 8192 tokens, its input
    fragments split once before the timed region (ditch_hip_split_device),
    then ditch_hip_matmulT_frags_device: the launch the q, o and down
    projections make."""
    import torch
    from ditch_amd import hipmem, synth
    gen = torch.Generator().manual_seed(7)
    n, ff, h = cfg["prompts"] * cfg["tokens"], cfg["inter"], cfg["hidden"]
    w = dev.upload(synth.QUANTIZERS[fmt](torch.randn(ff, h, generator=gen) * 0.02))
    x = hipmem.Buffer.from_array(np.random.default_rng(3).standard_normal((n, h)).astype(np.float32))
    fb = w.frag_bytes(n)
    assert fb, "the large-batch product does not take the FFN shape"
    xs, out = hipmem.Buffer(fb), hipmem.Buffer(n * ff * 4)
    w.split_device(xs.ptr, fb, x.ptr, n)
    ms = time_launches(dev, lambda: w.matmul_frags_device(out.ptr, xs.ptr, n, frag_bytes=fb), reps)
    w.free()
    flops = 2.0 * n * ff * h
    achieved = flops / (ms * 1e-3) / 1e12
    peak = FP6_FP4_PEAK_TFLOPS if fmt == "mxfp4" else BF16_PEAK_TFLOPS
    return {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4), "traffic": traffic_for(f"gemm_{fmt}"), "avg_launch_ms": round(ms, 4),
            "algorithmic_flops_per_launch": flops, "kernel": f"large-batch {fmt} product {n}x{ff}x{h}"}


def gemv_leg(dev, reps):
    """Q8_0 14336 x 4096 times [M, 4096] activations."""
    import torch
    from ditch_amd import synth
    gen = torch.Generator().manual_seed(11)
    N, K = 14336, 4096
    w = synth.q8_0_random(N, K, gen)
    t = dev.upload(w)
    out = []
    wbytes = N * (K // 32) * 34
    for m in (1, 4, 16, 64, 256):
        ms = time_matmul(dev, t, m, K, reps)
        # algorithmic bytes: packed weight + bf16 activations + f32 outputs
        nbytes = wbytes + m * K * 2 + m * N * 4
        gbs = nbytes / (ms * 1e-3) / 1e9
        out.append({"M": m, "avg_launch_us": round(ms * 1e3, 2), "GB_s": round(gbs, 1),
                    "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": nbytes,
                    "TFLOP_s": round(2.0 * m * N * K / (ms * 1e-3) / 1e12, 3)})
    t.free()
    return out


def c1_leg(dev, steps, warmup, cpu=True, trial=True):
    from ditch_amd.hip import Model
    spec = c1_spec()
    model = Model(dev, spec)
    r = time_forward(dev, model, C1, steps, warmup)
    tr = trial_leg(dev, model, spec) if trial else None
    model.free()
    n = C1["prompts"] * C1["tokens"]
    out = {"workload": "c1: Qwen2.5-0.5B-shaped, 24 layers, d 896, FFN 4864, GQA 14/2 x 64, vocab 151936, f32 "
                       "weights N(0,0.02), q/k/v bias, tied embedding; 16 prompts x 64 tokens",
           "ms_per_step": round(r["ms"], 3), "tokens_per_s": round(n / (r["ms"] * 1e-3), 1),
           "outputs_finite": bool(np.isfinite(r["logprobs"]).all() and np.isfinite(r["res"]).all()),
           "trial": tr}
    if cpu:
        out["cpu_baseline"], out["parity_vs_cpu_sample"] = cpu_leg(spec, C1, r, prompts=4)
    return out


def trial_leg(dev, model, spec):
    """The other timed parts of a search trial the reference publishes for
    this model shape (tools/real-model-validation.md:56-66, Qwen2.5-0.5B),
    on the C1 model: the residual-mean pass over 400 prompts
    (engine.zig:314-438: forward with every layer entry's last-token
    residual, the window mean and the f64 sums per entry; batches of 16
    prompts of 32 tokens), greedy decode of 16 prompts x 32 tokens
    (generateKeep, model.zig:5378-5444; prefill included), and the apply of
    the none / pre / full edits of every layer's o_proj and down_proj with
    one direction (abliterate.zig:148-210; full: lora rank 3)."""
    from ditch_amd import abi, hipmem
    c = C1
    L, H, V = c["layers"], c["hidden"], c["vocab"]
    rng = np.random.default_rng(77)
    # residual-mean pass
    B, T, NP = 16, 32, 400
    E = L + 1
    bres = hipmem.Buffer(E * B * H * 4)
    blog = hipmem.Buffer(B * V * 4)
    bsum = hipmem.Buffer(E * H * 8)
    bsum.zero()
    bvout = hipmem.Buffer(B * E * H * 4)
    bmean = hipmem.Buffer(E * H * 4)
    rows = np.array([(b, p) for b in range(B) for p in range(T)], dtype=np.uint32)
    last = np.array([b * T + T - 1 for b in range(B)], dtype=np.uint64)
    first = np.arange(B, dtype=np.uint32)
    take = np.ones(B, dtype=np.uint32)
    br, bl = hipmem.Buffer.from_array(rows), hipmem.Buffer.from_array(last)
    bf, btk = hipmem.Buffer.from_array(first), hipmem.Buffer.from_array(take)
    batches = [hipmem.Buffer.from_array(rng.integers(0, V, B * T).astype(np.uint32)) for _ in range(NP // B)]
    dev.sync()
    e0, e1 = hipmem.Event(), hipmem.Event()
    t0 = time.perf_counter()
    e0.record(dev.stream)
    for bt in batches:
        model.forward_device(bt.ptr, br.ptr, B * T, B, T, bl.ptr, B, bres.ptr, bl.ptr, B, blog.ptr)
        dev.check(dev.lib.ditch_hip_residual_reduce_device(dev.h, bres.ptr, E, B, H, bf.ptr, btk.ptr, B, -1.0,
                                                           bvout.ptr, bsum.ptr, None, None))
    dev.check(dev.lib.ditch_hip_residual_mean_device(dev.h, bmean.ptr, bsum.ptr, NP, E * H, None))
    e1.record(dev.stream)
    e1.synchronize()
    mean_pass_s = time.perf_counter() - t0
    mean_pass_gpu_s = e0.elapsed_ms(e1) / 1e3
    means = bmean.download(np.float32, (E, H))
    # decode
    prompts = [list(rng.integers(0, V, T)) for _ in range(B)]
    cache = model.kv_cache(B, 2 * T + 8)
    try:
        model.generate(cache, prompts, 4)  # warm-up
        dev.sync()
        t0 = time.perf_counter()
        outs, _ = model.generate(cache, prompts, T)
        gen_s = time.perf_counter() - t0
    finally:
        model.kv_cache_free(cache)
    new_tokens = sum(len(o) for o in outs)
    # apply: every layer's o_proj and down_proj, one direction per layer
    dirs = []
    for li in range(L):
        v = rng.standard_normal(H)
        dirs.append(np.ascontiguousarray((v / np.linalg.norm(v))[None, :], dtype=np.float32))
    targets = []
    for li in range(L):
        targets.append((li, abi.SLOT["O"], -1, dirs[li], 1.0))
        targets.append((li, abi.SLOT["DOWN"], -1, dirs[li], 1.0))
    apply_ms = {}
    prepared = model.edit_targets(targets, 1)
    for mode in ("none", "pre", "full"):
        runs = []
        for rep in range(3):
            model.reset_deltas()
            dev.sync()
            t0 = time.perf_counter()
            if mode == "none":
                model.edit_batch(prepared)
            else:
                for li, slot, e, v, wt in targets:
                    model.edit_ex(li, slot, e, v, wt, mode=mode, lora_rank=3, seed=li)
            dev.sync()
            runs.append((time.perf_counter() - t0) * 1e3)
        apply_ms[mode] = round(float(np.median(runs)), 3)
    model.reset_deltas()
    return {"workload": "c1 model (Qwen2.5-0.5B shape, f32 weights): the reference's per-trial timings "
                        "(tools/real-model-validation.md:56-66: 4 vCPU, bf16 weights)",
            "residual_mean_pass_s": round(mean_pass_s, 3), "residual_mean_pass_gpu_s": round(mean_pass_gpu_s, 3),
            "residual_mean_pass_prompts": NP, "residual_mean_pass_tokens_per_prompt": T,
            "residual_means_finite": bool(np.isfinite(means).all()),
            "decode_tokens_per_s": round(new_tokens / gen_s, 1), "decode_prompts": B, "decode_new_tokens": T,
            "decode_s_incl_prefill": round(gen_s, 4),
            "apply_ms": apply_ms, "apply_matrices": len(targets),
            "reference_cpu": {"residual_mean_pass_s": 36.55, "decode_tokens_per_s": 143.1,
                              "apply_ms": {"none": 8.7, "pre": 16.1, "full": 293.8},
                              "source": "tools/real-model-validation.md:63-65 (4 threads, bf16 Qwen2.5-0.5B)"}}


def c4_cpu_leg(spec, cfg, fwd, layers_run=4):
    """The oracle on configs[3]'s first prompt (128 tokens) through the first
    `layers_run` layers (every layer has the same shapes; the experts kept
    packed and decoded per use, the reference's streamed mode), scaled to
    the full depth: tokens/s of the 48-layer forward on this host's cores."""
    from oracle import ref as oref
    cores = cpu_share()
    tokens, rows, last = fwd["batch"]
    T, L = cfg["tokens"], cfg["layers"]
    with tempfile.TemporaryDirectory() as d:
        so = os.path.join(d, "libcpu_ref_native.so")
        try:
            oref.build(so, arch="native")
        except Exception:
            so = oref.LIB
        m = oref.RefModel(spec, path=so, threads=cores, keep_packed=True)
        m.limit_layers(0, layers_run)
        t0 = time.perf_counter()
        m.forward(tokens[:T], [tuple(x) for x in rows[:T]], capture_rows=last[:1], logit_rows=last[:1])
        secs = time.perf_counter() - t0
        m.free()
    full = secs * L / layers_run
    return {"value": round(T / full, 3), "unit": "tokens/s", "cores": cores, "kind": "port", "cpu_model": cpu_model(),
            "sample": (f"oracle/cpu_ref.c -O3 -march=native, {cores} threads: 1 prompt x {T} tokens through the "
                       f"first {layers_run} of {L} layers with lm_head ({secs:.1f}s), scaled to {L} layers; "
                       "INT4 experts decoded per use"),
            "cpu_seconds": round(secs, 2)}


def c5_cpu_leg(layers_run=4):
    """The oracle on configs[4]'s first prompt (256 tokens) through its first
    `layers_run` layers (the 3 dense layers and the first routed one; FP8
    experts kept packed and decoded per use, the reference's streamed mode),
    scaled to a step's 16 prompts and 12 layers: tokens/s on this host's
    cores. A prompt is the unit: each one's routed layer decodes the experts
    it uses again (about 8 tokens an expert), so the figure is that of a
    prompt-at-a-time CPU run, not of one batch over all 16."""
    from oracle import ref as oref
    c = C5
    cores = cpu_share()
    spec = c5_spec(layers=layers_run)
    tokens, rows, last = make_batch(dict(prompts=c["prompts"], tokens=c["tokens"], vocab=c["vocab"]))
    T = c["tokens"]
    with tempfile.TemporaryDirectory() as d:
        so = os.path.join(d, "libcpu_ref_native.so")
        try:
            oref.build(so, arch="native")
        except Exception:
            so = oref.LIB
        m = oref.RefModel(spec, path=so, threads=cores, keep_packed=True)
        dense = c["dense_layers"]
        times = []
        for hi in (dense, layers_run):  # the dense layers alone, then with the routed one
            m.limit_layers(0, hi)
            t0 = time.perf_counter()
            m.forward(tokens[:T], [tuple(x) for x in rows[:T]], capture_rows=[T - 1], logit_rows=[T - 1])
            times.append(time.perf_counter() - t0)
        m.free()
    t_dense, t_all = times
    routed = (t_all - t_dense) / (layers_run - dense)  # one routed layer of one prompt
    full = c["prompts"] * (t_dense + routed * (c["layers"] - dense))
    return {"value": round(c["prompts"] * T / full, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": (f"oracle/cpu_ref.c -O3 -march=native, {cores} threads: 1 prompt x {T} tokens through its "
                       f"{dense} dense layers ({t_dense:.1f}s) and through those and the first routed layer "
                       f"({t_all:.1f}s), both with lm_head; the routed layer's time taken for each of the "
                       f"{c['layers'] - dense}, scaled to {c['prompts']} prompts; FP8 experts decoded per use, "
                       "again for each prompt"),
            "cpu_seconds": round(t_dense + t_all, 2)}


def c2_cpu_leg(reps_s=2.0):
    """The oracle's dequant-fused matmulT (tensor.zig:827-913 restated) on
    configs[1]'s Q8_0 14336 x 4096 weight for each M, on this host's cores."""
    import torch
    from ditch_amd import synth
    from oracle import ref as oref
    cores = cpu_share()
    rng = np.random.default_rng(3)
    N, K = 14336, 4096
    w = synth.q8_0_random(N, K, torch.Generator().manual_seed(11))
    wbytes = N * (K // 32) * 34
    out = []
    with tempfile.TemporaryDirectory() as d:
        so = os.path.join(d, "libcpu_ref_native.so")
        try:
            oref.build(so, arch="native")
        except Exception:
            so = oref.LIB
        r = oref.Ref(path=so, threads=cores)
        for m in (1, 4, 16, 64, 256):
            x = rng.standard_normal((m, K)).astype(np.float32)
            r.matmulT(x, w)
            n, t0 = 0, time.perf_counter()
            while True:
                r.matmulT(x, w)
                n += 1
                el = time.perf_counter() - t0
                if n >= 3 and el >= reps_s / 5:
                    break
            ms = el / n * 1e3
            nbytes = wbytes + m * K * 2 + m * N * 4
            out.append({"M": m, "ms": round(ms, 3), "GB_s": round(nbytes / (ms * 1e-3) / 1e9, 2),
                        "GFLOP_s": round(2.0 * m * N * K / (ms * 1e-3) / 1e9, 1)})
    return {"cores": cores, "kind": "port", "cpu_model": cpu_model(),
            "sample": f"oracle ref_matmulT, Q8_0 {N}x{K}, {cores} threads, at least 3 calls per M", "per_M": out}


def c4_leg(dev, steps, warmup, layers=48, cpu=True):
    """configs[3] at full depth: the forward, the rank-2 none-mode edit of
    every o_proj and every expert's down_proj (abliterate.zig:148-210,
    264-280; R = QR of a 2048 x 2 Gaussian, lambda 1) made by one batch
    call and timed as one apply, then the edited forward."""
    from ditch_amd import abi
    from ditch_amd.hip import Model
    c = dict(C4, layers=layers)
    t0 = time.time()
    spec = c4_spec(layers)
    log(f"c4 spec in {time.time() - t0:.1f}s")
    t0 = time.time()
    model = Model(dev, spec)
    log(f"c4 uploaded {model.nbytes / 1e9:.2f} GB in {time.time() - t0:.1f}s")
    base = time_forward(dev, model, c, steps, warmup)
    stats0 = model.path_stats()
    rng = np.random.default_rng(14)
    v, _ = np.linalg.qr(rng.standard_normal((c["hidden"], 2)))
    v = np.ascontiguousarray(v.T, dtype=np.float32)
    targets = []
    for li in range(layers):
        targets.append((li, abi.SLOT["O"], -1, v, 1.0))
        targets += [(li, abi.SLOT["EXPERT_DOWN"], e, v, 1.0) for e in range(c["experts"])]
    # one ditch_hip_model_edit_batch call per apply (abliterate.apply), the
    # target array built beforehand (the caller's list of matrices); the
    # first apply pays the allocator's growth, the rest are timed
    prepared = model.edit_targets(targets, 2)
    applies = []
    for rep in range(4):
        dev.sync()
        t0 = time.perf_counter()
        model.edit_batch(prepared)
        dev.sync()
        applies.append(time.perf_counter() - t0)
    apply_s = float(np.median(applies[1:]))
    # algorithmic bytes of one apply: the INT4 codes, f16 scales and 4-bit
    # zero points of every edited matrix (read once), plus its delta
    def int4_bytes(rows, cols):
        groups = cols // 128
        return rows * cols // 2 + rows * groups * 2 + rows * groups // 2 + 2 * 4 * (rows + cols)
    apply_bytes = layers * (int4_bytes(c["hidden"], c["heads"] * c["head_dim"]) +
                            c["experts"] * int4_bytes(c["hidden"], c["moe_inter"]))
    stats1 = model.path_stats()
    edited = time_forward(dev, model, c, steps, warmup, batch=base["batch"])
    stats2 = model.path_stats()
    model.free()
    cpu_b = c4_cpu_leg(spec, c, base) if cpu else None
    n = c["prompts"] * c["tokens"]
    flops = 2.0 * n * c["top_k"] * 3 * c["hidden"] * c["moe_inter"] * layers
    return {"workload": f"c4: Qwen3-30B-A3B-shaped MoE, {layers} layers, d 2048, 128 experts top-8 of FFN 768, "
                        "INT4 g128 asymmetric, vocab 151936; 32 prompts x 128 tokens",
            "ms_per_step": round(base["ms"], 3), "tokens_per_s": round(n / (base["ms"] * 1e-3), 1),
            "routed_expert_tflops_over_step": round(flops / (base["ms"] * 1e-3) / 1e12, 2),
            "edit_apply_ms": round(apply_s * 1e3, 3),
            "edit_apply_ms_runs": [round(a * 1e3, 3) for a in applies],
            "edit_matrices": len(targets),
            "edit_apply_bytes": int(apply_bytes),
            "edit_apply_GB_s": round(apply_bytes / apply_s / 1e9, 1),
            "edited_ms_per_step": round(edited["ms"], 3),
            "edited_tokens_per_s": round(n / (edited["ms"] * 1e-3), 1),
            "edited_over_unedited": round(edited["ms"] / base["ms"], 4),
            "moe_layers_device_planned_unedited": stats0["moe_device_planned"],
            "moe_layers_device_planned_edited": stats2["moe_device_planned"] - stats1["moe_device_planned"],
            "moe_layers_host_planned_edited": stats2["moe_host_planned"] - stats1["moe_host_planned"],
            "edit_changed_logits": bool(np.abs(edited["logits"] - base["logits"]).max() > 1e-4),
            "cpu_baseline": cpu_b,
            "outputs_finite": bool(np.isfinite(base["logprobs"]).all() and np.isfinite(edited["logprobs"]).all())}


def c5_leg(dev, steps, warmup):
    """12 layers with the routed experts streamed from pinned
    host memory through a 96 GB HBM cache (fewer bytes than the 101.5 GB of
    routed experts, so every forward copies some experts back in)."""
    from ditch_amd.hip import Model
    c = C5
    t0 = time.time()
    spec = c5_spec()
    log(f"c5 spec in {time.time() - t0:.1f}s")
    t0 = time.time()
    model = Model(dev, spec, expert_cache_bytes=c["cache_bytes"])
    up_s = time.time() - t0
    log(f"c5 registered in {up_s:.1f}s (experts to host memory: pinned up to the library's limit, then pageable)")
    cfg = dict(layers=c["layers"], hidden=c["hidden"], vocab=c["vocab"], prompts=c["prompts"], tokens=c["tokens"])
    s0 = model.expert_cache_stats()
    first = time_forward(dev, model, cfg, 1, 0)
    s1 = model.expert_cache_stats()
    r = time_forward(dev, model, cfg, steps, warmup, batch=first["batch"])
    s2 = model.expert_cache_stats()
    model.free()
    n = c["prompts"] * c["tokens"]
    per_step = (s2["bytes_read"] - s1["bytes_read"]) / max(steps + warmup, 1)
    return {"workload": "c5: DeepSeek-V3-shaped first 12 layers (3 dense + 9 MoE), d 7168, MLA 128 heads, 256 routed "
                        "experts top-8 of FFN 2048 + shared, FP8 128x128; experts streamed from host memory (48 GiB "
                        "pinned, the rest pageable through a pinned staging ring) through a 96 GB HBM cache; "
                        "16 prompts x 256 tokens",
            "ms_per_step": round(r["ms"], 3), "tokens_per_s": round(n / (r["ms"] * 1e-3), 1),
            "first_forward_ms": round(first["ms"], 3),
            "cache": {k: s2[k] for k in ("capacity", "slots", "slot_bytes", "hits", "misses", "prefetched",
                                         "evictions", "bytes_read", "bytes_staged")},
            "host_to_hbm_bytes_per_step": int(per_step),
            "host_to_hbm_GB_s_over_step": round(per_step / (r["ms"] * 1e-3) / 1e9, 2),
            "first_forward_host_to_hbm_GB_s": round((s1["bytes_read"] - s0["bytes_read"]) / (first["ms"] * 1e-3) / 1e9,
                                                    2),
            "register_s": round(up_s, 1),
            "outputs_finite": bool(np.isfinite(r["logprobs"]).all())}


def copy_leg(dev, reps):
    """A plain streaming kernel of known size for calibrating the HBM
    counters: the decode of a 64 MiB bf16 tensor to f32 (reads 64 MiB of
    tiles, writes 128 MiB)."""
    from ditch_amd import hipmem
    from ditch_amd.weights import HostWeight
    rows, cols = 8192, 4096
    w = HostWeight.bf16(np.random.default_rng(5).integers(0, 1 << 15, (rows, cols)).astype(np.uint16))
    t = dev.upload(w)
    out = hipmem.Buffer(rows * cols * 4)  # plain bf16 weights decode to f32
    ms = time_launches(dev, lambda: t.dequant_device(out.ptr, out.nbytes, 0, rows), reps)
    t.free()
    return {"bytes_read": rows * cols * 2, "bytes_written": rows * cols * 4, "avg_launch_us": round(ms * 1e3, 2),
            "GB_s": round(6 * rows * cols / (ms * 1e-3) / 1e9, 1)}


def traffic_for(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE,
    WRITE_SIZE), when the summary has been recorded under profiles/."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(p):
        return None
    return json.load(open(p)).get(name)


# ---------------------------------------------------------------------------
# CPU baseline (oracle, bounded sample)


def cpu_leg(spec, cfg, fwd, prompts=4):
    """The oracle on the first `prompts` prompts of the benchmark batch through
    the whole model (every layer, the final norm, the lm_head and the
    log-softmax): tokens/s of that sample on this host's cores. The GPU's
    residuals, logits and log-probs of the same prompts (prompts are
    independent: each has its own KV slot) are compared with the oracle's."""
    from oracle import ref as oref
    cores = cpu_share()
    tokens, rows, last = fwd["batch"]
    T = cfg["tokens"]
    n = prompts * T
    with tempfile.TemporaryDirectory() as d:
        so = os.path.join(d, "libcpu_ref_native.so")
        try:
            oref.build(so, arch="native")
        except Exception:
            so = oref.LIB
        t0 = time.perf_counter()
        m = oref.RefModel(spec, path=so, threads=cores)
        setup = time.perf_counter() - t0
        r = oref.Ref(path=so, threads=cores)
        t0 = time.perf_counter()
        res, logits = m.forward(tokens[:n], [tuple(x) for x in rows[:n]], capture_rows=last[:prompts],
                                logit_rows=last[:prompts])
        lp = r.log_softmax_rows(logits)
        secs = time.perf_counter() - t0
        m.free()
        kl = r.kl_rows(lp, fwd["logits"][:prompts])
    g_res = fwd["res"][:, :prompts, :]
    rel_res = float((np.abs(g_res - res).max(axis=-1) / np.abs(res).max(axis=-1)).max())
    rel_log = float(np.abs(fwd["logits"][:prompts] - logits).max() / np.abs(logits).max())
    lp_err = float(np.abs(fwd["logprobs"][:prompts] - lp).max())
    return {"value": round(n / secs, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": (f"oracle/cpu_ref.c -O3 -march=native, {cores} threads (the GPU box's CPU share): the first "
                       f"{prompts} of the {cfg['prompts']} benchmark prompts x {T} tokens through all "
                       f"{cfg['layers']} layers, final norm, lm_head and log-softmax ({secs:.1f}s; model set-up "
                       f"{setup:.1f}s not counted)"),
            "cpu_seconds": round(secs, 2)}, {
        "sample_prompts": prompts, "residual_max_rel_err": rel_res, "logits_max_err_over_max_logit": rel_log,
        "logprob_max_abs_err": lp_err, "kl_cpu_gpu_max": float(kl.max())}


# ---------------------------------------------------------------------------


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="c3_mxfp4", choices=["c3_mxfp4", "c3_fp8"])
    ap.add_argument("--layers", type=int, default=None, help="override the C3 layer count (quick runs)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemv", action="store_true")
    ap.add_argument("--no-other", action="store_true", help="skip the second C3 format")
    ap.add_argument("--no-c1", action="store_true")
    ap.add_argument("--no-c4", action="store_true")
    ap.add_argument("--c4-layers", type=int, default=48)
    ap.add_argument("--c5-cpu", action="store_true", help="with --kernel-only c5: also time the oracle on a C5 "
                    "sample (one prompt through the dense layers, then with the first routed layer)")
    ap.add_argument("--no-c5", action="store_true", help="skip configs[4] (it pins ~48 GB and holds ~100 GB of "
                                                         "host memory)")
    ap.add_argument("--no-trial", action="store_true", help="skip the decode / residual-mean / apply timings")
    ap.add_argument("--kernel-only", choices=["glu", "gemm", "gemv", "copy", "c1", "c4", "c5"], default=None,
                    help="run only one leg (for rocprofv3 runs)")
    ap.add_argument("--reps", type=int, default=20)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: --gpus {args.gpus} is not supported (the prompt forward would shard "
              f"data-parallel over prompts, one model copy per GPU; nothing of that is built)", file=sys.stderr)
        sys.exit(2)

    from ditch_amd.hip import Device
    fmt = {"c3_mxfp4": "mxfp4", "c3_fp8": "fp8"}[args.workload]
    other = "fp8" if fmt == "mxfp4" else "mxfp4"
    cfg = dict(C3)
    if args.layers:
        cfg["layers"] = args.layers
    dev = Device(0)
    log(f"device: {dev.name}")

    if args.kernel_only == "glu":
        print(json.dumps({"kernel_only": "glu", "roofline": roofline_leg(dev, fmt, cfg, args.reps)}))
        return
    if args.kernel_only == "gemm":
        print(json.dumps({"kernel_only": "gemm", "roofline": gemm_leg(dev, fmt, cfg, args.reps)}))
        return
    if args.kernel_only == "gemv":
        print(json.dumps({"kernel_only": "gemv", "gemv": gemv_leg(dev, args.reps)}))
        return
    if args.kernel_only == "copy":
        print(json.dumps({"kernel_only": "copy", "copy": copy_leg(dev, args.reps)}))
        return
    if args.kernel_only == "c1":
        print(json.dumps({"kernel_only": "c1", "c1": c1_leg(dev, args.steps, args.warmup)}))
        return
    if args.kernel_only == "c4":
        print(json.dumps({"kernel_only": "c4", "c4": c4_leg(dev, args.steps, args.warmup, args.c4_layers)}))
        return
    if args.kernel_only == "c5":
        c5 = c5_leg(dev, args.steps, args.warmup)
        if args.c5_cpu:
            c5["cpu_baseline"] = c5_cpu_leg()
        print(json.dumps({"kernel_only": "c5", "c5": c5}))
        return

    head = forward_leg(dev, fmt, cfg, args.steps, args.warmup)
    value = head["tokens_per_s"]
    finite = bool(np.isfinite(head["logprobs"]).all() and np.isfinite(head["res"]).all())
    second = None
    if not args.no_other:
        o = forward_leg(dev, other, cfg, args.steps, args.warmup)
        second = {"workload": f"c3_{other}: the same forward with {other} linear weights",
                  "ms_per_step": round(o["ms"], 3), "tokens_per_s": round(o["tokens_per_s"], 1),
                  "outputs_finite": bool(np.isfinite(o["logprobs"]).all())}
        del o
    roof = roofline_leg(dev, fmt, cfg, args.reps)
    log(f"roofline: {roof['achieved']} TFLOP/s ({roof['frac'] * 100:.1f}% of the {roof['peak']:.0f} TFLOP/s peak)")
    roof_other = None if args.no_other else roofline_leg(dev, other, cfg, args.reps)
    gemv = None if args.no_gemv else gemv_leg(dev, args.reps)
    if gemv:
        for g in gemv:
            log(f"gemv M={g['M']}: {g['avg_launch_us']} us, {g['GB_s']} GB/s ({g['frac_hbm_peak'] * 100:.1f}%)")
    c2_cpu = None if (args.no_gemv or args.no_cpu) else c2_cpu_leg()
    if gemv and c2_cpu:
        for g, cg in zip(gemv, c2_cpu["per_M"]):
            g["cpu_ms"] = cg["ms"]
            g["cpu_GB_s"] = cg["GB_s"]
    c1 = None if args.no_c1 else c1_leg(dev, args.steps, args.warmup, cpu=not args.no_cpu, trial=not args.no_trial)
    if c1:
        log(f"c1: {c1['ms_per_step']} ms/step, {c1['tokens_per_s']} tokens/s; trial {c1['trial']}")
    c4 = None if args.no_c4 else c4_leg(dev, args.steps, args.warmup, args.c4_layers, cpu=not args.no_cpu)
    if c4:
        log(f"c4: {c4['ms_per_step']} ms/step ({c4['tokens_per_s']} tokens/s), edit apply {c4['edit_apply_ms']} ms "
            f"({c4['edit_apply_GB_s']} GB/s), edited {c4['edited_ms_per_step']} ms/step")
    c5 = None
    if not args.no_c5:
        avail = host_mem_available()
        if avail is not None and avail < C5_HOST_BYTES:
            c5 = {"skipped": f"host memory: {avail / 1e9:.0f} GB available, the C5 leg holds about "
                             f"{C5_HOST_BYTES / 1e9:.0f} GB of expert blobs"}
        else:
            c5 = c5_leg(dev, args.steps, args.warmup)
            log(f"c5: {c5['ms_per_step']} ms/step ({c5['tokens_per_s']} tokens/s), host->HBM "
                f"{c5['host_to_hbm_GB_s_over_step']} GB/s over the step")
            if not args.no_cpu:
                c5["cpu_baseline"] = c5_cpu_leg()
                log(f"c5 cpu baseline: {c5['cpu_baseline']['value']} tokens/s ({c5['cpu_baseline']['cpu_seconds']}s)")
    cpu, parity = None, None
    if not args.no_cpu:
        t0 = time.time()
        cpu, parity = cpu_leg(head["spec"], cfg, head)
        log(f"cpu baseline: {cpu['value']} tokens/s in {time.time() - t0:.1f}s; parity {parity}")
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp6xfp4" if fmt == "mxfp4" else "bf16",
        "data": "synthetic: N(0,0.02) weights quantised by the build (4 distinct random layers cycled over the "
                "layers, each layer its own HBM copy), uniform random token ids",
        "config": {"workload": f"{args.workload}: Llama-3-8B-shaped, {cfg['layers']} layers, d=4096, ffn=14336, "
                               f"GQA 32/8x128, vocab 128256, {fmt} linear weights, bf16 embedding/lm_head",
                   "prompts": cfg["prompts"], "tokens_per_prompt": cfg["tokens"],
                   "tokens_per_step": cfg["prompts"] * cfg["tokens"],
                   "step": "forward_device (last-token residual at every layer entry + last-token logits) + "
                           "log-softmax of the logit rows on the device",
                   "arithmetic": ("scaled MFMA: exact MXFP4 codes and E8M0 scales x activations split into four "
                                  "fp6 (e2m3) terms with E8M0 block scales, f32 accumulate; bf16 lm_head; f32 "
                                  "element-wise" if fmt == "mxfp4" else
                                  "bf16 MFMA on exact bf16 weights x activations split into two bf16 terms, "
                                  "f32 accumulate; f32 element-wise"), "outputs_finite": finite,
                   "parity_vs_cpu_sample": parity},
        "roofline": roof,
        "cpu_baseline": cpu,
        f"c3_{other}": second,
        f"roofline_{other}": roof_other,
        "gemv": gemv,
        "gemv_cpu_baseline": c2_cpu,
        "c1": c1,
        "c4": c4,
        "c5": c5,
    }
    print(json.dumps(out))
    dev.close()


if __name__ == "__main__":
    main()
