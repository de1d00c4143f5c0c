"""Benchmark of the MI355X backend on BASELINE.json's headline metric.

Default workload: Llama-3-8B-shaped decoder, 32 layers, d=4096,
FFN 14336, GQA 32/8 x 128, vocab 128256, linear weights MXFP4 (`--workload
c3_fp8` for FP8 E4M3 with 128x128 block scales), bf16 embedding and lm_head;
a step is one resident forward over 64 prompts x 128 random tokens with the
last-token residual captured at every layer entry and last-token logits.
`value` = prompt tokens/s with inputs already in HBM.

Beside it, in the same JSON line:
  roofline     - the dominant kernel (the MXFP4 GEMM at the FFN shape of the
                 forward) timed with HIP events on the library's stream;
  gemv         - configs[1]: the Q8_0 14336x4096 dequant-fused product for
                 M in {1, 4, 16, 64, 256}, achieved HBM GB/s vs 8 TB/s;
  moe_c4_layer - configs[3]'s layer shape: one INT4 MoE layer (128 experts
                 top-8) over 32 x 128 tokens, its forward time;
  cpu_baseline - the CPU oracle (oracle/cpu_ref.c, built -march=native on
                 this host) on a bounded sample of the same forward.
Only rank 0 / one GPU: `--gpus N` with N > 1 exits with a message.
"""
import argparse
import ctypes
import json
import os
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "prompt tokens/s (8B MXFP4/FP8 forward) + dequant-GEMV HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP6_FP4_PEAK_TFLOPS = 10100.0  # dense MFMA, fp6 and fp4 operands
MX_TERMS = 4  # fp6 terms per activation on the scaled-MFMA (MXFP4) path

C3 = dict(hidden=4096, inter=14336, layers=32, heads=32, kv_heads=8, head_dim=128, vocab=128256,
          rope_theta=500000.0, rms_eps=1e-5, prompts=64, tokens=128)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# synthetic model


def build_spec(fmt, cfg, layers=None, distinct=4, seed=0):
    """Llama-3-8B-shaped ModelSpec: N(0, 0.02) linear weights quantised to
    `fmt`; norms 1 + N(0, 0.02); bf16 embedding and lm_head. `distinct`
    random layers are generated and cycled over the layers (every layer is
    registered, so each has its own copy in HBM)."""
    import torch
    from ditch_amd import synth
    from ditch_amd.spec import ModelSpec

    torch.set_num_threads(min(16, os.cpu_count() or 1))
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


def make_batch(cfg, seed=1):
    rng = np.random.default_rng(seed)
    P, T = cfg["prompts"], cfg["tokens"]
    tokens = rng.integers(0, cfg["vocab"], P * T).astype(np.uint32)
    rows = np.array([(b, p) for b in range(P) for p in range(T)], dtype=np.uint32)
    last = np.array([b * T + T - 1 for b in range(P)], dtype=np.uint64)
    return tokens, rows, last


# ---------------------------------------------------------------------------
# GPU legs


def time_forward(dev, model, cfg, steps, warmup):
    from ditch_amd import hipmem
    tokens, rows, last = make_batch(cfg)
    n = tokens.size
    L, hidden, V = cfg["layers"], cfg["hidden"], cfg["vocab"]
    bt, br = hipmem.Buffer.from_array(tokens), hipmem.Buffer.from_array(rows)
    bc, bl = hipmem.Buffer.from_array(last), hipmem.Buffer.from_array(last)
    bres = hipmem.Buffer((L + 1) * last.size * hidden * 4)
    blog = hipmem.Buffer(last.size * V * 4)
    args = (bt.ptr, br.ptr, n, bc.ptr, last.size, bres.ptr, bl.ptr, last.size, blog.ptr)
    for _ in range(warmup):
        model.forward_device(*args)
    dev.sync()
    hipmem.synchronize()
    e0, e1 = hipmem.Event(), hipmem.Event()
    t0 = time.perf_counter()
    e0.record(dev.stream)
    for _ in range(steps):
        model.forward_device(*args)
    e1.record(dev.stream)
    e1.synchronize()
    hipmem.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_ms(e1) / steps
    res = bres.download(np.float32, (L + 1, last.size, hidden))
    logits = blog.download(np.float32, (last.size, V))
    return ms, wall, res, logits, (tokens, rows, last)


def time_matmul(dev, tensor, n, k, reps, frags=False):
    """Average launch time of the tensor's product on n x k activations (events
    on the context stream, which the kernel is launched on). With `frags` the
    activations are split into fragments once, untimed, and only the tiled
    product is launched in the timed region."""
    from ditch_amd import hipmem
    rng = np.random.default_rng(3)
    x = hipmem.Buffer.from_array(rng.standard_normal((n, k)).astype(np.float32))
    out = hipmem.Buffer(n * tensor.rows * 4)
    if frags:
        fb = tensor.frag_bytes(n)
        xs = hipmem.Buffer(fb)
        tensor.split_device(xs.ptr, fb, x.ptr, n)

        def launch():
            tensor.matmul_frags_device(out.ptr, xs.ptr, n)
    else:
        def launch():
            tensor.matmul_device(out.ptr, x.ptr, n)
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


def roofline_leg(dev, fmt, cfg, reps):
    """The dominant kernel of the forward: the quantised GEMM at the FFN gate/up
    shape (N = 14336, K = 4096) on the forward's 8192 tokens."""
    import torch
    from ditch_amd import synth
    gen = torch.Generator().manual_seed(7)
    w = synth.QUANTIZERS[fmt](torch.randn(cfg["inter"], cfg["hidden"], generator=gen) * 0.02)
    t = dev.upload(w)
    n = cfg["prompts"] * cfg["tokens"]
    ms = time_matmul(dev, t, n, cfg["hidden"], reps, frags=True)
    flops = 2.0 * n * cfg["inter"] * cfg["hidden"]
    t.free()
    achieved = flops / (ms * 1e-3) / 1e12
    if fmt == "mxfp4":
        # fp6 (activation terms) x fp4 (codes) scaled MFMA: the published
        # fp6/fp4 dense peak; the four terms make the MFMA work four times
        # the algorithmic flops, so the split's own ceiling is peak / 4
        return {"bound": "mfma", "achieved": round(achieved, 2), "peak": FP6_FP4_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / FP6_FP4_PEAK_TFLOPS, 4), "traffic": traffic_for(f"gemm_{fmt}"),
                "kernel": f"mx_gemm_kernel (v_mfma_scale_f32_16x16x128_f8f6f4, fp6 x fp4) {n}x{cfg['inter']}x{cfg['hidden']}",
                "avg_launch_ms": round(ms, 4), "algorithmic_flops_per_launch": flops,
                "mfma_flops_per_algorithmic_flop": MX_TERMS,
                "frac_of_split_ceiling": round(achieved / (FP6_FP4_PEAK_TFLOPS / MX_TERMS), 4)}
    return {"bound": "mfma", "achieved": round(achieved, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / BF16_PEAK_TFLOPS, 4), "traffic": traffic_for(f"gemm_{fmt}"),
            "kernel": f"tile_gemm_kernel<{fmt}> (bf16 MFMA, two bf16 activation terms) {n}x{cfg['inter']}x{cfg['hidden']}",
            "avg_launch_ms": round(ms, 4), "algorithmic_flops_per_launch": flops, "mfma_flops_per_algorithmic_flop": 2}


C4 = dict(hidden=2048, heads=32, kv_heads=4, head_dim=128, experts=128, top_k=8, moe_inter=768, vocab=8192,
          prompts=32, tokens=128)


def moe_leg(dev, steps=5, warmup=2):
    """configs[3]'s layer: one Qwen3-30B-A3B-shaped MoE layer (d 2048, 32/4
    heads of 128, 128 experts top-8 of FFN 768, INT4 group 128 drawn in the
    packed domain, reduced vocab) over 32 prompts x 128 tokens. Reported
    beside the headline: the forward's time and the routed-expert products'
    algorithmic throughput over it (a lower bound for those kernels)."""
    import torch
    from ditch_amd import abi, synth
    from ditch_amd.hip import Model
    from ditch_amd.spec import ModelSpec
    c = C4
    rng = np.random.default_rng(21)
    h, nh, nkv, hd, E, mi, V = (c["hidden"], c["heads"], c["kv_heads"], c["head_dim"], c["experts"], c["moe_inter"],
                                c["vocab"])
    spec = ModelSpec(hidden=h, inter=4 * h, layers=1, heads=nh, kv_heads=nkv, head_dim=hd, vocab=V, rms_eps=1e-6,
                     qk_norm=1, tie_embeddings=0, rope_theta=1e6, rope_len=512, n_experts=E, top_k=c["top_k"],
                     moe_inter=mi, norm_topk_prob=1, scoring=abi.SCORING_SOFTMAX, moe_layers=[1])
    spec.set("EMBED", synth.bf16_weight(torch.from_numpy(rng.normal(0, 0.02, (V, h)).astype(np.float32))))
    spec.set("LM_HEAD", synth.int4_random(V, h, rng))
    spec.set("FINAL_NORM", 1 + rng.normal(0, 0.02, h))
    spec.set("ATTN_NORM", 1 + rng.normal(0, 0.02, h), 0)
    spec.set("FFN_NORM", 1 + rng.normal(0, 0.02, h), 0)
    for name, r, cc in (("Q", nh * hd, h), ("K", nkv * hd, h), ("V", nkv * hd, h), ("O", h, nh * hd)):
        spec.set(name, synth.int4_random(r, cc, rng), 0)
    spec.set("Q_NORM", 1 + rng.normal(0, 0.02, hd), 0)
    spec.set("K_NORM", 1 + rng.normal(0, 0.02, hd), 0)
    spec.set("ROUTER", synth.bf16_weight(torch.from_numpy(rng.normal(0, 0.02, (E, h)).astype(np.float32))), 0)
    for e in range(E):
        spec.set("EXPERT_GATE", synth.int4_random(mi, h, rng), 0, e)
        spec.set("EXPERT_UP", synth.int4_random(mi, h, rng), 0, e)
        spec.set("EXPERT_DOWN", synth.int4_random(h, mi, rng), 0, e)
    model = Model(dev, spec)
    cfg = dict(layers=1, hidden=h, vocab=V, prompts=c["prompts"], tokens=c["tokens"])
    ms, _, _, logits, _ = time_forward(dev, model, cfg, steps, warmup)
    model.free()
    n = c["prompts"] * c["tokens"]
    flops = 2.0 * n * c["top_k"] * 3 * h * mi
    return {"workload": "c4 layer: Qwen3-30B-A3B-shaped MoE layer (d 2048, 128 experts top-8, FFN 768, INT4 g128), "
                        "32 prompts x 128 tokens, vocab 8192",
            "ms_per_forward": round(ms, 3), "tokens_per_s": round(n / (ms * 1e-3), 1),
            "expert_flops": flops, "expert_tflops_over_forward": round(flops / (ms * 1e-3) / 1e12, 2),
            "outputs_finite": bool(np.isfinite(logits).all())}


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
    e0, e1 = hipmem.Event(), hipmem.Event()
    t.dequant_device(out.ptr, out.nbytes, 0, rows)
    dev.sync()
    e0.record(dev.stream)
    for _ in range(reps):
        t.dequant_device(out.ptr, out.nbytes, 0, rows)
    e1.record(dev.stream)
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / reps
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


def cpu_leg(spec, cfg, batch, gpu_res, prompts=None):
    """The oracle on the benchmark batch (all of its prompts unless `prompts`
    says fewer) through the first one and two layers of the same model (+
    embedding, final norm and lm_head); the per-layer time is extrapolated to
    the full depth (about 10 s of CPU work at the C3 shape on 16 cores). Also
    returns how far the GPU's residuals at those layer entries are from the
    oracle's."""
    from ditch_amd.spec import ModelSpec
    from oracle import ref as oref
    cores = min(16, os.cpu_count() or 1)
    small = ModelSpec(**{k: v for k, v in spec.config.items() if k != "layers"}, layers=2)
    for (layer, slot, expert), w in spec.tensors.items():
        if layer < 2:
            small.tensors[(layer, slot, expert)] = w
    tokens, rows, last = batch
    T = cfg["tokens"]
    prompts = cfg["prompts"] if prompts is None else prompts
    n = prompts * T
    with tempfile.TemporaryDirectory() as d:
        so = os.path.join(d, "libcpu_ref_native.so")
        try:
            oref.build(so, arch="native")
        except Exception:
            so = oref.LIB
        m = oref.RefModel(small, path=so, threads=cores)
        timings = {}
        res = None
        for L in (1, 2):
            m.limit_layers(0, L)
            t0 = time.perf_counter()
            r, _ = m.forward(tokens[:n], [tuple(x) for x in rows[:n]], capture_rows=last[:prompts],
                             logit_rows=last[:prompts])
            timings[L] = time.perf_counter() - t0
            res = r
        m.free()
    per_layer = max(timings[2] - timings[1], 1e-9)
    full = timings[1] + (cfg["layers"] - 1) * per_layer
    tps = prompts * T / full
    # residual entries 0..2 of the sampled prompts, GPU vs oracle
    g = gpu_res[:3, :prompts, :]
    c = res[:3]
    rel = float((np.abs(g - c).max(axis=-1) / np.abs(c).max(axis=-1)).max())
    return {"value": round(tps, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": (f"oracle/cpu_ref.c -O3 -march=native, {cores} threads: {prompts} prompts x {T} tokens of "
                       f"the benchmark batch through 1 and 2 layers of the same model (+ embedding, final norm, "
                       f"lm_head); per-layer {per_layer:.2f}s extrapolated to {cfg['layers']} layers "
                       f"({full:.1f}s for the sample)"),
            "cpu_seconds": round(timings[1] + timings[2], 2)}, rel


# ---------------------------------------------------------------------------


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="c3_mxfp4", choices=["c3_mxfp4", "c3_fp8"])
    ap.add_argument("--layers", type=int, default=None, help="override the layer count (quick runs)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemv", action="store_true")
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--kernel-only", choices=["gemm", "gemv", "copy", "moe"], default=None,
                    help="run only the roofline kernel (for rocprofv3 runs)")
    ap.add_argument("--reps", type=int, default=20)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: --gpus {args.gpus} is not supported (the prompt forward would shard "
              f"data-parallel over prompts, one model copy per GPU; nothing of that is built)", file=sys.stderr)
        sys.exit(2)

    from ditch_amd.hip import Device, Model
    fmt = {"c3_mxfp4": "mxfp4", "c3_fp8": "fp8"}[args.workload]
    cfg = dict(C3)
    if args.layers:
        cfg["layers"] = args.layers
    dev = Device(0)
    log(f"device: {dev.name}")

    if args.kernel_only == "gemm":
        r = roofline_leg(dev, fmt, cfg, args.reps)
        print(json.dumps({"kernel_only": "gemm", "roofline": r}))
        return
    if args.kernel_only == "gemv":
        print(json.dumps({"kernel_only": "gemv", "gemv": gemv_leg(dev, args.reps)}))
        return
    if args.kernel_only == "moe":
        print(json.dumps({"kernel_only": "moe", "moe_c4_layer": moe_leg(dev)}))
        return
    if args.kernel_only == "copy":
        print(json.dumps({"kernel_only": "copy", "copy": copy_leg(dev, args.reps)}))
        return

    t0 = time.time()
    spec = build_spec(fmt, cfg)
    log(f"synthetic {args.workload} spec in {time.time() - t0:.1f}s; uploading")
    t0 = time.time()
    model = Model(dev, spec)
    log(f"uploaded {model.nbytes / 1e9:.2f} GB in {time.time() - t0:.1f}s")
    ms, wall, res, logits, batch = time_forward(dev, model, cfg, args.steps, args.warmup)
    n_tok = cfg["prompts"] * cfg["tokens"]
    value = n_tok / (ms * 1e-3)
    log(f"forward: {ms:.2f} ms/step, {value:.0f} tokens/s (wall {wall:.2f}s for {args.steps} steps)")
    finite = bool(np.isfinite(logits).all() and np.isfinite(res).all())
    model.free()

    roof = roofline_leg(dev, fmt, cfg, args.reps)
    log(f"roofline: {roof['achieved']} TFLOP/s ({roof['frac'] * 100:.1f}% of the {roof['peak']:.0f} TFLOP/s peak)")
    gemv = None if args.no_gemv else gemv_leg(dev, args.reps)
    if gemv:
        for g in gemv:
            log(f"gemv M={g['M']}: {g['avg_launch_us']} us, {g['GB_s']} GB/s ({g['frac_hbm_peak'] * 100:.1f}%)")
    moe = None if args.no_moe else moe_leg(dev)
    if moe:
        log(f"c4 MoE layer: {moe['ms_per_forward']} ms per forward, expert products >= "
            f"{moe['expert_tflops_over_forward']} TFLOP/s")
    cpu, parity = None, None
    if not args.no_cpu:
        t0 = time.time()
        cpu, parity = cpu_leg(spec, cfg, batch, res)
        log(f"cpu baseline: {cpu['value']} tokens/s in {time.time() - t0:.1f}s; residual parity {parity:.2e}")
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp6xfp4" if fmt == "mxfp4" else "bf16",
        "data": "synthetic: N(0,0.02) weights quantised by the build (4 distinct random layers cycled over the "
                "layers, each layer its own HBM copy), uniform random token ids",
        "config": {"workload": f"{args.workload}: Llama-3-8B-shaped, {cfg['layers']} layers, d=4096, ffn=14336, "
                               f"GQA 32/8x128, vocab 128256, {fmt} linear weights, bf16 embedding/lm_head",
                   "prompts": cfg["prompts"], "tokens_per_prompt": cfg["tokens"], "tokens_per_step": n_tok,
                   "outputs": "last-token residual at every layer entry + last-token logits",
                   "arithmetic": ("scaled MFMA: exact MXFP4 codes and E8M0 scales x activations split into four "
                                  "fp6 (e2m3) terms with E8M0 block scales, f32 accumulate; bf16 lm_head; f32 "
                                  "element-wise" if fmt == "mxfp4" else
                                  "bf16 MFMA on exact bf16 weights x activations split into two bf16 terms, "
                                  "f32 accumulate; f32 element-wise"), "outputs_finite": finite,
                   "residual_max_rel_err_vs_cpu_first_2_layers": parity},
        "roofline": roof,
        "cpu_baseline": cpu,
        "gemv": gemv,
        "moe_c4_layer": moe,
    }
    print(json.dumps(out))
    dev.close()


if __name__ == "__main__":
    main()
