"""Seeded synthetic models (ModelSpec) in the benchmark configurations'
families and formats, scaled down for the parity tests."""
import numpy as np
import torch

from ditch_amd import abi, synth
from ditch_amd.spec import ModelSpec


def _q(fmt, rows, cols, gen, std=0.02):
    w = torch.randn(rows, cols, generator=gen) * std
    return synth.QUANTIZERS[fmt](w)


def dense(fmt="bf16", hidden=256, inter=512, layers=2, heads=4, kv_heads=2, head_dim=64, vocab=1000, seed=0,
          qkv_bias=False, qk_norm=False, embed_fmt="bf16", tie=True, rope_theta=1e6):
    gen = torch.Generator().manual_seed(seed)
    spec = ModelSpec(hidden=hidden, inter=inter, layers=layers, heads=heads, kv_heads=kv_heads, head_dim=head_dim,
                     vocab=vocab, rms_eps=1e-6, qkv_bias=int(qkv_bias), qk_norm=int(qk_norm), tie_embeddings=int(tie),
                     rope_theta=rope_theta, rope_len=512)
    spec.set("EMBED", _q(embed_fmt, vocab, hidden, gen))
    if not tie:
        spec.set("LM_HEAD", _q(embed_fmt, vocab, hidden, gen))
    spec.set("FINAL_NORM", 1 + torch.randn(hidden, generator=gen).numpy() * 0.02)
    for li in range(layers):
        spec.set("ATTN_NORM", 1 + torch.randn(hidden, generator=gen).numpy() * 0.02, li)
        spec.set("FFN_NORM", 1 + torch.randn(hidden, generator=gen).numpy() * 0.02, li)
        spec.set("Q", _q(fmt, heads * head_dim, hidden, gen), li)
        spec.set("K", _q(fmt, kv_heads * head_dim, hidden, gen), li)
        spec.set("V", _q(fmt, kv_heads * head_dim, hidden, gen), li)
        spec.set("O", _q(fmt, hidden, heads * head_dim, gen), li)
        if qkv_bias:
            for s, d in (("Q_BIAS", heads * head_dim), ("K_BIAS", kv_heads * head_dim), ("V_BIAS", kv_heads * head_dim)):
                spec.set(s, torch.randn(d, generator=gen).numpy() * 0.02, li)
        if qk_norm:
            spec.set("Q_NORM", 1 + torch.randn(head_dim, generator=gen).numpy() * 0.02, li)
            spec.set("K_NORM", 1 + torch.randn(head_dim, generator=gen).numpy() * 0.02, li)
        spec.set("GATE", _q(fmt, inter, hidden, gen), li)
        spec.set("UP", _q(fmt, inter, hidden, gen), li)
        spec.set("DOWN", _q(fmt, hidden, inter, gen), li)
    return spec


def moe(fmt="int4", hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, vocab=1000, experts=16, top_k=4,
        moe_inter=128, seed=0, sigmoid=False, n_group=1, topk_group=1, shared=0, scaling=1.0, dense_first=0):
    gen = torch.Generator().manual_seed(seed)
    moe_layers = [0] * dense_first + [1] * (layers - dense_first)
    spec = ModelSpec(hidden=hidden, inter=4 * hidden, layers=layers, heads=heads, kv_heads=kv_heads,
                     head_dim=head_dim, vocab=vocab, rms_eps=1e-6, qk_norm=1, tie_embeddings=1, rope_theta=1e6,
                     rope_len=512, n_experts=experts, top_k=top_k, moe_inter=moe_inter, norm_topk_prob=1,
                     scoring=abi.SCORING_SIGMOID if sigmoid else abi.SCORING_SOFTMAX,
                     group_limited=int(n_group > 1), n_group=n_group, topk_group=topk_group,
                     routed_scaling=scaling, shared_inter=shared, moe_layers=moe_layers)
    spec.set("EMBED", _q("bf16", vocab, hidden, gen))
    spec.set("FINAL_NORM", 1 + torch.randn(hidden, generator=gen).numpy() * 0.02)
    for li in range(layers):
        spec.set("ATTN_NORM", 1 + torch.randn(hidden, generator=gen).numpy() * 0.02, li)
        spec.set("FFN_NORM", 1 + torch.randn(hidden, generator=gen).numpy() * 0.02, li)
        for s, r, c in (("Q", heads * head_dim, hidden), ("K", kv_heads * head_dim, hidden),
                        ("V", kv_heads * head_dim, hidden), ("O", hidden, heads * head_dim)):
            spec.set(s, _q(fmt, r, c, gen), li)
        spec.set("Q_NORM", 1 + torch.randn(head_dim, generator=gen).numpy() * 0.02, li)
        spec.set("K_NORM", 1 + torch.randn(head_dim, generator=gen).numpy() * 0.02, li)
        if moe_layers[li]:
            spec.set("ROUTER", synth.f32_weight(torch.randn(experts, hidden, generator=gen) * 0.02), li)
            if sigmoid:
                spec.set("ROUTER_CORRECTION", torch.randn(experts, generator=gen).numpy() * 0.01, li)
            for e in range(experts):
                spec.set("EXPERT_GATE", _q(fmt, moe_inter, hidden, gen), li, e)
                spec.set("EXPERT_UP", _q(fmt, moe_inter, hidden, gen), li, e)
                spec.set("EXPERT_DOWN", _q(fmt, hidden, moe_inter, gen), li, e)
            if shared:
                spec.set("SHARED_GATE", _q(fmt, shared, hidden, gen), li)
                spec.set("SHARED_UP", _q(fmt, shared, hidden, gen), li)
                spec.set("SHARED_DOWN", _q(fmt, hidden, shared, gen), li)
        else:
            spec.set("GATE", _q(fmt, 4 * hidden, hidden, gen), li)
            spec.set("UP", _q(fmt, 4 * hidden, hidden, gen), li)
            spec.set("DOWN", _q(fmt, hidden, 4 * hidden, gen), li)
    return spec


def mla(fmt="fp8", hidden=256, layers=2, heads=4, q_lora=96, kv_lora=64, nope=32, rope=16, v_dim=32, vocab=1000,
        experts=8, top_k=2, moe_inter=64, seed=0):
    gen = torch.Generator().manual_seed(seed)
    hd = nope + rope
    spec = ModelSpec(hidden=hidden, inter=2 * hidden, layers=layers, heads=heads, kv_heads=heads, head_dim=hd,
                     v_head_dim=v_dim, vocab=vocab, rms_eps=1e-6, tie_embeddings=0, rope_theta=10000.0, rope_len=512,
                     rope_style=abi.ROPE_GPTJ, mla=1, q_lora_rank=q_lora, kv_lora_rank=kv_lora, qk_nope_dim=nope,
                     qk_rope_dim=rope, attn_scale=float(np.float32(1) / np.sqrt(np.float32(hd))),
                     n_experts=experts, top_k=top_k, moe_inter=moe_inter, norm_topk_prob=1,
                     scoring=abi.SCORING_SIGMOID, group_limited=1, n_group=2, topk_group=1, routed_scaling=2.5,
                     shared_inter=moe_inter, moe_layers=[0] + [1] * (layers - 1))
    q = lambda r, c: _q(fmt, r, c, gen)
    spec.set("EMBED", _q("bf16", vocab, hidden, gen))
    spec.set("LM_HEAD", _q("bf16", vocab, hidden, gen))
    spec.set("FINAL_NORM", 1 + torch.randn(hidden, generator=gen).numpy() * 0.02)
    for li in range(layers):
        spec.set("ATTN_NORM", 1 + torch.randn(hidden, generator=gen).numpy() * 0.02, li)
        spec.set("FFN_NORM", 1 + torch.randn(hidden, generator=gen).numpy() * 0.02, li)
        spec.set("MLA_Q_A", q(q_lora, hidden), li)
        spec.set("MLA_Q_A_NORM", 1 + torch.randn(q_lora, generator=gen).numpy() * 0.02, li)
        spec.set("MLA_Q_B", q(heads * hd, q_lora), li)
        spec.set("MLA_KV_A", q(kv_lora + rope, hidden), li)
        spec.set("MLA_KV_A_NORM", 1 + torch.randn(kv_lora, generator=gen).numpy() * 0.02, li)
        spec.set("MLA_KV_B", q(heads * (nope + v_dim), kv_lora), li)
        spec.set("O", q(hidden, heads * v_dim), li)
        if li == 0:
            spec.set("GATE", q(2 * hidden, hidden), li)
            spec.set("UP", q(2 * hidden, hidden), li)
            spec.set("DOWN", q(hidden, 2 * hidden), li)
        else:
            spec.set("ROUTER", synth.f32_weight(torch.randn(experts, hidden, generator=gen) * 0.02), li)
            spec.set("ROUTER_CORRECTION", torch.randn(experts, generator=gen).numpy() * 0.01, li)
            for e in range(experts):
                spec.set("EXPERT_GATE", q(moe_inter, hidden), li, e)
                spec.set("EXPERT_UP", q(moe_inter, hidden), li, e)
                spec.set("EXPERT_DOWN", q(hidden, moe_inter), li, e)
            spec.set("SHARED_GATE", q(moe_inter, hidden), li)
            spec.set("SHARED_UP", q(moe_inter, hidden), li)
            spec.set("SHARED_DOWN", q(hidden, moe_inter), li)
    return spec


def moe_c4(layers=2, vocab=8192, seed=0):
    """Config C4's layer shape (Qwen3-30B-A3B: d=2048, 32/4 heads of 128, q/k
    head norm, 128 experts top-8 of FFN 768, softmax router with renorm, INT4
    group-128 asymmetric linear weights, router N(0, 0.02)), a reduced vocab
    and layer count; the INT4 fields are drawn in the packed domain."""
    hidden, heads, kv_heads, head_dim, experts, moe_inter = 2048, 32, 4, 128, 128, 768
    rng = np.random.default_rng(seed)
    spec = ModelSpec(hidden=hidden, inter=4 * hidden, layers=layers, heads=heads, kv_heads=kv_heads,
                     head_dim=head_dim, vocab=vocab, rms_eps=1e-6, qk_norm=1, tie_embeddings=0, rope_theta=1e6,
                     rope_len=512, n_experts=experts, top_k=8, moe_inter=moe_inter, norm_topk_prob=1,
                     scoring=abi.SCORING_SOFTMAX, moe_layers=[1] * layers)
    spec.set("EMBED", synth.bf16_weight(torch.from_numpy(rng.normal(0, 0.02, (vocab, hidden)).astype(np.float32))))
    spec.set("LM_HEAD", synth.int4_random(vocab, hidden, rng))
    spec.set("FINAL_NORM", 1 + rng.normal(0, 0.02, hidden))
    for li in range(layers):
        spec.set("ATTN_NORM", 1 + rng.normal(0, 0.02, hidden), li)
        spec.set("FFN_NORM", 1 + rng.normal(0, 0.02, hidden), li)
        for s_, r, c in (("Q", heads * head_dim, hidden), ("K", kv_heads * head_dim, hidden),
                         ("V", kv_heads * head_dim, hidden), ("O", hidden, heads * head_dim)):
            spec.set(s_, synth.int4_random(r, c, rng), li)
        spec.set("Q_NORM", 1 + rng.normal(0, 0.02, head_dim), li)
        spec.set("K_NORM", 1 + rng.normal(0, 0.02, head_dim), li)
        spec.set("ROUTER", synth.f32_weight(torch.from_numpy(rng.normal(0, 0.02, (experts, hidden)).astype(np.float32))),
                 li)
        for e in range(experts):
            spec.set("EXPERT_GATE", synth.int4_random(moe_inter, hidden, rng), li, e)
            spec.set("EXPERT_UP", synth.int4_random(moe_inter, hidden, rng), li, e)
            spec.set("EXPERT_DOWN", synth.int4_random(hidden, moe_inter, rng), li, e)
    return spec


def mla_c5(experts=64, vocab=8192, seed=0):
    """Config C5's layer shapes (DeepSeek-V3: d=7168, MLA q_lora 1536 /
    kv_lora 512 / nope 128 / rope 64 / v 128 over 128 heads, a dense first
    layer of FFN 18432, then routed experts of FFN 2048, top-8 of 8 groups
    with 4 groups kept, sigmoid router with correction bias 0, scaling 2.5,
    one shared expert; FP8 E4M3 weights with 128 x 128 f32 block scales):
    one dense and one routed layer, `experts` routed experts, a reduced vocab;
    the FP8 codes drawn in the code domain."""
    hidden, heads, q_lora, kv_lora, nope, rope, v_dim, dense_ff, moe_inter = 7168, 128, 1536, 512, 128, 64, 128, 18432, 2048
    rng = np.random.default_rng(seed)
    hd = nope + rope
    spec = ModelSpec(hidden=hidden, inter=dense_ff, layers=2, heads=heads, kv_heads=heads, head_dim=hd,
                     v_head_dim=v_dim, vocab=vocab, rms_eps=1e-6, tie_embeddings=0, rope_theta=10000.0, rope_len=512,
                     rope_style=abi.ROPE_GPTJ, mla=1, q_lora_rank=q_lora, kv_lora_rank=kv_lora, qk_nope_dim=nope,
                     qk_rope_dim=rope, attn_scale=float(np.float32(1) / np.sqrt(np.float32(hd))),
                     n_experts=experts, top_k=8, moe_inter=moe_inter, norm_topk_prob=1,
                     scoring=abi.SCORING_SIGMOID, group_limited=1, n_group=8, topk_group=4, routed_scaling=2.5,
                     shared_inter=moe_inter, moe_layers=[0, 1])
    f8 = lambda r, c: synth.fp8_random(r, c, rng)
    bf = lambda r, c: synth.bf16_weight(torch.from_numpy(rng.normal(0, 0.02, (r, c)).astype(np.float32)))
    spec.set("EMBED", bf(vocab, hidden))
    spec.set("LM_HEAD", bf(vocab, hidden))
    spec.set("FINAL_NORM", 1 + rng.normal(0, 0.02, hidden))
    for li in range(2):
        spec.set("ATTN_NORM", 1 + rng.normal(0, 0.02, hidden), li)
        spec.set("FFN_NORM", 1 + rng.normal(0, 0.02, hidden), li)
        spec.set("MLA_Q_A", f8(q_lora, hidden), li)
        spec.set("MLA_Q_A_NORM", 1 + rng.normal(0, 0.02, q_lora), li)
        spec.set("MLA_Q_B", f8(heads * hd, q_lora), li)
        spec.set("MLA_KV_A", f8(kv_lora + rope, hidden), li)
        spec.set("MLA_KV_A_NORM", 1 + rng.normal(0, 0.02, kv_lora), li)
        spec.set("MLA_KV_B", f8(heads * (nope + v_dim), kv_lora), li)
        spec.set("O", f8(hidden, heads * v_dim), li)
        if li == 0:
            spec.set("GATE", f8(dense_ff, hidden), li)
            spec.set("UP", f8(dense_ff, hidden), li)
            spec.set("DOWN", f8(hidden, dense_ff), li)
        else:
            spec.set("ROUTER", synth.f32_weight(torch.from_numpy(rng.normal(0, 0.02, (experts, hidden)).astype(np.float32))),
                     li)
            spec.set("ROUTER_CORRECTION", np.zeros(experts), li)
            for e in range(experts):
                spec.set("EXPERT_GATE", f8(moe_inter, hidden), li, e)
                spec.set("EXPERT_UP", f8(moe_inter, hidden), li, e)
                spec.set("EXPERT_DOWN", f8(hidden, moe_inter), li, e)
            spec.set("SHARED_GATE", f8(moe_inter, hidden), li)
            spec.set("SHARED_UP", f8(moe_inter, hidden), li)
            spec.set("SHARED_DOWN", f8(hidden, moe_inter), li)
    return spec


def batch(prompts, lens, vocab, seed=0):
    """Flattened prompts (engine.zig:395-410): tokens, rows {b, pos}, the last
    row of each prompt (capture + logits)."""
    rng = np.random.default_rng(seed)
    tokens, rows, last = [], [], []
    for b in range(prompts):
        n = lens[b % len(lens)]
        for p in range(n):
            tokens.append(int(rng.integers(0, vocab)))
            rows.append((b, p))
        last.append(len(tokens) - 1)
    return np.array(tokens, dtype=np.uint32), rows, last
