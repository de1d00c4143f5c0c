"""Readers for the reference's committed test fixtures (tests/golden/fixtures).

The fixtures are small Hugging Face checkpoints (safetensors, config.json) or
GGUF files written by the reference's NumPy generator, with their goldens in
reference.json. This module maps them onto a ModelSpec (the same host
description the device and the oracle take). Only data is read; nothing in a
fixture is executed.
"""
import json
import math
import os
import re
import struct

import numpy as np

from ditch_amd import abi
from ditch_amd.spec import ModelSpec, rope_len_for, yarn_mscale
from ditch_amd.weights import HostWeight, vector

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = os.path.join(GOLDEN, "fixtures")

# ---------------------------------------------------------------------------
# safetensors


def read_safetensors(path):
    """name -> (dtype string, shape, raw bytes)."""
    out = {}
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(n))
        base = 8 + n
        for name, info in header.items():
            if name == "__metadata__":
                continue
            a, b = info["data_offsets"]
            f.seek(base + a)
            out[name] = (info["dtype"], info["shape"], f.read(b - a))
    return out


_NP = {"F32": np.float32, "F16": np.float16, "BF16": np.uint16, "F8_E4M3": np.uint8, "F8_E5M2": np.uint8,
       "U8": np.uint8, "I8": np.int8, "I32": np.int32, "I64": np.int64}


def as_array(entry):
    dt, shape, raw = entry
    return np.frombuffer(raw, dtype=_NP[dt]).reshape(shape).copy()


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def load_fixture_tensors(d):
    tensors = {}
    for f in sorted(os.listdir(d)):
        if f.endswith(".safetensors"):
            tensors.update(read_safetensors(os.path.join(d, f)))
    return tensors


# ---------------------------------------------------------------------------
# GGUF (v3): header, metadata and tensor infos; tensors stay in their block type

GGML_TYPES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0", 12: "Q4_K", 14: "Q6_K",
              15: "Q8_K", 30: "BF16"}
GGUF_TO_DITCH = {"Q8_0": abi.Q8_0, "Q4_0": abi.Q4_0, "Q4_1": abi.Q4_1, "Q5_0": abi.Q5_0, "Q5_1": abi.Q5_1,
                 "Q4_K": abi.Q4_K, "Q6_K": abi.Q6_K, "Q8_K": abi.Q8_K}
BLOCK = {"Q8_0": (32, 34), "Q4_0": (32, 18), "Q4_1": (32, 20), "Q5_0": (32, 22), "Q5_1": (32, 24),
         "Q4_K": (256, 144), "Q6_K": (256, 210), "Q8_K": (256, 292), "F32": (1, 4), "F16": (1, 2), "BF16": (1, 2)}


def read_gguf(path):
    data = open(path, "rb").read()
    pos = 0

    def take(fmt):
        nonlocal pos
        v = struct.unpack_from("<" + fmt, data, pos)
        pos += struct.calcsize("<" + fmt)
        return v[0] if len(v) == 1 else v

    def string():
        nonlocal pos
        n = take("Q")
        s = data[pos:pos + n].decode("utf-8", "replace")
        pos += n
        return s

    scalar = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}

    def value(t):
        if t in scalar:
            return take(scalar[t])
        if t == 8:
            return string()
        if t == 9:
            it, n = take("I"), take("Q")
            return [value(it) for _ in range(n)]
        raise ValueError(f"gguf value type {t}")

    assert data[:4] == b"GGUF"
    pos = 4
    version = take("I")
    n_tensors, n_kv = take("Q"), take("Q")
    meta = {}
    for _ in range(n_kv):
        k = string()
        meta[k] = value(take("I"))
    infos = []
    for _ in range(n_tensors):
        name = string()
        nd = take("I")
        dims = [take("Q") for _ in range(nd)]
        ttype = take("I")
        off = take("Q")
        infos.append((name, dims, GGML_TYPES[ttype], off))
    align = int(meta.get("general.alignment", 32))
    base = (pos + align - 1) // align * align
    tensors = {}
    for name, dims, tt, off in infos:
        cols = dims[0]
        rows = int(np.prod(dims[1:])) if len(dims) > 1 else 1
        bs, bb = BLOCK[tt]
        nbytes = rows * (cols // bs) * bb
        tensors[name] = (tt, rows, cols, data[base + off: base + off + nbytes])
    return version, meta, tensors


# ---------------------------------------------------------------------------
# fixture -> ModelSpec


def _w_plain(entry):
    dt, shape, raw = entry
    if dt == "BF16":
        return HostWeight.bf16(as_array(entry))
    if dt == "F32":
        return HostWeight.f32(as_array(entry))
    if dt == "F16":
        return HostWeight.f16(as_array(entry))
    raise ValueError(dt)


def _vec(entry):
    dt = entry[0]
    a = as_array(entry)
    if dt == "BF16":
        a = bf16_to_f32(a)
    return vector(np.asarray(a, dtype=np.float32))


def _quant_weight(tensors, prefix, qc):
    """The weight at `prefix` (…proj): plain, FP8 (dequant.zig:855-947) or
    pack-quantized INT (dequant.zig:1072-1187)."""
    if prefix + ".weight_packed" in tensors:
        shape = as_array(tensors[prefix + ".weight_shape"])
        rows, cols = int(shape[0]), int(shape[1])
        words = as_array(tensors[prefix + ".weight_packed"])
        sc_entry = tensors[prefix + ".weight_scale"]
        scale = ("bf16", as_array(sc_entry)) if sc_entry[0] == "BF16" else as_array(sc_entry)
        zp = as_array(tensors[prefix + ".weight_zero_point"]) if prefix + ".weight_zero_point" in tensors else None
        gidx = as_array(tensors[prefix + ".weight_g_idx"]) if prefix + ".weight_g_idx" in tensors else None
        groups = as_array(sc_entry).shape[1]
        bits = qc["num_bits"]
        group = qc.get("group_size") or (cols + groups - 1) // groups
        return HostWeight.int_packed(words, scale, rows, cols, bits, group, zero=zp, g_idx=gidx)
    entry = tensors[prefix + ".weight"]
    if entry[0] in ("F8_E4M3", "F8_E5M2"):
        codes = as_array(entry)
        sk = prefix + ".weight_scale_inv" if prefix + ".weight_scale_inv" in tensors else prefix + ".weight_scale"
        se = tensors[sk]
        scale = as_array(se)
        if se[0] == "BF16":
            scale = ("bf16", scale)
        br, bcol = qc.get("block", (0, 0))
        srows, scols = as_array(se).shape
        if not br:
            br = -(-codes.shape[0] // srows)
            bcol = -(-codes.shape[1] // scols)
        return HostWeight.fp8(codes, scale, br, bcol, e5m2=entry[0] == "F8_E5M2")
    return _w_plain(entry)


def _quant_config(cfg):
    qc = cfg.get("quantization_config")
    if not qc:
        return {}
    if qc.get("quant_method") == "fp8":
        bs = qc.get("weight_block_size")
        return {"block": tuple(bs) if bs else (0, 0)}
    if qc.get("format") == "pack-quantized":
        g = next(iter(qc["config_groups"].values()))["weights"]
        return {"num_bits": g.get("num_bits", 4), "group_size": g.get("group_size")}
    return {}


def spec_from_hf(name):
    """ModelSpec of a Hugging Face fixture directory (qwen2, llama, qwen3_moe,
    deepseek_v3 and the quantised qwen2 variants)."""
    d = os.path.join(FIXTURES, name)
    cfg = json.load(open(os.path.join(d, "config.json")))
    tensors = load_fixture_tensors(d)
    qc = _quant_config(cfg)
    mt = cfg["model_type"]
    hidden = cfg["hidden_size"]
    heads = cfg["num_attention_heads"]
    layers = cfg["num_hidden_layers"]
    hd = cfg.get("head_dim") or hidden // heads
    c = dict(hidden=hidden, inter=cfg.get("intermediate_size", 0), layers=layers, heads=heads,
             kv_heads=cfg.get("num_key_value_heads", heads), head_dim=hd, vocab=cfg["vocab_size"],
             rms_eps=cfg.get("rms_norm_eps", 1e-6), rope_theta=cfg.get("rope_theta", 10000.0),
             rope_len=rope_len_for(cfg.get("max_position_embeddings", 2048)),
             tie_embeddings=int(cfg.get("tie_word_embeddings", False)))
    if mt == "qwen2":
        c["qkv_bias"] = int(cfg.get("attention_bias", True))
    if mt in ("qwen3_moe", "qwen3"):
        c["qk_norm"] = 1
    rs = cfg.get("rope_scaling") or {}
    rt = rs.get("rope_type") or rs.get("type") or ""
    if rt == "llama3":
        c.update(rope_scaling=abi.ROPE_SCALING_LLAMA3, rope_factor=rs.get("factor", 8.0),
                 rope_low_freq_factor=rs.get("low_freq_factor", 1.0),
                 rope_high_freq_factor=rs.get("high_freq_factor", 4.0),
                 rope_original_max_position=rs.get("original_max_position_embeddings", 8192))
    elif rt == "yarn":
        factor = rs.get("factor", 1.0)
        ms, msa = rs.get("mscale", 1.0), rs.get("mscale_all_dim", 0.0)
        if "attention_factor" in rs:
            af = rs["attention_factor"]
        elif ms and msa:
            af = float(np.float32(yarn_mscale(factor, ms)) / np.float32(yarn_mscale(factor, msa)))
        else:
            af = yarn_mscale(factor, 1.0)
        c.update(rope_scaling=abi.ROPE_SCALING_YARN, rope_factor=factor,
                 rope_original_max_position=rs.get("original_max_position_embeddings",
                                                   cfg.get("original_max_position_embeddings", 4096)),
                 yarn_beta_fast=rs.get("beta_fast", 32), yarn_beta_slow=rs.get("beta_slow", 1),
                 yarn_attention_factor=af, yarn_truncate=int(rs.get("truncate", True)))
    n_exp = cfg.get("num_experts") or cfg.get("n_routed_experts") or 0
    moe_layers = None
    if n_exp:
        step = max(cfg.get("decoder_sparse_step") or cfg.get("moe_layer_freq") or 1, 1)
        first = cfg.get("first_k_dense_replace", 0)
        if "moe_layer_freq" in cfg:
            moe_layers = [int(i >= first and i % step == 0) for i in range(layers)]
        else:
            moe_layers = [int(i >= first and (i + 1) % step == 0) for i in range(layers)]
        for i in cfg.get("mlp_only_layers", []):
            moe_layers[i] = 0
        c.update(n_experts=n_exp, top_k=cfg.get("num_experts_per_tok", 2),
                 moe_inter=cfg.get("moe_intermediate_size"), norm_topk_prob=int(cfg.get("norm_topk_prob", False)))
    if mt == "deepseek_v3":
        nope, rd = cfg["qk_nope_head_dim"], cfg["qk_rope_head_dim"]
        scale = np.float32(1.0) / np.sqrt(np.float32(nope + rd))
        if rt == "yarn" and rs.get("mscale_all_dim"):
            ms = np.float32(yarn_mscale(rs.get("factor", 1.0), rs["mscale_all_dim"]))
            scale = scale * ms * ms
        c.update(mla=1, head_dim=nope + rd, v_head_dim=cfg["v_head_dim"], kv_heads=heads,
                 q_lora_rank=cfg.get("q_lora_rank") or 0, kv_lora_rank=cfg["kv_lora_rank"], qk_nope_dim=nope,
                 qk_rope_dim=rd, rotary_dim=rd, attn_scale=float(scale),
                 rope_style=abi.ROPE_GPTJ if cfg.get("rope_interleave", True) else abi.ROPE_NEOX,
                 scoring=abi.SCORING_SIGMOID if cfg.get("scoring_func") == "sigmoid" else abi.SCORING_SOFTMAX,
                 group_limited=int(cfg.get("topk_method") in ("noaux_tc", "group_limited_greedy")),
                 n_group=max(1, cfg.get("n_group", 1)), topk_group=max(1, cfg.get("topk_group", 1)),
                 routed_scaling=cfg.get("routed_scaling_factor", 1.0),
                 shared_inter=cfg.get("moe_intermediate_size", 0) * cfg.get("n_shared_experts", 0))
    spec = ModelSpec(moe_layers=moe_layers, **c)
    spec.set("EMBED", _w_plain(tensors["model.embed_tokens.weight"]))
    spec.set("FINAL_NORM", _vec(tensors["model.norm.weight"]))
    if "lm_head.weight" in tensors:
        spec.set("LM_HEAD", _w_plain(tensors["lm_head.weight"]))
    for li in range(layers):
        p = f"model.layers.{li}."
        spec.set("ATTN_NORM", _vec(tensors[p + "input_layernorm.weight"]), li)
        spec.set("FFN_NORM", _vec(tensors[p + "post_attention_layernorm.weight"]), li)
        a = p + "self_attn."
        if c.get("mla"):
            if a + "q_a_proj.weight" in tensors:
                spec.set("MLA_Q_A", _quant_weight(tensors, a + "q_a_proj", qc), li)
                spec.set("MLA_Q_A_NORM", _vec(tensors[a + "q_a_layernorm.weight"]), li)
                spec.set("MLA_Q_B", _quant_weight(tensors, a + "q_b_proj", qc), li)
            else:
                spec.set("MLA_Q_B", _quant_weight(tensors, a + "q_proj", qc), li)
            spec.set("MLA_KV_A", _quant_weight(tensors, a + "kv_a_proj_with_mqa", qc), li)
            spec.set("MLA_KV_A_NORM", _vec(tensors[a + "kv_a_layernorm.weight"]), li)
            spec.set("MLA_KV_B", _quant_weight(tensors, a + "kv_b_proj", qc), li)
        else:
            for s, nm in (("Q", "q_proj"), ("K", "k_proj"), ("V", "v_proj")):
                spec.set(s, _quant_weight(tensors, a + nm, qc), li)
                if a + nm + ".bias" in tensors:
                    spec.set(s + "_BIAS", _vec(tensors[a + nm + ".bias"]), li)
            if a + "q_norm.weight" in tensors:
                spec.set("Q_NORM", _vec(tensors[a + "q_norm.weight"]), li)
                spec.set("K_NORM", _vec(tensors[a + "k_norm.weight"]), li)
        spec.set("O", _quant_weight(tensors, a + "o_proj", qc), li)
        m = p + "mlp."
        if moe_layers and moe_layers[li]:
            spec.set("ROUTER", _w_plain(tensors[m + "gate.weight"]), li)
            if m + "gate.e_score_correction_bias" in tensors:
                spec.set("ROUTER_CORRECTION", _vec(tensors[m + "gate.e_score_correction_bias"]), li)
            fused = tensors.get(m + "experts.gate_up_proj") or tensors.get(m + "experts.gate_up_proj.weight")
            if fused is not None:
                _set_fused_experts(spec, li, fused, tensors.get(m + "experts.down_proj")
                                   or tensors[m + "experts.down_proj.weight"], c["moe_inter"], hidden)
            for e in range(n_exp if fused is None else 0):
                ep = f"{m}experts.{e}."
                spec.set("EXPERT_GATE", _quant_weight(tensors, ep + "gate_proj", qc), li, e)
                spec.set("EXPERT_UP", _quant_weight(tensors, ep + "up_proj", qc), li, e)
                spec.set("EXPERT_DOWN", _quant_weight(tensors, ep + "down_proj", qc), li, e)
            if m + "shared_experts.gate_proj.weight" in tensors:
                sp = m + "shared_experts."
                spec.set("SHARED_GATE", _quant_weight(tensors, sp + "gate_proj", qc), li)
                spec.set("SHARED_UP", _quant_weight(tensors, sp + "up_proj", qc), li)
                spec.set("SHARED_DOWN", _quant_weight(tensors, sp + "down_proj", qc), li)
        else:
            spec.set("GATE", _quant_weight(tensors, m + "gate_proj", qc), li)
            spec.set("UP", _quant_weight(tensors, m + "up_proj", qc), li)
            spec.set("DOWN", _quant_weight(tensors, m + "down_proj", qc), li)
    return spec


def _set_fused_experts(spec, li, gate_up, down, inter, hidden):
    """Stacked routed experts (moe.zig:83-93): gate_up [E, 2I, H] with down
    [E, H, I] (gate = rows :I, up = rows I:), or the transposed pair
    gate_up [E, H, 2I] with down [E, I, H]."""
    gu, dn = as_array(gate_up), as_array(down)
    dt = gate_up[0]
    wrap = {"BF16": HostWeight.bf16, "F32": HostWeight.f32, "F16": HostWeight.f16}[dt]
    if gu.shape[1:] == (2 * inter, hidden):
        gates, ups, downs = gu[:, :inter, :], gu[:, inter:, :], dn
    else:
        assert gu.shape[1:] == (hidden, 2 * inter) and dn.shape[1:] == (inter, hidden)
        gates = gu[:, :, :inter].transpose(0, 2, 1)
        ups = gu[:, :, inter:].transpose(0, 2, 1)
        downs = dn.transpose(0, 2, 1)
    for e in range(gu.shape[0]):
        spec.set("EXPERT_GATE", wrap(np.ascontiguousarray(gates[e])), li, e)
        spec.set("EXPERT_UP", wrap(np.ascontiguousarray(ups[e])), li, e)
        spec.set("EXPERT_DOWN", wrap(np.ascontiguousarray(downs[e])), li, e)


def _gguf_weight(entry):
    tt, rows, cols, raw = entry
    if tt in GGUF_TO_DITCH:
        return HostWeight.gguf(GGUF_TO_DITCH[tt], np.frombuffer(raw, dtype=np.uint8), rows, cols)
    if tt == "F32":
        return HostWeight.f32(np.frombuffer(raw, dtype=np.float32).reshape(rows, cols))
    if tt == "F16":
        return HostWeight.f16(np.frombuffer(raw, dtype=np.float16).reshape(rows, cols))
    if tt == "BF16":
        return HostWeight.bf16(np.frombuffer(raw, dtype=np.uint16).reshape(rows, cols))
    raise ValueError(tt)


def _gguf_vec(entry):
    tt, rows, cols, raw = entry
    if tt == "F32":
        return vector(np.frombuffer(raw, dtype=np.float32))
    if tt == "F16":
        return vector(np.frombuffer(raw, dtype=np.float16).astype(np.float32))
    if tt == "BF16":
        return vector(bf16_to_f32(np.frombuffer(raw, dtype=np.uint16)))
    raise ValueError(tt)


def unpermute_rows(raw, rows, row_bytes, n_head):
    """Undoes llama.cpp's q/k permutation on whole rows (gguf_model.zig:649-680):
    the file holds head rows in (pair, half) order; HF holds (half, pair)."""
    a = np.frombuffer(raw, dtype=np.uint8).reshape(rows, row_bytes)
    hd = rows // n_head
    a = a.reshape(n_head, hd // 2, 2, row_bytes).transpose(0, 2, 1, 3).reshape(rows, row_bytes)
    return a.tobytes()


def spec_from_gguf(name):
    d = os.path.join(FIXTURES, name)
    _, meta, t = read_gguf(os.path.join(d, "model.gguf"))
    arch = meta["general.architecture"]
    k = lambda s, dflt=None: meta.get(f"{arch}.{s}", dflt)
    hidden = k("embedding_length")
    heads = k("attention.head_count")
    kvh = k("attention.head_count_kv", heads)
    layers = k("block_count")
    vocab = t["token_embd.weight"][1]
    hd = k("attention.key_length", hidden // heads)
    c = dict(hidden=hidden, inter=k("feed_forward_length"), layers=layers, heads=heads, kv_heads=kvh, head_dim=hd,
             vocab=vocab, rms_eps=k("attention.layer_norm_rms_epsilon", 1e-6),
             rope_theta=k("rope.freq_base", 10000.0), rope_len=rope_len_for(k("context_length", 2048)))
    if arch == "qwen2":
        c["qkv_bias"] = 1
    permute = arch == "llama"
    if "rope_freqs.weight" in t:
        # gguf_model.zig:320-336: llama3 factors are written back as llama3
        # scaling only when they match Llama 3's own constants (8192 original
        # positions); a fixture's factors are carried as divisors.
        c.update(rope_scaling=abi.ROPE_SCALING_FACTORS,
                 rope_factors=np.frombuffer(t["rope_freqs.weight"][3], dtype=np.float32).copy())
    spec = ModelSpec(**c)
    spec.set("EMBED", _gguf_weight(t["token_embd.weight"]))
    spec.set("FINAL_NORM", _gguf_vec(t["output_norm.weight"]))
    if "output.weight" in t:
        spec.set("LM_HEAD", _gguf_weight(t["output.weight"]))
    for li in range(layers):
        b = f"blk.{li}."
        spec.set("ATTN_NORM", _gguf_vec(t[b + "attn_norm.weight"]), li)
        spec.set("FFN_NORM", _gguf_vec(t[b + "ffn_norm.weight"]), li)
        for s, nm, nh in (("Q", "attn_q", heads), ("K", "attn_k", kvh), ("V", "attn_v", None)):
            tt, rows, cols, raw = t[b + nm + ".weight"]
            if permute and nh:
                bs, bb = BLOCK[tt]
                raw = unpermute_rows(raw, rows, cols // bs * bb, nh)
            spec.set(s, _gguf_weight((tt, rows, cols, raw)), li)
            if b + nm + ".bias" in t:
                bt, br, bc, braw = t[b + nm + ".bias"]
                if permute and nh:
                    braw = unpermute_rows(braw, bc, BLOCK[bt][1], nh)
                spec.set(s + "_BIAS", _gguf_vec((bt, br, bc, braw)), li)
        spec.set("O", _gguf_weight(t[b + "attn_output.weight"]), li)
        spec.set("GATE", _gguf_weight(t[b + "ffn_gate.weight"]), li)
        spec.set("UP", _gguf_weight(t[b + "ffn_up.weight"]), li)
        spec.set("DOWN", _gguf_weight(t[b + "ffn_down.weight"]), li)
    return spec


def golden(name):
    return json.load(open(os.path.join(FIXTURES, name, "reference.json")))


def case_rows(ids):
    """One prompt in batch slot 0: rows (0, pos)."""
    return [(0, p) for p in range(len(ids))]
