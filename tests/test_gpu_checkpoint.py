"""The checkpoint reader (ditch_hip_model_load) on the GPU: every reference
fixture (Hugging Face directories and GGUF files) read from disk by the
library gives the fixture's goldens (model_test.zig:58-75, 2e-3) and the
same forward, bit for bit, as the model built from the test-side reader
(tests/fixture_io.py); the benchmark configurations' formats (MXFP4
mxfp4-pack-quantized, FP8 with 128 x 128 weight_scale_inv, INT4 group-128
pack-quantized, routed experts) written to a temporary checkpoint and read
back give the forward of the model registered from memory."""
import json
import os
import struct
import tempfile

import numpy as np
import pytest

import fixture_io as fx
import model_gen as mg
from ditch_amd import abi
from ditch_amd.hip import DeviceError, Model

pytestmark = pytest.mark.gpu

HF = ["qwen2", "llama", "qwen2_fp8", "qwen2_int4", "qwen2_int4_actorder", "qwen3_moe", "qwen3_moe_fused",
      "qwen3_moe_fused_t", "qwen3_moe_big", "deepseek_v3"]
GGUF = ["qwen2_gguf", "llama_gguf"]


def _forward(m, ids):
    n = len(ids)
    return m.forward(np.asarray(ids, np.uint32), fx.case_rows(ids), capture_rows=[n - 1], logit_rows=[n - 1])


@pytest.mark.parametrize("name", HF + GGUF)
def test_fixture_loaded_from_disk(dev, name):
    d = os.path.join(fx.FIXTURES, name)
    path = os.path.join(d, "model.gguf") if name in GGUF else d
    spec = fx.spec_from_gguf(name) if name in GGUF else fx.spec_from_hf(name)
    lm = Model.load(dev, path)
    sm = Model(dev, spec)
    try:
        for key in ("hidden", "layers", "heads", "kv_heads", "head_dim", "vocab", "n_experts", "mla"):
            assert lm.spec.config[key] == spec.config[key], key
        for case in fx.golden(name)["cases"]:
            rl, ll = _forward(lm, case["ids"])
            rs, ls = _forward(sm, case["ids"])
            np.testing.assert_array_equal(ll, ls)
            np.testing.assert_array_equal(rl, rs)
            np.testing.assert_allclose(ll[0], case["last_logits"], atol=2e-3, rtol=0)
            np.testing.assert_allclose(rl[:, 0, :], case["last_hidden"], atol=2e-3, rtol=0)
    finally:
        lm.free()
        sm.free()


def test_moe_fixture_loaded_with_expert_streaming(dev):
    name = "qwen3_moe"
    lm = Model.load(dev, os.path.join(fx.FIXTURES, name), expert_cache_bytes=1 << 30)
    sm = Model(dev, fx.spec_from_hf(name))
    try:
        for case in fx.golden(name)["cases"]:
            rl, ll = _forward(lm, case["ids"])
            rs, ls = _forward(sm, case["ids"])
            np.testing.assert_array_equal(ll, ls)
        assert lm.expert_cache_stats()["misses"] > 0
    finally:
        lm.free()
        sm.free()


# ---------------------------------------------------------------------------
# writing the configurations' formats to disk


def write_safetensors(path, tensors):
    """name -> numpy array (with its safetensors dtype string)."""
    header, blobs, off = {}, [], 0
    for name, (dt, a) in tensors.items():
        raw = np.ascontiguousarray(a).tobytes()
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def _weight_tensors(prefix, w):
    """The checkpoint tensors of one registered weight (the on-disk layouts
    of dequant.zig's formats)."""
    data, scale, zero, g_idx = w.arrays
    s = w.struct
    if w.dtype == abi.BF16:
        return {prefix + ".weight": ("BF16", data)}
    if w.dtype == abi.F32:
        return {prefix + ".weight": ("F32", data)}
    if w.dtype == abi.MXFP4:
        return {prefix + ".weight_packed": ("U8", data), prefix + ".weight_scale": ("U8", scale)}
    if w.dtype == abi.FP8:
        sdt = {abi.F32: "F32", abi.BF16: "BF16", abi.F16: "F16"}[s.scale_dtype]
        return {prefix + ".weight": ("F8_E5M2" if s.fp8_e5m2 else "F8_E4M3", data),
                prefix + ".weight_scale_inv": (sdt, scale)}
    if w.dtype == abi.INT_PACKED:
        sdt = {abi.F32: "F32", abi.BF16: "BF16", abi.F16: "F16"}[s.scale_dtype]
        out = {prefix + ".weight_packed": ("I32", data), prefix + ".weight_scale": (sdt, scale),
               prefix + ".weight_shape": ("I64", np.array([s.rows, s.cols], dtype=np.int64))}
        if zero is not None:
            out[prefix + ".weight_zero_point"] = ("I32", zero)
        return out
    raise ValueError(w.dtype)


def _vec_tensor(name, w):
    return {name: ("F32", w.arrays[0].reshape(-1))}


def write_checkpoint(d, spec, model_type, qc=None, extra=None):
    c = spec.config
    cfg = {"model_type": model_type, "hidden_size": c["hidden"], "intermediate_size": c["inter"],
           "num_hidden_layers": c["layers"], "num_attention_heads": c["heads"], "num_key_value_heads": c["kv_heads"],
           "head_dim": c["head_dim"], "vocab_size": c["vocab"], "rms_norm_eps": c["rms_eps"],
           "rope_theta": c["rope_theta"], "max_position_embeddings": c["rope_len"],
           "tie_word_embeddings": bool(c["tie_embeddings"])}
    if qc:
        cfg["quantization_config"] = qc
    cfg.update(extra or {})
    t = {}
    t.update(_weight_tensors("model.embed_tokens", spec.get("EMBED")))
    t.update(_vec_tensor("model.norm.weight", spec.get("FINAL_NORM")))
    if spec.get("LM_HEAD") is not None:
        t.update(_weight_tensors("lm_head", spec.get("LM_HEAD")))
    for li in range(c["layers"]):
        p = f"model.layers.{li}."
        t.update(_vec_tensor(p + "input_layernorm.weight", spec.get("ATTN_NORM", li)))
        t.update(_vec_tensor(p + "post_attention_layernorm.weight", spec.get("FFN_NORM", li)))
        for s, nm in (("Q", "q_proj"), ("K", "k_proj"), ("V", "v_proj"), ("O", "o_proj")):
            t.update(_weight_tensors(p + "self_attn." + nm, spec.get(s, li)))
        if spec.get("Q_NORM", li) is not None:
            t.update(_vec_tensor(p + "self_attn.q_norm.weight", spec.get("Q_NORM", li)))
            t.update(_vec_tensor(p + "self_attn.k_norm.weight", spec.get("K_NORM", li)))
        if spec.moe_layers[li]:
            t.update(_weight_tensors(p + "mlp.gate", spec.get("ROUTER", li)))
            for e in range(c["n_experts"]):
                for s, nm in (("EXPERT_GATE", "gate_proj"), ("EXPERT_UP", "up_proj"), ("EXPERT_DOWN", "down_proj")):
                    t.update(_weight_tensors(f"{p}mlp.experts.{e}.{nm}", spec.get(s, li, e)))
        else:
            for s, nm in (("GATE", "gate_proj"), ("UP", "up_proj"), ("DOWN", "down_proj")):
                t.update(_weight_tensors(p + "mlp." + nm, spec.get(s, li)))
    names = sorted(t)
    half = len(names) // 2  # two shards
    write_safetensors(os.path.join(d, "model-00001-of-00002.safetensors"), {n: t[n] for n in names[:half]})
    write_safetensors(os.path.join(d, "model-00002-of-00002.safetensors"), {n: t[n] for n in names[half:]})
    json.dump(cfg, open(os.path.join(d, "config.json"), "w"))


QC = {
    "mxfp4": {"quant_method": "compressed-tensors", "format": "mxfp4-pack-quantized",
              "config_groups": {"group_0": {"weights": {"num_bits": 4, "group_size": 32}}}},
    "fp8": {"quant_method": "fp8", "weight_block_size": [128, 128]},
    "int4": {"quant_method": "compressed-tensors", "format": "pack-quantized",
             "config_groups": {"group_0": {"weights": {"num_bits": 4, "group_size": 128}}}},
}


@pytest.mark.parametrize("fmt", ["mxfp4", "fp8", "int4"])
def test_configuration_formats_round_trip(dev, fmt):
    spec = mg.dense(fmt, hidden=512, inter=1024, layers=2, heads=8, kv_heads=2, head_dim=64, vocab=1000, seed=7,
                    tie=False)
    tokens, rows, last = mg.batch(3, [40, 7, 130], spec.config["vocab"], seed=8)
    with tempfile.TemporaryDirectory() as d:
        write_checkpoint(d, spec, "llama", QC[fmt])
        lm = Model.load(dev, d)
    sm = Model(dev, spec)
    try:
        rl, ll = lm.forward(tokens, rows, capture_rows=last, logit_rows=last)
        rs, ls = sm.forward(tokens, rows, capture_rows=last, logit_rows=last)
        np.testing.assert_array_equal(ll, ls)
        np.testing.assert_array_equal(rl, rs)
    finally:
        lm.free()
        sm.free()


def test_moe_checkpoint_round_trip(dev):
    spec = mg.moe("int4", hidden=256, layers=2, experts=8, top_k=2, moe_inter=128, vocab=1000, seed=9)
    extra = {"num_experts": 8, "num_experts_per_tok": 2, "moe_intermediate_size": 128, "norm_topk_prob": True,
             "decoder_sparse_step": 1}
    tokens, rows, last = mg.batch(2, [30, 12], spec.config["vocab"], seed=10)
    with tempfile.TemporaryDirectory() as d:
        write_checkpoint(d, spec, "qwen3_moe", QC["int4"], extra)
        lm = Model.load(dev, d)
    sm = Model(dev, spec)
    try:
        np.testing.assert_array_equal(lm.forward(tokens, rows, logit_rows=last)[1],
                                      sm.forward(tokens, rows, logit_rows=last)[1])
    finally:
        lm.free()
        sm.free()


def test_load_failures_are_reported(dev):
    with pytest.raises(DeviceError, match="cannot stat"):
        Model.load(dev, "/nonexistent/checkpoint")
    with tempfile.TemporaryDirectory() as d:
        json.dump({"model_type": "gpt2"}, open(os.path.join(d, "config.json"), "w"))
        with pytest.raises(DeviceError, match="model_type"):
            Model.load(dev, d)
        json.dump({"model_type": "llama"}, open(os.path.join(d, "config.json"), "w"))
        open(os.path.join(d, "model.safetensors"), "wb").write(struct.pack("<Q", 1 << 40))
        with pytest.raises(DeviceError, match="header past the end"):
            Model.load(dev, d)
    with tempfile.NamedTemporaryFile(suffix=".gguf") as f:
        f.write(b"GGUF" + struct.pack("<I", 3) + b"\x00" * 4)
        f.flush()
        with pytest.raises(DeviceError, match="truncated"):
            Model.load(dev, f.name)


def _gguf_string(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def test_inconsistent_checkpoints_are_refused_on_the_host(dev):
    """Tensors that disagree with each other are refused before anything is
    uploaded: pack-quantized codes narrower than weight_shape needs, MXFP4
    scales shorter than the codes need, a GGUF tensor whose size
    overflows."""
    spec = mg.dense("int4", hidden=256, inter=512, layers=1, heads=4, kv_heads=2, head_dim=64, vocab=300, seed=3,
                    tie=False)
    with tempfile.TemporaryDirectory() as d:
        write_checkpoint(d, spec, "llama", QC["int4"])
        shard = [f for f in sorted(os.listdir(d)) if f.endswith(".safetensors")]
        tensors = {}
        for f in shard:
            tensors.update({k: (dt, fx.as_array((dt, shp, raw))) for k, (dt, shp, raw) in
                            fx.read_safetensors(os.path.join(d, f)).items()})
            os.remove(os.path.join(d, f))
        name = "model.layers.0.mlp.down_proj.weight_packed"
        tensors[name] = ("I32", np.ascontiguousarray(tensors[name][1][:, :-1]))
        write_safetensors(os.path.join(d, "model.safetensors"), tensors)
        with pytest.raises(DeviceError, match="fewer bytes"):
            Model.load(dev, d)
    spec = mg.dense("mxfp4", hidden=256, inter=512, layers=1, heads=4, kv_heads=2, head_dim=64, vocab=300, seed=3,
                    tie=False)
    with tempfile.TemporaryDirectory() as d:
        write_checkpoint(d, spec, "llama", QC["mxfp4"])
        tensors = {}
        for f in [f for f in sorted(os.listdir(d)) if f.endswith(".safetensors")]:
            tensors.update({k: (dt, fx.as_array((dt, shp, raw))) for k, (dt, shp, raw) in
                            fx.read_safetensors(os.path.join(d, f)).items()})
            os.remove(os.path.join(d, f))
        name = "model.layers.0.self_attn.o_proj.weight_scale"
        tensors[name] = ("U8", np.ascontiguousarray(tensors[name][1][:, :-1]))
        write_safetensors(os.path.join(d, "model.safetensors"), tensors)
        with pytest.raises(DeviceError, match="fewer bytes"):
            Model.load(dev, d)
    with tempfile.NamedTemporaryFile(suffix=".gguf") as f:
        hdr = b"GGUF" + struct.pack("<IQQ", 3, 1, 1)
        hdr += _gguf_string("general.architecture") + struct.pack("<I", 8) + _gguf_string("llama")
        # Q8_0 (type 8) tensor of 2^39 x 2^39: its byte count overflows 64 bits
        hdr += _gguf_string("token_embd.weight") + struct.pack("<IQQIQ", 2, 1 << 39, 1 << 39, 8, 0)
        f.write(hdr + b"\x00" * 64)
        f.flush()
        with pytest.raises(DeviceError, match="overflows"):
            Model.load(dev, f.name)
