"""ctypes mirror of include/ditch_hip.h (structs, enums and prototypes).

The C header is the boundary; this module only restates its layout so that
Python callers (tests, bench.py, the smoke entry) can fill the same structs.
Every field order and width here must match include/ditch_hip.h.
"""
import ctypes as C

# status codes (compute.zig:54-60)
OK, UNSUPPORTED, DEVICE_FAILED, OUT_OF_MEMORY, INVALID_ARGUMENT = 0, 1, 2, 3, 4
STATUS_NAMES = {
    OK: "ok",
    UNSUPPORTED: "Unsupported",
    DEVICE_FAILED: "DeviceFailed",
    OUT_OF_MEMORY: "OutOfMemory",
    INVALID_ARGUMENT: "InvalidArgument",
}

# storage formats (tensor.zig:11-33 numbering, then dequant.zig formats)
F32, F16, BF16, I64, I32 = 0, 1, 2, 3, 4
Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q4_K, Q6_K, Q8_K = 5, 6, 7, 8, 9, 10, 11, 12
FP8, MXFP4, MXFP4_T, INT_PACKED = 32, 33, 34, 35
E8M0 = 40

ROPE_NEOX, ROPE_GPTJ = 0, 1
ROPE_SCALING_NONE, ROPE_SCALING_LINEAR, ROPE_SCALING_LLAMA3, ROPE_SCALING_YARN, ROPE_SCALING_FACTORS = 0, 1, 2, 3, 4
SCORING_SOFTMAX, SCORING_SIGMOID = 0, 1

SLOT = dict(
    EMBED=0, FINAL_NORM=1, LM_HEAD=2,
    ATTN_NORM=10, Q=11, K=12, V=13, O=14, Q_BIAS=15, K_BIAS=16, V_BIAS=17,
    Q_NORM=18, K_NORM=19, FFN_NORM=20, GATE=21, UP=22, DOWN=23,
    ROUTER=30, ROUTER_CORRECTION=31, EXPERT_GATE=32, EXPERT_UP=33,
    EXPERT_DOWN=34, SHARED_GATE=35, SHARED_UP=36, SHARED_DOWN=37,
    MLA_Q_A=40, MLA_Q_A_NORM=41, MLA_Q_B=42, MLA_KV_A=43, MLA_KV_A_NORM=44,
    MLA_KV_B=45,
)
VECTOR_SLOTS = {
    SLOT[k] for k in ("FINAL_NORM", "ATTN_NORM", "Q_BIAS", "K_BIAS", "V_BIAS",
                      "Q_NORM", "K_NORM", "FFN_NORM", "ROUTER_CORRECTION",
                      "MLA_Q_A_NORM", "MLA_KV_A_NORM")
}


class Weight(C.Structure):
    """`ditch_weight` (tensor.Weight widened with the Dequant pieces)."""
    _fields_ = [
        ("data", C.c_void_p),
        ("dtype", C.c_int32),
        ("scale_dtype", C.c_int32),
        ("rows", C.c_uint64),
        ("cols", C.c_uint64),
        ("scale", C.c_void_p),
        ("scale_rows", C.c_uint64),
        ("scale_cols", C.c_uint64),
        ("block_rows", C.c_uint64),
        ("block_cols", C.c_uint64),
        ("row_shard", C.c_uint64),
        ("fp8_e5m2", C.c_int32),
        ("bits", C.c_int32),
        ("group", C.c_uint64),
        ("zero", C.c_void_p),
        ("g_idx", C.c_void_p),
    ]


class ModelConfig(C.Structure):
    """`ditch_model_config`."""
    _fields_ = [
        ("hidden", C.c_uint64),
        ("inter", C.c_uint64),
        ("layers", C.c_uint64),
        ("heads", C.c_uint64),
        ("kv_heads", C.c_uint64),
        ("head_dim", C.c_uint64),
        ("v_head_dim", C.c_uint64),
        ("vocab", C.c_uint64),
        ("rms_eps", C.c_float),
        ("attn_scale", C.c_float),
        ("qkv_bias", C.c_int32),
        ("qk_norm", C.c_int32),
        ("tie_embeddings", C.c_int32),
        ("rope_style", C.c_int32),
        ("rotary_dim", C.c_uint64),
        ("rope_len", C.c_uint64),
        ("rope_theta", C.c_float),
        ("rope_scaling", C.c_int32),
        ("rope_factor", C.c_float),
        ("rope_low_freq_factor", C.c_float),
        ("rope_high_freq_factor", C.c_float),
        ("rope_original_max_position", C.c_float),
        ("yarn_beta_fast", C.c_float),
        ("yarn_beta_slow", C.c_float),
        ("yarn_attention_factor", C.c_float),
        ("yarn_truncate", C.c_int32),
        ("rope_factors", C.c_void_p),
        ("n_experts", C.c_uint64),
        ("top_k", C.c_uint64),
        ("moe_inter", C.c_uint64),
        ("shared_inter", C.c_uint64),
        ("scoring", C.c_int32),
        ("norm_topk_prob", C.c_int32),
        ("group_limited", C.c_int32),
        ("n_group", C.c_uint64),
        ("topk_group", C.c_uint64),
        ("routed_scaling", C.c_float),
        ("moe_layers", C.c_void_p),
        ("mla", C.c_int32),
        ("q_lora_rank", C.c_uint64),
        ("kv_lora_rank", C.c_uint64),
        ("qk_nope_dim", C.c_uint64),
        ("qk_rope_dim", C.c_uint64),
        ("mla_norm_eps", C.c_float),
    ]


class Row(C.Structure):
    """`ditch_row` (model.Row {b, pos})."""
    _fields_ = [("b", C.c_uint32), ("pos", C.c_uint32)]


class EditOptions(C.Structure):
    """`ditch_edit_options` (abliterate.Options)."""
    _fields_ = [("row_normalization", C.c_int32), ("lora_rank", C.c_uint32), ("seed", C.c_uint64),
                ("ablate_inputs", C.c_int32)]


ROWNORM = {"none": 0, "pre": 1, "full": 2}


class EditTarget(C.Structure):
    """`ditch_edit_target`: one matrix of a batch edit."""
    _fields_ = [("layer", C.c_int32), ("slot", C.c_int32), ("expert", C.c_int32), ("weight", C.c_float),
                ("v", C.c_void_p)]


class Sampler(C.Structure):
    """`ditch_sampler` (model.Sampler): set it with `sampler(lib, ...)`."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float), ("reserved", C.c_uint32),
                ("rng", C.c_uint64 * 4)]


def sampler(lib, seed=0, temperature=1.0, top_k=50, top_p=0.95):
    """Sampler.init (model.zig:5216-5218) through ditch_hip_sampler_init."""
    s = Sampler()
    if lib.ditch_hip_sampler_init(C.byref(s), seed, temperature, top_k, top_p) != 0:
        raise ValueError("ditch_hip_sampler_init failed")
    return s


class PathStats(C.Structure):
    """`ditch_model_path_stats`."""
    _fields_ = [("moe_device_planned", C.c_uint64), ("moe_host_planned", C.c_uint64)]


class ResidencyStats(C.Structure):
    """`ditch_residency_stats` (compute.Residency's counters)."""
    _fields_ = [(n, C.c_uint64) for n in ("budget", "used", "entries", "hits", "misses", "evictions", "enabled")]


class ExpertCacheStats(C.Structure):
    """`ditch_expert_cache_stats` (expert_cache.Stats)."""
    _fields_ = [(n, C.c_uint64) for n in ("capacity", "slots", "resident", "hits", "misses", "prefetched",
                                          "bytes_read", "evictions", "slot_bytes", "warmed", "bytes_staged")]


class HotExpert(C.Structure):
    """`ditch_hot_expert` (ExpertCache.Hot)."""
    _fields_ = [("layer", C.c_uint32), ("expert", C.c_uint32), ("uses", C.c_uint64)]


P = C.c_void_p
U64 = C.c_uint64
I32 = C.c_int32
U32 = C.c_uint32
FLT = C.c_float

# name -> (restype, argtypes) for every function of include/ditch_hip.h
PROTOTYPES = {
    "ditch_hip_open": (P, [I32, C.c_char_p, C.c_size_t]),
    "ditch_hip_close": (None, [P]),
    "ditch_hip_name": (C.c_char_p, [P]),
    "ditch_hip_last_error": (C.c_char_p, [P]),
    "ditch_hip_forget_weights": (None, [P]),
    "ditch_hip_set_residency": (I32, [P, U64, I32]),
    "ditch_hip_model_hot_experts": (I32, [P, P, U64, P]),
    "ditch_hip_model_warm_experts": (I32, [P, P, U64, P]),
    "ditch_hip_residency_stats": (I32, [P, P]),
    "ditch_hip_stream": (P, [P]),
    "ditch_hip_sync": (I32, [P]),
    "ditch_hip_matmulT": (I32, [P, P, P, U64, P]),
    "ditch_hip_matvecTMulti": (I32, [P, P, P, P, U64]),
    "ditch_hip_rowNorms": (I32, [P, P, P]),
    "ditch_hip_attentionScores": (I32, [P, P, U64, P, U64, P, U64, FLT]),
    "ditch_hip_attentionValues": (I32, [P, P, U64, P, U64, P, U64]),
    "ditch_hip_gatedActivation": (I32, [P, U32, P, P, P, U64, U64, U64, U64]),
    "ditch_hip_rmsnormRows": (I32, [P, P, P, P, U64, U64, U64, FLT, I32]),
    "ditch_hip_layernormRows": (I32, [P, P, P, P, U64, P, U64, U64, FLT, I32]),
    "ditch_hip_softmaxRows": (I32, [P, P, U64, U64]),
    "ditch_hip_ropeRows": (I32, [P, P, U64, U64, P, P, U64, U64, P, U32]),
    "ditch_hip_dequant": (I32, [P, P, P, U64, U64]),
    "ditch_hip_upload": (P, [P, P]),
    "ditch_hip_tensor_free": (None, [P, P]),
    "ditch_hip_tensor_bytes": (U64, [P]),
    "ditch_hip_tensor_dequant": (I32, [P, P, U64, P, U64, U64]),
    "ditch_hip_matmulT_device": (I32, [P, P, U64, P, U64, U64, P, P, I32, P]),
    "ditch_hip_matmulT_device_noalloc": (I32, [P, P, U64, P, U64, U64, P, P, I32, P]),
    "ditch_hip_static_scratch_bytes": (U64, []),
    "ditch_hip_frag_bytes": (U64, [P, U64]),
    "ditch_hip_split_device": (I32, [P, P, U64, P, U64, P, P]),
    "ditch_hip_glu_frag_bytes": (U64, [P, P, U64]),
    "ditch_hip_glu_device": (I32, [P, P, U64, P, U64, U64, P, P, U32, P]),
    "ditch_hip_matmulT_frags_device": (I32, [P, P, U64, P, U64, U64, P, P, I32, P]),
    "ditch_hip_model_create": (P, [P, P]),
    "ditch_hip_model_free": (None, [P]),
    "ditch_hip_model_set": (I32, [P, I32, I32, I32, P]),
    "ditch_hip_model_set_delta": (I32, [P, I32, I32, I32, U64, P, P]),
    "ditch_hip_model_set_expert_cache": (I32, [P, U64]),
    "ditch_hip_model_expert_cache_stats": (I32, [P, P]),
    "ditch_hip_model_reset_deltas": (I32, [P]),
    "ditch_hip_model_bytes": (U64, [P]),
    "ditch_hip_forward": (I32, [P, P, P, U64, P, U64, P, P, U64, P]),
    "ditch_hip_forward_device": (I32, [P, P, P, U64, U32, U32, P, U64, P, U64, P, U64, P, U64]),
    "ditch_hip_model_path_stats": (I32, [P, P]),
    "ditch_hip_model_load": (P, [P, C.c_char_p, U64]),
    "ditch_hip_model_get_config": (I32, [P, P]),
    "ditch_hip_kv_cache_create": (P, [P, U32, U32]),
    "ditch_hip_kv_cache_free": (None, [P]),
    "ditch_hip_forward_cached": (I32, [P, P, P, P, U64, P, U64, P, U64]),
    "ditch_hip_sampler_init": (I32, [P, U64, FLT, U64, FLT]),
    "ditch_hip_pick_tokens_device": (I32, [P, P, P, U64, U64, P, P]),
    "ditch_hip_generate": (I32, [P, P, P, P, U64, U64, P, U64, P, P, P, P]),
    "ditch_hip_edit_delta": (I32, [P, P, P, P, P, U64, FLT]),
    "ditch_hip_model_edit": (I32, [P, I32, I32, I32, P, U64, FLT]),
    "ditch_hip_model_edit_batch": (I32, [P, P, U64, U64]),
    "ditch_hip_logSoftmaxRows": (I32, [P, P, P, U64, U64]),
    "ditch_hip_klRows": (I32, [P, P, P, P, U64, U64]),
    "ditch_hip_edit_rank": (U64, [U64, U64, U64, P]),
    "ditch_hip_edit_delta_ex": (I32, [P, P, U64, P, U64, P, P, U64, FLT, P]),
    "ditch_hip_model_edit_ex": (I32, [P, I32, I32, I32, P, U64, FLT, P]),
    "ditch_hip_edit_gaussian": (None, [P, U64, U64]),
    "ditch_hip_logSoftmaxRows_device": (I32, [P, P, P, U64, U64, P]),
    "ditch_hip_residual_reduce_device": (I32, [P, P, U64, U64, U64, P, P, U64, FLT, P, P, P, P]),
    "ditch_hip_residual_mean_device": (I32, [P, P, P, U64, U64, P]),
    "ditch_hip_directions_device": (I32, [P, P, P, P, U64, U64, I32, P]),
    "ditch_hip_sketch_add_device": (I32, [P, P, P, P, U64, P, P, U64, U64, U64, P]),
    "ditch_hip_basis_device": (I32, [P, P, P, P, U64, U64, U64, I32, P, P, U64, P]),
    "ditch_hip_klRows_device": (I32, [P, P, P, P, U64, U64, P]),
}


def header_symbols(header_path):
    """Names of the functions declared in include/ditch_hip.h."""
    import re
    text = open(header_path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ditch_hip_\w+)\s*\(", text)))
