"""ModelSpec: the host description of a model to register on the device.

A spec is a config dict (the fields of `ditch_model_config`) plus the
tensors keyed by (layer, slot, expert) as `HostWeight`s. The same spec feeds
the device (`ditch_amd.hip.Model`) and, in the tests, the CPU oracle.
"""
import ctypes
import math

import numpy as np

from . import abi
from .weights import HostWeight, vector

DEFAULTS = dict(
    hidden=0, inter=0, layers=0, heads=0, kv_heads=0, head_dim=0, v_head_dim=0, vocab=0,
    rms_eps=1e-6, attn_scale=0.0, qkv_bias=0, qk_norm=0, tie_embeddings=0,
    rope_style=abi.ROPE_NEOX, rotary_dim=0, rope_len=512, rope_theta=10000.0,
    rope_scaling=abi.ROPE_SCALING_NONE, rope_factor=1.0, rope_low_freq_factor=1.0,
    rope_high_freq_factor=4.0, rope_original_max_position=8192.0, yarn_beta_fast=32.0,
    yarn_beta_slow=1.0, yarn_attention_factor=1.0, yarn_truncate=1, rope_factors=None,
    n_experts=0, top_k=0, moe_inter=0, shared_inter=0, scoring=abi.SCORING_SOFTMAX,
    norm_topk_prob=0, group_limited=0, n_group=1, topk_group=1, routed_scaling=1.0,
    mla=0, q_lora_rank=0, kv_lora_rank=0, qk_nope_dim=0, qk_rope_dim=0, mla_norm_eps=1e-6,
)


def rope_len_for(max_position):
    """model.zig:2179: clamp(max_position_embeddings, 512, 8192)."""
    return min(max(int(max_position), 512), 8192)


def yarn_mscale(scale, mscale):
    """arch.zig:1722-1725 (f32 arithmetic)."""
    if scale <= 1:
        return 1.0
    return float(np.float32(np.float32(0.1) * np.float32(mscale) * np.float32(math.log(np.float32(scale))) + np.float32(1.0)))


class ModelSpec:
    def __init__(self, **config):
        self.config = dict(DEFAULTS)
        unknown = set(config) - set(DEFAULTS) - {"moe_layers"}
        if unknown:
            raise ValueError(f"unknown config keys {sorted(unknown)}")
        self.config.update({k: v for k, v in config.items() if k != "moe_layers"})
        c = self.config
        if not c["v_head_dim"]:
            c["v_head_dim"] = c["head_dim"]
        if not c["rotary_dim"]:
            c["rotary_dim"] = c["qk_rope_dim"] if c["mla"] else c["head_dim"]
        if not c["attn_scale"]:
            c["attn_scale"] = float(np.float32(1.0) / np.sqrt(np.float32(c["head_dim"])))
        self.moe_layers = np.zeros(c["layers"], dtype=np.uint8)
        if config.get("moe_layers") is not None:
            self.moe_layers[:] = np.asarray(config["moe_layers"], dtype=np.uint8)
        self.tensors = {}

    def set(self, slot, weight, layer=-1, expert=-1):
        if isinstance(slot, str):
            slot = abi.SLOT[slot]
        if not isinstance(weight, HostWeight):
            weight = vector(weight) if slot in abi.VECTOR_SLOTS else HostWeight.f32(weight)
        self.tensors[(layer, slot, expert)] = weight

    def get(self, slot, layer=-1, expert=-1):
        if isinstance(slot, str):
            slot = abi.SLOT[slot]
        return self.tensors.get((layer, slot, expert))

    def config_struct(self):
        s = abi.ModelConfig()
        for k, v in self.config.items():
            if k != "rope_factors":
                setattr(s, k, v)
        s.moe_layers = self.moe_layers.ctypes.data_as(ctypes.c_void_p)
        self._keep = [self.moe_layers]
        if self.config["rope_factors"] is not None:
            f = np.ascontiguousarray(self.config["rope_factors"], dtype=np.float32)
            s.rope_factors = f.ctypes.data_as(ctypes.c_void_p)
            self._keep.append(f)
        return s
