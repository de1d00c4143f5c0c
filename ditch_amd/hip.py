"""ctypes binding of libditch_hip.so for Python callers.

`Device` mirrors the operations of compute.zig's VTable (compute.zig:90-117)
with numpy arrays; `Model` wraps the resident forward. Every call goes to the
HIP library; a failing status raises `DeviceError` (there is no CPU path
here, the reference's own tensor.zig is the CPU path of a Zig caller).
"""
import ctypes
import os

import numpy as np

from . import abi, load_library
from .weights import HostWeight


class DeviceError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"{abi.STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class Device:
    def __init__(self, index=0):
        self.lib = load_library()
        err = ctypes.create_string_buffer(512)
        self.h = self.lib.ditch_hip_open(index, err, 512)
        if not self.h:
            raise DeviceError(abi.DEVICE_FAILED, err.value.decode())

    def close(self):
        if self.h:
            self.lib.ditch_hip_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def name(self):
        return self.lib.ditch_hip_name(self.h).decode()

    @property
    def stream(self):
        return self.lib.ditch_hip_stream(self.h)

    def check(self, rc):
        if rc != abi.OK:
            raise DeviceError(rc, self.lib.ditch_hip_last_error(self.h).decode())

    def sync(self):
        self.check(self.lib.ditch_hip_sync(self.h))

    def set_residency(self, budget_bytes, weights_stable=True):
        """compute.Residency for the per-call entry points (0: upload, compute, drop)."""
        self.check(self.lib.ditch_hip_set_residency(self.h, int(budget_bytes), 1 if weights_stable else 0))

    def residency_stats(self):
        st = abi.ResidencyStats()
        self.check(self.lib.ditch_hip_residency_stats(self.h, ctypes.byref(st)))
        return {k: getattr(st, k) for k, _ in abi.ResidencyStats._fields_}

    def forget_weights(self):
        self.lib.ditch_hip_forget_weights(self.h)

    # VTable -----------------------------------------------------------------

    def matmulT(self, x, w: HostWeight):
        x = _f32(x)
        n = x.shape[0]
        out = np.empty((n, w.rows), dtype=np.float32)
        self.check(self.lib.ditch_hip_matmulT(self.h, _p(out), _p(x), n, w.ref()))
        return out

    def matvecTMulti(self, w: HostWeight, y):
        y = _f32(y)
        q = y.shape[0]
        out = np.empty((q, w.cols), dtype=np.float32)
        self.check(self.lib.ditch_hip_matvecTMulti(self.h, _p(out), w.ref(), _p(y), q))
        return out

    def rowNorms(self, w: HostWeight):
        out = np.empty(w.rows, dtype=np.float32)
        self.check(self.lib.ditch_hip_rowNorms(self.h, _p(out), w.ref()))
        return out

    def attentionScores(self, q, k, n_keys, stride, scale):
        q, k = _f32(q), _f32(k)
        out = np.empty(n_keys, dtype=np.float32)
        self.check(self.lib.ditch_hip_attentionScores(self.h, _p(out), n_keys, _p(q), q.size, _p(k), stride, scale))
        return out

    def attentionValues(self, scores, v, vd, stride):
        scores, v = _f32(scores), _f32(v)
        out = np.empty(vd, dtype=np.float32)
        self.check(self.lib.ditch_hip_attentionValues(self.h, _p(out), vd, _p(scores), scores.size, _p(v), stride))
        return out

    def gatedActivation(self, act, gate, up, n, length, in_stride, out_stride, out=None):
        gate = _f32(gate)
        up = None if up is None else _f32(up)
        if out is None:
            out = np.zeros(((n - 1) * out_stride + length,), dtype=np.float32)
        self.check(self.lib.ditch_hip_gatedActivation(self.h, act, _p(out), _p(gate), _p(up), n, length,
                                                      in_stride, out_stride))
        return out

    def rmsnormRows(self, x, weight, eps, gemma_style=False):
        x = _f32(x)
        n, length = x.shape
        w = None if weight is None else _f32(weight)
        out = np.empty_like(x)
        self.check(self.lib.ditch_hip_rmsnormRows(self.h, _p(out), _p(x), _p(w), 0 if w is None else w.size, n,
                                                  length, eps, int(gemma_style)))
        return out

    def layernormRows(self, x, weight, bias, eps, one_plus=False):
        x = _f32(x)
        n, length = x.shape
        w = None if weight is None else _f32(weight)
        b = None if bias is None else _f32(bias)
        out = np.empty_like(x)
        self.check(self.lib.ditch_hip_layernormRows(self.h, _p(out), _p(x), _p(w), 0 if w is None else w.size,
                                                    _p(b), n, length, eps, int(one_plus)))
        return out

    def softmaxRows(self, x):
        x = _f32(x).copy()
        n, length = x.shape
        self.check(self.lib.ditch_hip_softmaxRows(self.h, _p(x), n, length))
        return x

    def ropeRows(self, x, cos_t, sin_t, pos, style):
        x = _f32(x).copy()
        n, dim = x.shape
        cos_t, sin_t = _f32(cos_t), _f32(sin_t)
        pos = np.ascontiguousarray(pos, dtype=np.uint32)
        self.check(self.lib.ditch_hip_ropeRows(self.h, _p(x), n, dim, _p(cos_t), _p(sin_t), cos_t.shape[0],
                                               cos_t.shape[1], _p(pos), style))
        return x

    # extensions ---------------------------------------------------------------

    def dequant(self, w: HostWeight, row0=0, nrows=None):
        nrows = w.rows - row0 if nrows is None else nrows
        bf16 = w.dtype in (abi.FP8, abi.MXFP4, abi.MXFP4_T, abi.INT_PACKED)
        out = np.empty((nrows, w.cols), dtype=np.uint16 if bf16 else np.float32)
        self.check(self.lib.ditch_hip_dequant(self.h, _p(out), w.ref(), row0, nrows))
        return out

    def upload(self, w: HostWeight):
        t = self.lib.ditch_hip_upload(self.h, w.ref())
        if not t:
            raise DeviceError(abi.DEVICE_FAILED, self.lib.ditch_hip_last_error(self.h).decode())
        return Tensor(self, t, w)

    def edit_delta(self, w: HostWeight, v, weight):
        v = _f32(v)
        k = v.shape[0]
        a = np.empty((k, w.cols), dtype=np.float32)
        b = np.empty((w.rows, k), dtype=np.float32)
        self.check(self.lib.ditch_hip_edit_delta(self.h, _p(a), _p(b), w.ref(), _p(v), k, weight))
        return a, b

    def edit_delta_ex(self, w: HostWeight, v, weight, mode="full", lora_rank=3, seed=0, ablate=False):
        """abliterate.computeDelta in any mode: (a [rank][cols], b [rows][rank])."""
        v = _f32(v)
        k = v.shape[0]
        o = abi.EditOptions(abi.ROWNORM[mode], lora_rank, seed, int(ablate))
        rank = self.lib.ditch_hip_edit_rank(w.rows, w.cols, k, ctypes.byref(o))
        a = np.empty((rank, w.cols), dtype=np.float32)
        b = np.empty((w.rows, rank), dtype=np.float32)
        self.check(self.lib.ditch_hip_edit_delta_ex(self.h, _p(a), a.size, _p(b), b.size, w.ref(), _p(v), k, weight,
                                                    ctypes.byref(o)))
        return a, b

    def logSoftmaxRows(self, x):
        x = _f32(x)
        out = np.empty_like(x)
        self.check(self.lib.ditch_hip_logSoftmaxRows(self.h, _p(out), _p(x), x.shape[0], x.shape[1]))
        return out

    def klRows(self, base_logprobs, trial_logits):
        b, t = _f32(base_logprobs), _f32(trial_logits)
        out = np.empty(b.shape[0], dtype=np.float64)
        self.check(self.lib.ditch_hip_klRows(self.h, _p(out), _p(b), _p(t), b.shape[0], b.shape[1]))
        return out

    def logSoftmaxRows_device(self, d_out, d_x, n, length, stream=None):
        self.check(self.lib.ditch_hip_logSoftmaxRows_device(self.h, d_out, d_x, n, length, stream))

    def klRows_device(self, d_kl, d_base, d_trial, n, vocab, stream=None):
        self.check(self.lib.ditch_hip_klRows_device(self.h, d_kl, d_base, d_trial, n, vocab, stream))


class Tensor:
    """A weight resident in HBM (ditch_hip_upload)."""

    def __init__(self, dev, handle, host):
        self.dev, self.handle, self.rows, self.cols = dev, handle, host.rows, host.cols
        self.dtype = host.dtype

    @property
    def nbytes(self):
        return self.dev.lib.ditch_hip_tensor_bytes(self.handle)

    def free(self):
        if self.handle:
            self.dev.lib.ditch_hip_tensor_free(self.dev.h, self.handle)
            self.handle = None

    def matmul_device(self, d_out, d_x, n, d_bias=None, accumulate=False, stream=None, out_bytes=None,
                      x_bytes=None):
        """out_bytes / x_bytes: the device buffers' lengths (default: exactly n rows)."""
        ob = n * self.rows * 4 if out_bytes is None else out_bytes
        xb = n * self.cols * 4 if x_bytes is None else x_bytes
        self.dev.check(self.dev.lib.ditch_hip_matmulT_device(self.dev.h, d_out, ob, d_x, xb, n, self.handle, d_bias,
                                                             int(accumulate), stream))

    def matmul_device_noalloc(self, d_out, d_x, n, d_bias=None, accumulate=False, stream=None, out_bytes=None,
                              x_bytes=None):
        """matmul_device with its scratch in the library's static array
        (ditch_hip_matmulT_device_noalloc): allocates no device memory."""
        ob = n * self.rows * 4 if out_bytes is None else out_bytes
        xb = n * self.cols * 4 if x_bytes is None else x_bytes
        self.dev.check(self.dev.lib.ditch_hip_matmulT_device_noalloc(self.dev.h, d_out, ob, d_x, xb, n, self.handle,
                                                                     d_bias, int(accumulate), stream))

    def frag_bytes(self, n):
        """Bytes of the activation fragments of n rows for products over this
        tensor (0: the large-batch product does not take it)."""
        return self.dev.lib.ditch_hip_frag_bytes(self.handle, n)

    def split_device(self, d_frags, frag_bytes, d_x, n, stream=None):
        """Writes the fragments of d_x [n][cols] (device f32) for this tensor."""
        self.dev.check(self.dev.lib.ditch_hip_split_device(self.dev.h, d_frags, frag_bytes, d_x, n, self.handle,
                                                           stream))

    def matmul_frags_device(self, d_out, d_frags, n, d_bias=None, accumulate=False, stream=None, out_bytes=None,
                            frag_bytes=None):
        """The large-batch product on activation fragments (ditch_hip_split_device)."""
        ob = n * self.rows * 4 if out_bytes is None else out_bytes
        fb = self.frag_bytes(n) if frag_bytes is None else frag_bytes
        self.dev.check(self.dev.lib.ditch_hip_matmulT_frags_device(self.dev.h, d_out, ob, d_frags, fb, n, self.handle,
                                                                   d_bias, int(accumulate), stream))

    def glu_frag_bytes(self, up, n):
        """Bytes of the fused gate/up product's output fragments (0: not taken)."""
        return self.dev.lib.ditch_hip_glu_frag_bytes(self.handle, up.handle, n)

    def glu_device(self, up, d_out_frags, out_bytes, d_frags, frag_bytes, n, act=0, stream=None):
        """act(x self^T) * (x up^T) on fragments split for this tensor, written
        as the down projection's input fragments (ditch_hip_glu_device)."""
        self.dev.check(self.dev.lib.ditch_hip_glu_device(self.dev.h, d_out_frags, out_bytes, d_frags, frag_bytes, n,
                                                         self.handle, up.handle, act, stream))

    def dequant_device(self, d_out, out_bytes, row0, nrows):
        self.dev.check(self.dev.lib.ditch_hip_tensor_dequant(self.dev.h, d_out, out_bytes, self.handle, row0, nrows))


class _LoadedSpec:
    """The configuration of a model read from disk (what Model needs of a spec)."""

    def __init__(self, config):
        self.config = config


class Model:
    """A resident model (ditch_hip_model) built from a ModelSpec."""

    def __init__(self, dev: Device, spec, expert_cache_bytes=0):
        """expert_cache_bytes > 0: routed experts stream from pinned host memory
        through a device cache of that many bytes (ditch_hip_model_set_expert_cache)."""
        self.dev = dev
        self.spec = spec
        self.cfg = spec.config_struct()
        self.h = dev.lib.ditch_hip_model_create(dev.h, ctypes.byref(self.cfg))
        if not self.h:
            raise DeviceError(abi.DEVICE_FAILED, dev.lib.ditch_hip_last_error(dev.h).decode())
        if expert_cache_bytes:
            dev.check(dev.lib.ditch_hip_model_set_expert_cache(self.h, int(expert_cache_bytes)))
        for (layer, slot, expert), w in spec.tensors.items():
            dev.check(dev.lib.ditch_hip_model_set(self.h, layer, slot, expert, w.ref()))

    @classmethod
    def load(cls, dev: Device, path, expert_cache_bytes=0):
        """A model read from a checkpoint on disk (ditch_hip_model_load): a
        Hugging Face directory or a GGUF file."""
        h = dev.lib.ditch_hip_model_load(dev.h, os.fsencode(path), int(expert_cache_bytes))
        if not h:
            raise DeviceError(abi.DEVICE_FAILED, dev.lib.ditch_hip_last_error(dev.h).decode())
        m = cls.__new__(cls)
        m.dev, m.h = dev, h
        cfg = abi.ModelConfig()
        dev.check(dev.lib.ditch_hip_model_get_config(h, ctypes.byref(cfg)))
        m.cfg = cfg
        m.spec = _LoadedSpec({name: getattr(cfg, name) for name, _ in cfg._fields_ if name not in ("moe_layers",
                                                                                                   "rope_factors")})
        return m

    def expert_cache_stats(self):
        st = abi.ExpertCacheStats()
        self.dev.check(self.dev.lib.ditch_hip_model_expert_cache_stats(self.h, ctypes.byref(st)))
        return {name: getattr(st, name) for name, _ in st._fields_}

    def hot_experts(self):
        """[(layer, expert, uses)], most used first (ExpertCache.hotExperts)."""
        n = ctypes.c_uint64(0)
        self.dev.check(self.dev.lib.ditch_hip_model_hot_experts(self.h, None, 0, ctypes.byref(n)))
        arr = (abi.HotExpert * max(n.value, 1))()
        self.dev.check(self.dev.lib.ditch_hip_model_hot_experts(self.h, arr, n.value, ctypes.byref(n)))
        return [(h.layer, h.expert, h.uses) for h in arr[:n.value]]

    def warm_experts(self, hot):
        """ExpertCache.warm: copies the hottest experts of `hot` in; returns how many."""
        arr = (abi.HotExpert * max(len(hot), 1))(*[abi.HotExpert(l, e, u) for l, e, u in hot])
        w = ctypes.c_uint64(0)
        self.dev.check(self.dev.lib.ditch_hip_model_warm_experts(self.h, arr, len(hot), ctypes.byref(w)))
        return w.value

    def free(self):
        if self.h:
            self.dev.lib.ditch_hip_model_free(self.h)
            self.h = None

    @property
    def nbytes(self):
        return self.dev.lib.ditch_hip_model_bytes(self.h)

    def set_delta(self, layer, slot, expert, a, b):
        a, b = _f32(a), _f32(b)
        rank = a.shape[0]
        self.dev.check(self.dev.lib.ditch_hip_model_set_delta(self.h, layer, slot, expert, rank, _p(a), _p(b)))

    def edit(self, layer, slot, expert, v, weight):
        v = _f32(v)
        self.dev.check(self.dev.lib.ditch_hip_model_edit(self.h, layer, slot, expert, _p(v), v.shape[0], weight))

    @staticmethod
    def edit_targets(targets, k):
        """The ditch_edit_target array of [(layer, slot, expert, v [k][rows]
        f32 array, weight)] (with the arrays it points into)."""
        keep = {}
        arr = (abi.EditTarget * len(targets))()
        for i, (layer, slot, expert, v, weight) in enumerate(targets):
            if id(v) not in keep:
                keep[id(v)] = _f32(v)
            vv = keep[id(v)]
            assert vv.shape[0] == k
            arr[i] = abi.EditTarget(layer, slot, expert, weight, vv.ctypes.data)
        return (arr, list(keep.values()), k)

    def edit_batch(self, targets, k=None):
        """One call edits every target (ditch_hip_model_edit_batch): a list as
        for edit_targets, or what edit_targets returned."""
        arr, keep, k = targets if isinstance(targets, tuple) else self.edit_targets(targets, k)
        self.dev.check(self.dev.lib.ditch_hip_model_edit_batch(self.h, ctypes.byref(arr), len(arr), k))

    def edit_ex(self, layer, slot, expert, v, weight, mode="full", lora_rank=3, seed=0, ablate=False):
        v = _f32(v)
        o = abi.EditOptions(abi.ROWNORM[mode], lora_rank, seed, int(ablate))
        self.dev.check(self.dev.lib.ditch_hip_model_edit_ex(self.h, layer, slot, expert, _p(v), v.shape[0], weight,
                                                            ctypes.byref(o)))

    def reset_deltas(self):
        self.dev.check(self.dev.lib.ditch_hip_model_reset_deltas(self.h))

    def forward(self, tokens, rows, capture_rows=(), logit_rows=()):
        """tokens u32[n]; rows [(b, pos)]; returns (residuals [(L+1)][nc][hidden], logits [nl][vocab])."""
        tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
        rows_a = np.ascontiguousarray(rows, dtype=np.uint32).reshape(-1, 2)
        cap = np.ascontiguousarray(capture_rows, dtype=np.uint64)
        lr = np.ascontiguousarray(logit_rows, dtype=np.uint64)
        c = self.spec.config
        res = np.empty((c["layers"] + 1, cap.size, c["hidden"]), dtype=np.float32)
        logits = np.empty((lr.size, c["vocab"]), dtype=np.float32)
        self.dev.check(self.dev.lib.ditch_hip_forward(
            self.h, _p(tokens), _p(rows_a), tokens.size, _p(cap) if cap.size else None, cap.size,
            _p(res) if cap.size else None, _p(lr) if lr.size else None, lr.size,
            _p(logits) if lr.size else None))
        return res, logits

    def forward_device(self, d_tokens, d_rows, n, n_prompts, max_len, d_capture, n_capture, d_res, d_logit_rows,
                       n_logit, d_logits, res_bytes=None, logit_bytes=None):
        """Device buffers throughout; the KV cache holds n_prompts x max_len
        positions. res_bytes / logit_bytes default to exactly the outputs' sizes."""
        c = self.spec.config
        rb = (c["layers"] + 1) * n_capture * c["hidden"] * 4 if res_bytes is None else res_bytes
        lb = n_logit * c["vocab"] * 4 if logit_bytes is None else logit_bytes
        self.dev.check(self.dev.lib.ditch_hip_forward_device(self.h, d_tokens, d_rows, n, n_prompts, max_len,
                                                             d_capture, n_capture, d_res, rb, d_logit_rows, n_logit,
                                                             d_logits, lb))

    def kv_cache(self, n_prompts, max_len):
        """A persistent KV cache (ditch_hip_kv_cache_create); free it with
        kv_cache_free before the model."""
        c = self.dev.lib.ditch_hip_kv_cache_create(self.h, n_prompts, max_len)
        if not c:
            raise DeviceError(abi.DEVICE_FAILED, self.dev.lib.ditch_hip_last_error(self.dev.h).decode())
        return c

    def kv_cache_free(self, c):
        self.dev.lib.ditch_hip_kv_cache_free(c)

    def generate(self, cache, prompts, max_new_tokens, eos=(), sampler=None, first_logits=False):
        """generateKeep: prompts = list of token-id lists; sampler = None
        (greedy), a dict (a new Sampler) or an abi.Sampler (advanced in place
        by its draws); returns (list of generated token lists, first-token
        logits [prompts][vocab] or None)."""
        lens = np.array([len(p) for p in prompts], dtype=np.uint64)
        toks = np.ascontiguousarray(np.concatenate([np.asarray(p, dtype=np.uint32) for p in prompts]))
        B = len(prompts)
        out = np.zeros((B, max_new_tokens), dtype=np.uint32)
        out_lens = np.zeros(B, dtype=np.uint64)
        eos_a = np.ascontiguousarray(eos, dtype=np.uint32)
        fl = np.empty((B, self.spec.config["vocab"]), dtype=np.float32) if first_logits else None
        smp = sampler
        if isinstance(sampler, dict):
            smp = abi.sampler(self.dev.lib, sampler.get("seed", 0), sampler.get("temperature", 1.0),
                              sampler.get("top_k", 50), sampler.get("top_p", 0.95))
        self.dev.check(self.dev.lib.ditch_hip_generate(
            self.h, cache, _p(toks), _p(lens), B, max_new_tokens, _p(eos_a) if eos_a.size else None, eos_a.size,
            ctypes.byref(smp) if smp is not None else None, _p(out), _p(out_lens), _p(fl) if fl is not None else None))
        return [list(out[b, :int(out_lens[b])]) for b in range(B)], fl

    def path_stats(self):
        st = abi.PathStats()
        self.dev.check(self.dev.lib.ditch_hip_model_path_stats(self.h, ctypes.byref(st)))
        return {name: getattr(st, name) for name, _ in st._fields_}
