"""ctypes binding of oracle/libcpu_ref.so (the C restatement in cpu_ref.c).

TEST INFRASTRUCTURE ONLY: see oracle/__init__.py.
"""
import ctypes
import os
import subprocess

import numpy as np

from ditch_amd import abi

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libcpu_ref.so")

P, U64, I32, U32, FLT = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int32, ctypes.c_uint32, ctypes.c_float
SZ = ctypes.c_size_t
PROTOS = {
    "ref_f32_to_bf16": (ctypes.c_uint16, [FLT]),
    "ref_f16_to_f32": (FLT, [ctypes.c_uint16]),
    "ref_f32_to_f16": (ctypes.c_uint16, [FLT]),
    "ref_fp8_value": (FLT, [ctypes.c_uint8, ctypes.c_int]),
    "ref_e8m0_scale": (FLT, [ctypes.c_uint8]),
    "ref_f32_to_bf16_array": (None, [P, P, SZ]),
    "ref_gguf_dequant": (ctypes.c_int, [ctypes.c_int, P, P, SZ]),
    "ref_quantize_q8_0": (None, [P, SZ, P]),
    "ref_dequant_rows": (ctypes.c_int, [P, SZ, SZ, P]),
    "ref_dot": (FLT, [P, P, SZ]),
    "ref_matmulT": (ctypes.c_int, [P, P, SZ, P, SZ, P, P, ctypes.c_int]),
    "ref_matvecTMulti": (ctypes.c_int, [P, P, P, SZ, ctypes.c_int]),
    "ref_rowNorms": (ctypes.c_int, [P, P, ctypes.c_int]),
    "ref_attention_scores": (None, [P, SZ, P, SZ, P, SZ, FLT]),
    "ref_attention_values": (None, [P, SZ, P, SZ, P, SZ]),
    "ref_rmsnorm": (None, [P, P, P, SZ, SZ, FLT, ctypes.c_int]),
    "ref_layernorm": (None, [P, P, P, SZ, P, SZ, FLT, ctypes.c_int]),
    "ref_softmax_inplace": (None, [P, SZ]),
    "ref_log_softmax": (None, [P, P, SZ]),
    "ref_exp_cephes": (FLT, [FLT]),
    "ref_gated_activation": (None, [U32, P, P, P, SZ, SZ, SZ, SZ]),
    "ref_rope_rows": (None, [P, SZ, SZ, P, P, SZ, P, U32]),
    "ref_fill_rope": (ctypes.c_int, [P, P, P]),
    "ref_kl_row": (ctypes.c_double, [P, P, SZ]),
    "ref_edit_delta": (ctypes.c_int, [P, P, P, P, SZ, FLT, ctypes.c_int]),
    "ref_model_create": (P, [P]),
    "ref_model_free": (None, [P]),
    "ref_model_set": (ctypes.c_int, [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P]),
    "ref_model_set_delta": (ctypes.c_int, [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, SZ, P, P]),
    "ref_model_edit": (ctypes.c_int, [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, SZ, FLT]),
    "ref_forward": (ctypes.c_int, [P, P, P, SZ, P, SZ, P, P, SZ, P]),
    "ref_model_limit_layers": (None, [P, SZ, SZ]),
    "ref_set_threads": (None, [P, ctypes.c_int]),
    "ref_model_keep_packed": (None, [P, ctypes.c_int]),
    "ref_last_error": (ctypes.c_char_p, []),
    "ref_residual_reduce": (ctypes.c_int, [P, SZ, SZ, SZ, P, P, SZ, FLT, P, P, P]),
    "ref_directions": (None, [P, P, P, SZ, SZ, ctypes.c_int]),
    "ref_orthonormalize": (None, [P, SZ, SZ]),
    "ref_sketch_add": (None, [P, P, P, SZ, P, P, SZ, SZ, SZ]),
    "ref_symmetric_eigen": (None, [P, P, SZ]),
    "ref_basis": (ctypes.c_int, [P, P, P, SZ, SZ, SZ, ctypes.c_int, P, P, SZ]),
    "ref_edit_gaussian": (None, [P, SZ, U64]),
    "ref_zig_init": (None, [P, U64]),
    "ref_zig_draws": (None, [P, SZ, U64, ctypes.c_int]),
    "ref_zig_norm_tables": (None, [P, P]),
    "ref_sampler_pick": (None, [P, P, SZ, SZ, P, FLT, SZ, FLT]),
    "ref_jacobi_f32": (None, [P, P, SZ]),
    "ref_edit_delta_ex": (ctypes.c_int, [P, P, P, P, P, SZ, FLT, ctypes.c_int, SZ, U64, ctypes.c_int, ctypes.c_int]),
}

_lib = None


def build(path=LIB, arch=None):
    """Compiles the oracle with its Makefile (gcc)."""
    cmd = ["make", "-s", "-C", HERE, f"OUT={path}"]
    if arch:
        cmd.append(f"ARCH={arch}")
    subprocess.run(cmd, check=True)
    return path


def load(path=LIB):
    global _lib
    if _lib is not None and path == LIB:
        return _lib
    if not os.path.exists(path):
        build(path)
    lib = ctypes.CDLL(path)
    for name, (res, args) in PROTOS.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    if path == LIB:
        _lib = lib
    return lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class OracleError(RuntimeError):
    pass


class Ref:
    """The oracle's functions over numpy arrays."""

    def __init__(self, path=LIB, threads=8):
        self.lib = load(path)
        self.threads = threads

    def _check(self, rc):
        if rc != 0:
            raise OracleError(self.lib.ref_last_error().decode())

    def f32_to_bf16(self, a):
        a = np.ascontiguousarray(a, dtype=np.float32)
        out = np.empty(a.shape, dtype=np.uint16)
        self.lib.ref_f32_to_bf16_array(_p(a), _p(out), a.size)
        return out

    def dequant(self, w, row0=0, nrows=None):
        nrows = w.rows - row0 if nrows is None else nrows
        bf16 = w.dtype in (abi.FP8, abi.MXFP4, abi.MXFP4_T, abi.INT_PACKED)
        out = np.empty((nrows, w.cols), dtype=np.uint16 if bf16 else np.float32)
        self._check(self.lib.ref_dequant_rows(w.ref(), row0, nrows, _p(out)))
        return out

    def gguf_dequant(self, dtype, raw, n):
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        out = np.empty(n, dtype=np.float32)
        self._check(self.lib.ref_gguf_dequant(dtype, _p(raw), _p(out), n))
        return out

    def quantize_q8_0(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        out = np.empty(x.size // 32 * 34, dtype=np.uint8)
        self.lib.ref_quantize_q8_0(_p(x), x.size, _p(out))
        return out

    def matmulT(self, x, w, delta=None):
        x = np.ascontiguousarray(x, dtype=np.float32)
        n = x.shape[0]
        out = np.empty((n, w.rows), dtype=np.float32)
        a = b = None
        rank = 0
        if delta is not None:
            a, b = (np.ascontiguousarray(t, dtype=np.float32) for t in delta)
            rank = a.shape[0]
        self._check(self.lib.ref_matmulT(_p(out), _p(x), n, w.ref(), rank, _p(a), _p(b), self.threads))
        return out

    def matvecTMulti(self, w, y):
        y = np.ascontiguousarray(y, dtype=np.float32)
        out = np.empty((y.shape[0], w.cols), dtype=np.float32)
        self._check(self.lib.ref_matvecTMulti(_p(out), w.ref(), _p(y), y.shape[0], self.threads))
        return out

    def rowNorms(self, w):
        out = np.empty(w.rows, dtype=np.float32)
        self._check(self.lib.ref_rowNorms(_p(out), w.ref(), self.threads))
        return out

    def rmsnorm_rows(self, x, w, eps, gemma=False):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = None if w is None else np.ascontiguousarray(w, dtype=np.float32)
        out = np.empty_like(x)
        for i in range(x.shape[0]):
            self.lib.ref_rmsnorm(_p(out[i]), _p(x[i]), _p(w), 0 if w is None else w.size, x.shape[1], eps, int(gemma))
        return out

    def softmax_rows(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32).copy()
        for i in range(x.shape[0]):
            self.lib.ref_softmax_inplace(_p(x[i]), x.shape[1])
        return x

    def log_softmax_rows(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty_like(x)
        for i in range(x.shape[0]):
            self.lib.ref_log_softmax(_p(out[i]), _p(x[i]), x.shape[1])
        return out

    def gated(self, act, gate, up, n, length, in_stride, out_stride):
        gate = np.ascontiguousarray(gate, dtype=np.float32)
        up = None if up is None else np.ascontiguousarray(up, dtype=np.float32)
        out = np.zeros(((n - 1) * out_stride + length,), dtype=np.float32)
        self.lib.ref_gated_activation(act, _p(out), _p(gate), _p(up), n, length, in_stride, out_stride)
        return out

    def rope_rows(self, x, cos_t, sin_t, pos, style):
        x = np.ascontiguousarray(x, dtype=np.float32).copy()
        cos_t = np.ascontiguousarray(cos_t, dtype=np.float32)
        sin_t = np.ascontiguousarray(sin_t, dtype=np.float32)
        pos = np.ascontiguousarray(pos, dtype=np.uint32)
        self.lib.ref_rope_rows(_p(x), x.shape[0], x.shape[1], _p(cos_t), _p(sin_t), cos_t.shape[1], _p(pos), style)
        return x

    def kl_rows(self, base_logprobs, trial_logits):
        b = np.ascontiguousarray(base_logprobs, dtype=np.float32)
        t = np.ascontiguousarray(trial_logits, dtype=np.float32)
        return np.array([self.lib.ref_kl_row(_p(b[i]), _p(t[i]), b.shape[1]) for i in range(b.shape[0])])

    def edit_delta(self, w, v, weight):
        v = np.ascontiguousarray(v, dtype=np.float32)
        k = v.shape[0]
        a = np.empty((k, w.cols), dtype=np.float32)
        b = np.empty((w.rows, k), dtype=np.float32)
        self._check(self.lib.ref_edit_delta(_p(a), _p(b), w.ref(), _p(v), k, weight, self.threads))
        return a, b

    def fill_rope(self, spec):
        cfg = spec.config_struct()
        half = spec.config["rotary_dim"] // 2
        cos_t = np.zeros((spec.config["rope_len"], half), dtype=np.float32)
        sin_t = np.zeros_like(cos_t)
        self.lib.ref_fill_rope(ctypes.byref(cfg), _p(cos_t), _p(sin_t))
        return cos_t, sin_t


    # -- direction pipeline (engine.zig:414-431, abliterate.zig:88-109,
    #    directions.zig:80-134, 371-500) --------------------------------

    def residual_reduce(self, res, first, take, q, sum_=None, sq=None):
        """res [entries][n_capture][hidden]; returns vout [prompts][entries][hidden]
        and adds into sum_/sq ([entries][hidden] f64) when given."""
        res = np.ascontiguousarray(res, dtype=np.float32)
        E, NC, H = res.shape
        first = np.ascontiguousarray(first, dtype=np.uint32)
        take = np.ascontiguousarray(take, dtype=np.uint32)
        vout = np.empty((first.size, E, H), dtype=np.float32)
        self._check(self.lib.ref_residual_reduce(_p(res), E, NC, H, _p(first), _p(take), first.size, q, _p(vout),
                                                 _p(sum_) if sum_ is not None else None,
                                                 _p(sq) if sq is not None else None))
        return vout

    def directions(self, good, bad, orthogonalize):
        good, bad = _f32(good), _f32(bad)
        out = np.empty_like(good)
        self.lib.ref_directions(_p(out), _p(good), _p(bad), good.shape[0], good.shape[1], int(orthogonalize))
        return out

    def orthonormalize(self, vecs):
        v = np.array(vecs, dtype=np.float32, order="C")
        self.lib.ref_orthonormalize(_p(v), v.shape[0], v.shape[1])
        return v

    def sketch_add(self, y, w, omega, center, v):
        omega, center, v = _f32(omega), _f32(center), _f32(v)
        P_, E, H = v.shape
        self.lib.ref_sketch_add(_p(y), _p(w), _p(omega), omega.shape[0], _p(center), _p(v), P_, E, H)

    def symmetric_eigen(self, m):
        a = np.array(m, dtype=np.float64, order="C")
        vecs = np.empty_like(a)
        self.lib.ref_symmetric_eigen(_p(a), _p(vecs), a.shape[0])
        return a, vecs

    def basis(self, first, good, k, orthogonalize, y, w):
        first, good = _f32(first), _f32(good)
        E, H = first.shape
        out = np.empty((E, k, H), dtype=np.float32)
        m = w.shape[1]
        self._check(self.lib.ref_basis(_p(out), _p(first), _p(good), E, H, k, int(orthogonalize),
                                       _p(np.ascontiguousarray(y)), _p(np.ascontiguousarray(w)), m))
        return out


    def edit_gaussian(self, n, seed):
        out = np.empty(n, dtype=np.float32)
        self.lib.ref_edit_gaussian(_p(out), n, seed)
        return out

    def zig_draws(self, n, seed, kind):
        """n draws of Zig's DefaultPrng.init(seed): kind 'u64' (int(u64)),
        'f64' (float(f64)) or 'norm' (floatNorm(f64))."""
        k = {"u64": 0, "f64": 1, "norm": 2}[kind]
        out = np.empty(n, dtype=np.uint64 if k == 0 else np.float64)
        self.lib.ref_zig_draws(_p(out), n, seed, k)
        return out

    def zig_norm_tables(self):
        x, f = np.empty(257), np.empty(257)
        self.lib.ref_zig_norm_tables(_p(x), _p(f))
        return x, f

    def sampler_init(self, seed):
        """Sampler.init's DefaultPrng state (4 x u64)."""
        st = np.empty(4, dtype=np.uint64)
        self.lib.ref_zig_init(_p(st), seed)
        return st

    def sampler_pick(self, logits, state, temperature, top_k, top_p):
        """Sampler.pick of each row in order; `state` advances in place."""
        logits = _f32(logits)
        n, V = logits.shape
        out = np.empty(n, dtype=np.uint32)
        self.lib.ref_sampler_pick(_p(out), _p(logits), n, V, _p(state), temperature, top_k, top_p)
        return out

    def jacobi_f32(self, m):
        a = np.array(m, dtype=np.float32, order="C")
        vecs = np.empty_like(a)
        self.lib.ref_jacobi_f32(_p(a), _p(vecs), a.shape[0])
        return a, vecs

    def edit_delta_ex(self, w, v, weight, mode=0, lora_rank=3, seed=0, ablate=False):
        """abliterate.computeDelta: (a [rank][cols], b [rows][rank]); mode 0 none,
        1 pre, 2 full."""
        v = _f32(v)
        k = v.shape[0]
        cap = max(lora_rank, k) + k
        a = np.empty((cap, w.cols), dtype=np.float32)
        b = np.empty((w.rows * cap,), dtype=np.float32)
        rank = ctypes.c_size_t()
        self._check(self.lib.ref_edit_delta_ex(_p(a), _p(b), ctypes.byref(rank), w.ref(), _p(v), k, weight, mode,
                                               lora_rank, seed, int(ablate), self.threads))
        r = rank.value
        return a[:r].copy(), b[:w.rows * r].reshape(w.rows, r).copy()


class RefModel:
    """The oracle's model.forward over a ModelSpec."""

    def __init__(self, spec, path=LIB, threads=8, keep_packed=False):
        """keep_packed: FP8 / MXFP4 / INT weights stay in the spec's packed
        arrays (held by this object) and are decoded row by row at use, as
        the reference's streamed mode does, instead of once to bf16."""
        self.lib = load(path)
        self.spec = spec
        self.cfg = spec.config_struct()
        self.h = self.lib.ref_model_create(ctypes.byref(self.cfg))
        self.lib.ref_set_threads(self.h, threads)
        self.lib.ref_model_keep_packed(self.h, int(keep_packed))
        for (layer, slot, expert), w in spec.tensors.items():
            if self.lib.ref_model_set(self.h, layer, slot, expert, w.ref()) != 0:
                raise OracleError(self.lib.ref_last_error().decode())

    def free(self):
        if self.h:
            self.lib.ref_model_free(self.h)
            self.h = None

    def __del__(self):
        self.free()

    def limit_layers(self, first, count):
        self.lib.ref_model_limit_layers(self.h, first, count)

    def set_delta(self, layer, slot, expert, a, b):
        a = np.ascontiguousarray(a, dtype=np.float32)
        b = np.ascontiguousarray(b, dtype=np.float32)
        if self.lib.ref_model_set_delta(self.h, layer, slot, expert, a.shape[0], _p(a), _p(b)) != 0:
            raise OracleError(self.lib.ref_last_error().decode())

    def edit(self, layer, slot, expert, v, weight):
        v = np.ascontiguousarray(v, dtype=np.float32)
        if self.lib.ref_model_edit(self.h, layer, slot, expert, _p(v), v.shape[0], weight) != 0:
            raise OracleError(self.lib.ref_last_error().decode())

    def forward(self, tokens, rows, capture_rows=(), logit_rows=()):
        tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
        rows_a = np.ascontiguousarray(rows, dtype=np.uint32).reshape(-1, 2)
        cap = np.ascontiguousarray(capture_rows, dtype=np.uint64)
        lr = np.ascontiguousarray(logit_rows, dtype=np.uint64)
        c = self.spec.config
        res = np.empty((c["layers"] + 1, cap.size, c["hidden"]), dtype=np.float32)
        logits = np.empty((lr.size, c["vocab"]), dtype=np.float32)
        rc = self.lib.ref_forward(self.h, _p(tokens), _p(rows_a), tokens.size, _p(cap) if cap.size else None,
                                  cap.size, _p(res) if cap.size else None, _p(lr) if lr.size else None, lr.size,
                                  _p(logits) if lr.size else None)
        if rc != 0:
            raise OracleError(self.lib.ref_last_error().decode())
        return res, logits
