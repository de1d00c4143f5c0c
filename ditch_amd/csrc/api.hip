// api.hip — the extern "C" entry points of include/ditch_hip.h.
//
// Every function catches everything (nothing unwinds across the boundary),
// returns a status code and leaves a message in ditch_hip_last_error; a NULL
// context fails cleanly (src/metal/shim.h:6-7 conventions).
#include <string.h>

#include <memory>
#include <mutex>

#include "internal.h"
#include "model.h"

namespace ditch {
void dequant_to_host(ditch_hip *h, void *out, const ditch_weight *w, uint64_t row0, uint64_t nrows);
ditch_hip_model *model_create(ditch_hip *h, const ditch_model_config *cfg);
void model_set(ditch_hip_model *m, int layer, int slot, int expert, const ditch_weight *w);
void model_set_delta(ditch_hip_model *m, int layer, int slot, int expert, uint64_t rank, const float *a,
                     const float *b);
void model_edit(ditch_hip_model *m, int layer, int slot, int expert, const float *v, uint64_t k, float weight);
void model_reset_deltas(ditch_hip_model *m);
void model_edit_batch(ditch_hip_model *m, const ditch_edit_target *targets, uint64_t n, uint64_t k);
void model_edit_ex(ditch_hip_model *m, int layer, int slot, int expert, const float *v, uint64_t k, float weight,
                   int mode, int64_t lora_rank, uint64_t seed, int ablate);
ditch_hip_kv_cache *kv_cache_create(ditch_hip_model *m, int64_t B, int64_t T);
ditch_hip_model *model_load(ditch_hip *h, const char *path, uint64_t expert_cache);
void generate(ditch_hip_model *m, ditch_hip_kv_cache *kc, const uint32_t *tokens, const uint64_t *lens, int64_t B,
              int64_t max_new, const uint32_t *eos, int64_t n_eos, ditch_sampler *smp, uint32_t *out_tokens,
              uint64_t *out_lens, float *first_logits);
uint64_t model_bytes(const ditch_hip_model *m);
void model_forward(ditch_hip_model *m, const uint32_t *d_tokens, const ditch_row *d_rows, int64_t n, int64_t B,
                   int64_t T, const uint64_t *d_capture, int64_t n_capture, float *d_res, const uint64_t *d_logit_rows,
                   int64_t n_logit, float *d_logits, ditch_hip_kv_cache *pc = nullptr);

// Device buffer owned for the duration of one call.
struct Tmp {
    void *p = nullptr;
    explicit Tmp(size_t bytes) { p = dev_alloc(bytes); }
    ~Tmp() { dev_free(p); }
    template <typename T>
    T *as() { return (T *)p; }
};

static void h2d(void *d, const void *hsrc, size_t bytes, hipStream_t s) {
    if (bytes) DITCH_TRY_HIP(hipMemcpyAsync(d, hsrc, bytes, hipMemcpyHostToDevice, s));
}
static void d2h(void *hdst, const void *d, size_t bytes, hipStream_t s) {
    if (bytes) DITCH_TRY_HIP(hipMemcpyAsync(hdst, d, bytes, hipMemcpyDeviceToHost, s));
}

template <typename F>
static int32_t guarded(ditch_hip *h, F &&f) {
    if (!h) return DITCH_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(h->mu);
    try {
        f();
        h->last_error.clear();
        return DITCH_OK;
    } catch (const Error &e) {
        h->last_error = e.msg;
        return e.code;
    } catch (const std::bad_alloc &) {
        h->last_error = "host out of memory";
        return DITCH_OUT_OF_MEMORY;
    } catch (...) {
        h->last_error = "unexpected failure";
        return DITCH_DEVICE_FAILED;
    }
}

}  // namespace ditch

using namespace ditch;

// The allocation-free product's scratch: activation fragments, GEMV term
// staging and split-K partial sums of ditch_hip_matmulT_device_noalloc.
// Each GPU the library runs on holds its own copy for the life of the
// process. Host code never uses this name as an address: the context keeps
// the device's copy from hipGetSymbolAddress (h->static_scratch).
static constexpr size_t STATIC_SCRATCH_BYTES = (size_t)64 << 20;
static __device__ __align__(256) uint8_t scratch[STATIC_SCRATCH_BYTES];

// The order of the calls that share one GPU's scratch: each call's stream
// waits for the event the previous call (any stream, any context) recorded
// after its last kernel, and records it again after its own. The events are
// created at context open, one per device, and kept for the life of the
// process, like the scratch array.
struct ScratchOrder {
    std::mutex mu;
    hipEvent_t last = nullptr;
    bool recorded = false;
};
static constexpr int MAX_DEVICES = 64;
static ScratchOrder scratch_order[MAX_DEVICES];

extern "C" {

ditch_hip *ditch_hip_open(int32_t device, char *err, size_t err_len) {
    auto fail = [&](const std::string &m) -> ditch_hip * {
        if (err && err_len) {
            strncpy(err, m.c_str(), err_len - 1);
            err[err_len - 1] = 0;
        }
        return nullptr;
    };
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return fail("no HIP device");
    if (device < 0 || device >= count) return fail("device index out of range");
    if (hipSetDevice(device) != hipSuccess) return fail("hipSetDevice failed");
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return fail("hipGetDeviceProperties failed");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(std::string("this library is built for gfx950, the device is ") + prop.gcnArchName);
    auto *h = new (std::nothrow) ditch_hip();
    if (!h) return fail("host out of memory");
    h->device = device;
    h->cu_count = prop.multiProcessorCount;
    h->name = std::string(prop.name) + " (" + prop.gcnArchName + ")";
    if (hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking) != hipSuccess) {
        delete h;
        return fail("hipStreamCreate failed");
    }
    // this device's copy of the static scratch array (device `device` is
    // current); on failure only the allocation-free entry point is refused
    const hipError_t se = hipGetSymbolAddress(&h->static_scratch, HIP_SYMBOL(scratch));
    if (se != hipSuccess) {
        h->static_scratch = nullptr;
        h->scratch_error = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(se);
        (void)hipGetLastError();
    } else if (device >= MAX_DEVICES) {
        h->static_scratch = nullptr;
        h->scratch_error = "device index beyond the scratch ordering table";
    } else {
        ScratchOrder &o = scratch_order[device];
        std::lock_guard<std::mutex> lk(o.mu);
        if (!o.last && hipEventCreateWithFlags(&o.last, hipEventDisableTiming) != hipSuccess) {
            o.last = nullptr;
            h->static_scratch = nullptr;
            h->scratch_error = "hipEventCreate for the scratch ordering failed";
            (void)hipGetLastError();
        }
    }
    return h;
}

void ditch_hip_close(ditch_hip *h) {
    if (!h) return;
    (void)hipStreamSynchronize(h->stream);
    residency_clear(h);
    (void)hipStreamDestroy(h->stream);
    delete h;
}

const char *ditch_hip_name(ditch_hip *h) { return h ? h->name.c_str() : ""; }
const char *ditch_hip_last_error(ditch_hip *h) { return h ? h->last_error.c_str() : "null context"; }
void ditch_hip_forget_weights(ditch_hip *h) {
    if (!h) return;
    std::lock_guard<std::mutex> lk(h->mu);
    (void)hipStreamSynchronize(h->stream);
    residency_clear(h);
}

int32_t ditch_hip_set_residency(ditch_hip *h, uint64_t budget_bytes, int32_t weights_stable) {
    return guarded(h, [&] {
        DITCH_TRY_HIP(hipStreamSynchronize(h->stream));
        residency_configure(h, budget_bytes, weights_stable != 0);
    });
}

int32_t ditch_hip_residency_stats(ditch_hip *h, ditch_residency_stats *out) {
    return guarded(h, [&] {
        DITCH_CHECK(out, DITCH_INVALID_ARGUMENT, "NULL stats");
        const auto &r = h->res;
        *out = ditch_residency_stats{r.budget, r.used, (uint64_t)r.entries.size(), r.hits, r.misses, r.evictions,
                                     (uint64_t)(r.budget > 0 && r.stable)};
    });
}
void *ditch_hip_stream(ditch_hip *h) { return h ? (void *)h->stream : nullptr; }
int32_t ditch_hip_sync(ditch_hip *h) {
    return guarded(h, [&] { DITCH_TRY_HIP(hipStreamSynchronize(h->stream)); });
}

// ---------------------------------------------------------------------------
// VTable operations, host memory

int32_t ditch_hip_matmulT(ditch_hip *h, float *out, const float *x, uint64_t n, const ditch_weight *w) {
    return guarded(h, [&] {
        DITCH_CHECK(w && out && x, DITCH_INVALID_ARGUMENT, "NULL argument");
        if (n == 0 || w->rows == 0) return;
        hipStream_t s = h->stream;
        WeightRef t;
        acquire_weight(h, w, s, t);
        Tmp dx(n * w->cols * 4), dout(n * w->rows * 4);
        h2d(dx.p, x, n * w->cols * 4, s);
        MatmulEpilogue ep;
        ep.exact = 1;
        launch_matmul(t->v, dout.as<float>(), dx.as<float>(), (int64_t)n, ep, s, nullptr, &h->split);
        d2h(out, dout.p, n * w->rows * 4, s);
        DITCH_TRY_HIP(hipStreamSynchronize(s));
    });
}

int32_t ditch_hip_matvecTMulti(ditch_hip *h, float *out, const ditch_weight *w, const float *y, uint64_t q) {
    return guarded(h, [&] {
        DITCH_CHECK(w && out && y, DITCH_INVALID_ARGUMENT, "NULL argument");
        if (q == 0) return;
        hipStream_t s = h->stream;
        WeightRef t;
        acquire_weight(h, w, s, t);
        Tmp dy(q * w->rows * 4), dout(q * w->cols * 4);
        h2d(dy.p, y, q * w->rows * 4, s);
        launch_matvecT(dout.as<float>(), t->v, dy.as<float>(), (int64_t)q, s);
        d2h(out, dout.p, q * w->cols * 4, s);
        DITCH_TRY_HIP(hipStreamSynchronize(s));
    });
}

int32_t ditch_hip_rowNorms(ditch_hip *h, float *out, const ditch_weight *w) {
    return guarded(h, [&] {
        DITCH_CHECK(w && out, DITCH_INVALID_ARGUMENT, "NULL argument");
        hipStream_t s = h->stream;
        WeightRef t;
        acquire_weight(h, w, s, t);
        Tmp dout(w->rows * 4);
        launch_row_norms(dout.as<float>(), t->v, s);
        d2h(out, dout.p, w->rows * 4, s);
        DITCH_TRY_HIP(hipStreamSynchronize(s));
    });
}

int32_t ditch_hip_attentionScores(ditch_hip *h, float *scores, uint64_t n_keys, const float *q, uint64_t hd,
                                  const float *k, uint64_t stride, float scale) {
    return guarded(h, [&] {
        DITCH_CHECK(scores && q && k && stride >= hd, DITCH_INVALID_ARGUMENT, "attentionScores arguments");
        if (n_keys == 0) return;
        hipStream_t s = h->stream;
        size_t kb = ((n_keys - 1) * stride + hd) * 4;
        Tmp dq(hd * 4), dk(kb), ds(n_keys * 4);
        h2d(dq.p, q, hd * 4, s);
        h2d(dk.p, k, kb, s);
        launch_attention_scores(ds.as<float>(), n_keys, dq.as<float>(), hd, dk.as<float>(), stride, scale, s);
        d2h(scores, ds.p, n_keys * 4, s);
        DITCH_TRY_HIP(hipStreamSynchronize(s));
    });
}

int32_t ditch_hip_attentionValues(ditch_hip *h, float *out, uint64_t vd, const float *scores, uint64_t n_keys,
                                  const float *v, uint64_t stride) {
    return guarded(h, [&] {
        DITCH_CHECK(out && scores && v && stride >= vd, DITCH_INVALID_ARGUMENT, "attentionValues arguments");
        hipStream_t s = h->stream;
        if (vd == 0) return;
        size_t vb = n_keys ? ((n_keys - 1) * stride + vd) * 4 : 4;
        Tmp dsc(n_keys * 4 + 4), dv(vb), dout(vd * 4);
        h2d(dsc.p, scores, n_keys * 4, s);
        if (n_keys) h2d(dv.p, v, vb, s);
        launch_attention_values(dout.as<float>(), vd, dsc.as<float>(), n_keys, dv.as<float>(), stride, s);
        d2h(out, dout.p, vd * 4, s);
        DITCH_TRY_HIP(hipStreamSynchronize(s));
    });
}

int32_t ditch_hip_gatedActivation(ditch_hip *h, uint32_t act, float *out, const float *gate, const float *up,
                                  uint64_t n, uint64_t len, uint64_t in_stride, uint64_t out_stride) {
    return guarded(h, [&] {
        DITCH_CHECK(out && gate && act <= 5 && in_stride >= len && out_stride >= len, DITCH_INVALID_ARGUMENT,
                    "gatedActivation arguments");
        if (n == 0 || len == 0) return;
        hipStream_t s = h->stream;
        size_t ib = ((n - 1) * in_stride + len) * 4, ob = ((n - 1) * out_stride + len) * 4;
        Tmp dg(ib), du(up ? ib : 4), dout(ob);
        h2d(dg.p, gate, ib, s);
        if (up) h2d(du.p, up, ib, s);
        // rows of `out` between the written spans keep their contents
        h2d(dout.p, out, ob, s);
        launch_gated_act(act, dout.as<float>(), dg.as<float>(), up ? du.as<float>() : nullptr, n, len, in_stride,
                         out_stride, s);
        d2h(out, dout.p, ob, s);
        DITCH_TRY_HIP(hipStreamSynchronize(s));
    });
}

int32_t ditch_hip_rmsnormRows(ditch_hip *h, float *out, const float *x, const float *weight, uint64_t weight_len,
                              uint64_t n, uint64_t len, float eps, int32_t gemma_style) {
    return guarded(h, [&] {
        DITCH_CHECK(out && x && (weight_len == 0 || (weight && weight_len >= len)), DITCH_INVALID_ARGUMENT,
                    "rmsnormRows arguments");
        if (n == 0 || len == 0) return;
        hipStream_t s = h->stream;
        Tmp dx(n * len * 4), dw(weight_len * 4 + 4), dout(n * len * 4);
        h2d(dx.p, x, n * len * 4, s);
        if (weight_len) h2d(dw.p, weight, len * 4, s);
        launch_rmsnorm(dout.as<float>(), dx.as<float>(), dw.as<float>(), weight_len ? (int64_t)len : 0, n, len, eps,
                       gemma_style, s);
        d2h(out, dout.p, n * len * 4, s);
        DITCH_TRY_HIP(hipStreamSynchronize(s));
    });
}

int32_t ditch_hip_layernormRows(ditch_hip *h, float *out, const float *x, const float *weight, uint64_t weight_len,
                                const float *bias, uint64_t n, uint64_t len, float eps, int32_t one_plus) {
    return guarded(h, [&] {
        DITCH_CHECK(out && x && (weight_len == 0 || (weight && weight_len >= len)), DITCH_INVALID_ARGUMENT,
                    "layernormRows arguments");
        if (n == 0 || len == 0) return;
        hipStream_t s = h->stream;
        Tmp dx(n * len * 4), dw(len * 4), db(len * 4), dout(n * len * 4);
        h2d(dx.p, x, n * len * 4, s);
        if (weight_len) h2d(dw.p, weight, len * 4, s);
        if (bias) h2d(db.p, bias, len * 4, s);
        launch_layernorm(dout.as<float>(), dx.as<float>(), dw.as<float>(), weight_len ? (int64_t)len : 0,
                         bias ? db.as<float>() : nullptr, n, len, eps, one_plus, s);
        d2h(out, dout.p, n * len * 4, s);
        DITCH_TRY_HIP(hipStreamSynchronize(s));
    });
}

int32_t ditch_hip_softmaxRows(ditch_hip *h, float *x, uint64_t n, uint64_t len) {
    return guarded(h, [&] {
        DITCH_CHECK(x, DITCH_INVALID_ARGUMENT, "NULL argument");
        if (n == 0 || len == 0) return;
        hipStream_t s = h->stream;
        Tmp dx(n * len * 4);
        h2d(dx.p, x, n * len * 4, s);
        launch_softmax_rows(dx.as<float>(), n, len, s);
        d2h(x, dx.p, n * len * 4, s);
        DITCH_TRY_HIP(hipStreamSynchronize(s));
    });
}

int32_t ditch_hip_ropeRows(ditch_hip *h, float *x, uint64_t n, uint64_t dim, const float *cos_table,
                           const float *sin_table, uint64_t table_len, uint64_t half, const uint32_t *pos,
                           uint32_t style) {
    return guarded(h, [&] {
        DITCH_CHECK(x && cos_table && sin_table && pos && style <= 1 && 2 * half >= dim, DITCH_INVALID_ARGUMENT,
                    "ropeRows arguments");
        for (uint64_t i = 0; i < n; i++) DITCH_CHECK(pos[i] < table_len, DITCH_INVALID_ARGUMENT, "position beyond the table");
        if (n == 0 || dim == 0) return;
        hipStream_t s = h->stream;
        Tmp dx(n * dim * 4), dc(table_len * half * 4), dsn(table_len * half * 4), dp(n * 4);
        h2d(dx.p, x, n * dim * 4, s);
        h2d(dc.p, cos_table, table_len * half * 4, s);
        h2d(dsn.p, sin_table, table_len * half * 4, s);
        h2d(dp.p, pos, n * 4, s);
        launch_rope_rows(dx.as<float>(), n, dim, dc.as<float>(), dsn.as<float>(), half, dp.as<uint32_t>(), style, s);
        d2h(x, dx.p, n * dim * 4, s);
        DITCH_TRY_HIP(hipStreamSynchronize(s));
    });
}

// ---------------------------------------------------------------------------
// Decode

int32_t ditch_hip_dequant(ditch_hip *h, void *out, const ditch_weight *w, uint64_t row0, uint64_t nrows) {
    return guarded(h, [&] {
        DITCH_CHECK(w && out, DITCH_INVALID_ARGUMENT, "NULL argument");
        if (nrows == 0) return;
        dequant_to_host(h, out, w, row0, nrows);
    });
}

// ---------------------------------------------------------------------------
// Resident tensors

ditch_hip_tensor *ditch_hip_upload(ditch_hip *h, const ditch_weight *w) {
    ditch_hip_tensor *t = nullptr;
    int32_t rc = guarded(h, [&] {
        DITCH_CHECK(w, DITCH_INVALID_ARGUMENT, "NULL weight");
        t = upload_weight(h, w, h->stream);
    });
    return rc == DITCH_OK ? t : nullptr;
}

void ditch_hip_tensor_free(ditch_hip *h, ditch_hip_tensor *t) {
    if (h) (void)hipStreamSynchronize(h->stream);
    free_tensor(t);
}

uint64_t ditch_hip_tensor_bytes(const ditch_hip_tensor *t) { return t ? t->bytes : 0; }

int32_t ditch_hip_tensor_dequant(ditch_hip *h, void *d_out, uint64_t out_bytes, const ditch_hip_tensor *t,
                                 uint64_t row0, uint64_t nrows) {
    return guarded(h, [&] {
        DITCH_CHECK(t && d_out && row0 + nrows <= (uint64_t)t->v.rows, DITCH_INVALID_ARGUMENT, "tensor_dequant range");
        uint64_t elem = is_bf16_virtual(t->v.orig_dtype) ? 2 : 4;
        DITCH_CHECK(nrows * (uint64_t)t->v.cols * elem <= out_bytes, DITCH_INVALID_ARGUMENT,
                    "tensor_dequant: output buffer too small");
        launch_dequant(t->v, d_out, (int64_t)row0, (int64_t)nrows, h->stream);
    });
}

int32_t ditch_hip_matmulT_device(ditch_hip *h, float *d_out, uint64_t out_bytes, const float *d_x, uint64_t x_bytes,
                                 uint64_t n, const ditch_hip_tensor *w, const float *d_bias, int32_t accumulate,
                                 void *stream) {
    return guarded(h, [&] {
        DITCH_CHECK(w && d_out && d_x, DITCH_INVALID_ARGUMENT, "NULL argument");
        DITCH_CHECK(out_bytes >= n * (uint64_t)w->v.rows * 4 && x_bytes >= n * (uint64_t)w->v.cols * 4,
                    DITCH_INVALID_ARGUMENT, "matmulT_device: output or input buffer shorter than n rows");
        MatmulEpilogue ep;
        ep.bias = d_bias;
        ep.accumulate = accumulate;
        launch_matmul(w->v, d_out, d_x, (int64_t)n, ep, stream ? (hipStream_t)stream : h->stream, nullptr, &h->split);
    });
}

int32_t ditch_hip_matmulT_device_noalloc(ditch_hip *h, float *d_out, uint64_t out_bytes, const float *d_x,
                                         uint64_t x_bytes, uint64_t n, const ditch_hip_tensor *w, const float *d_bias,
                                         int32_t accumulate, void *stream) {
    return guarded(h, [&] {
        DITCH_CHECK(w && d_out && d_x, DITCH_INVALID_ARGUMENT, "NULL argument");
        DITCH_CHECK(out_bytes >= n * (uint64_t)w->v.rows * 4 && x_bytes >= n * (uint64_t)w->v.cols * 4,
                    DITCH_INVALID_ARGUMENT, "matmulT_device_noalloc: output or input buffer shorter than n rows");
        DITCH_CHECK(h->static_scratch, DITCH_DEVICE_FAILED, "static scratch not resolved: " + h->scratch_error);
        MatmulEpilogue ep;
        ep.bias = d_bias;
        ep.accumulate = accumulate;
        DevBuf ws(h->static_scratch, STATIC_SCRATCH_BYTES);  // never allocates: too large a need is refused
        hipStream_t st = stream ? (hipStream_t)stream : h->stream;
        // after the previous call's kernels on this GPU, whatever its stream
        // (a stream under graph capture takes its order from the graph)
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        DITCH_TRY_HIP(hipStreamIsCapturing(st, &cap));
        ScratchOrder &o = scratch_order[h->device];
        std::lock_guard<std::mutex> lk(o.mu);
        if (cap == hipStreamCaptureStatusNone && o.recorded) DITCH_TRY_HIP(hipStreamWaitEvent(st, o.last, 0));
        launch_matmul(w->v, d_out, d_x, (int64_t)n, ep, st, nullptr, &ws);
        if (cap == hipStreamCaptureStatusNone) {
            DITCH_TRY_HIP(hipEventRecord(o.last, st));
            o.recorded = true;
        }
    });
}

uint64_t ditch_hip_static_scratch_bytes(void) { return STATIC_SCRATCH_BYTES; }

// fragment layout of the large-batch product over w: 2 = bf16 terms, 1 = MX
// fp6 terms, 0 = none
static int frag_kind(const TileView &w, int64_t n) {
    if (mx_gemm_takes(w, n)) return 1;
    if (tile_gemm_takes(w, n)) return 2;
    return 0;
}

uint64_t ditch_hip_frag_bytes(const ditch_hip_tensor *w, uint64_t n) {
    if (!w || n == 0) return 0;
    switch (frag_kind(w->v, (int64_t)n)) {
    case 1: return mx_frag_bytes((int64_t)n, w->v.units_k);
    case 2: return split_bytes_ldk((int64_t)n, split_ldk(w->v.cols), 2);
    default: return 0;
    }
}

int32_t ditch_hip_split_device(ditch_hip *h, void *d_frags, uint64_t frag_bytes, const float *d_x, uint64_t n,
                               const ditch_hip_tensor *w, void *stream) {
    return guarded(h, [&] {
        DITCH_CHECK(d_frags && d_x && w, DITCH_INVALID_ARGUMENT, "NULL argument");
        if (n == 0) return;
        const uint64_t need = ditch_hip_frag_bytes(w, n);
        DITCH_CHECK(need > 0, DITCH_UNSUPPORTED, "split: the large-batch product does not take this weight or batch");
        DITCH_CHECK(frag_bytes >= need, DITCH_INVALID_ARGUMENT, "split: fragment buffer too small");
        const TileView &v = w->v;
        hipStream_t s = stream ? (hipStream_t)stream : h->stream;
        if (frag_kind(v, (int64_t)n) == 1)
            launch_split_mx(d_frags, d_x, nullptr, (int64_t)n, v.cols, v.cols, v.units_k, s);
        else
            launch_split(d_frags, d_x, nullptr, (int64_t)n, v.cols, v.cols, split_ldk(v.cols), 2, s);
    });
}

int32_t ditch_hip_matmulT_frags_device(ditch_hip *h, float *d_out, uint64_t out_bytes, const void *d_frags,
                                       uint64_t frag_bytes, uint64_t n, const ditch_hip_tensor *w,
                                       const float *d_bias, int32_t accumulate, void *stream) {
    return guarded(h, [&] {
        DITCH_CHECK(w && d_out && d_frags, DITCH_INVALID_ARGUMENT, "NULL argument");
        if (n == 0) return;
        const int kind = frag_kind(w->v, (int64_t)n);
        DITCH_CHECK(kind != 0, DITCH_UNSUPPORTED,
                    "matmulT_frags: the large-batch product does not take this weight or batch");
        DITCH_CHECK(out_bytes >= n * (uint64_t)w->v.rows * 4 && frag_bytes >= ditch_hip_frag_bytes(w, n),
                    DITCH_INVALID_ARGUMENT, "matmulT_frags: output or fragment buffer shorter than n rows");
        MatmulEpilogue ep;
        ep.bias = d_bias;
        ep.accumulate = accumulate;
        hipStream_t s = stream ? (hipStream_t)stream : h->stream;
        if (kind == 1)
            launch_mx_gemm(w->v, d_out, w->v.rows, d_frags, w->v.units_k, (int64_t)n, ep, s);
        else {
            const size_t pb = tile_part_bytes(w->v, (int64_t)n, 2);
            launch_tile_gemm(w->v, d_out, w->v.rows, d_frags, split_ldk(w->v.cols), (int64_t)n, 2, ep, s,
                             pb ? h->split.get<float>(pb / sizeof(float)) : nullptr);
        }
    });
}

// the fused gate/up pair: 1 = scaled MFMA (MX fragments in and out), 2 =
// bf16-term tiled product, 0 = not taken
static int glu_kind(const TileView &g, const TileView &u, int64_t n) {
    if (mx_glu_takes(g, u, n) && g.rows % 128 == 0) return 1;
    if (!mx_gemm_takes(g, n) && tile_glu_takes(g, u, n)) return 2;
    return 0;
}

uint64_t ditch_hip_glu_frag_bytes(const ditch_hip_tensor *gate, const ditch_hip_tensor *up, uint64_t n) {
    if (!gate || !up || n == 0) return 0;
    switch (glu_kind(gate->v, up->v, (int64_t)n)) {
    case 1: return mx_frag_bytes((int64_t)n, gate->v.rows / 128);
    case 2: return split_bytes_ldk((int64_t)n, split_ldk(gate->v.rows), 2);
    default: return 0;
    }
}

int32_t ditch_hip_glu_device(ditch_hip *h, void *d_out_frags, uint64_t out_bytes, const void *d_frags,
                             uint64_t frag_bytes, uint64_t n, const ditch_hip_tensor *gate, const ditch_hip_tensor *up,
                             uint32_t act, void *stream) {
    return guarded(h, [&] {
        DITCH_CHECK(d_out_frags && d_frags && gate && up, DITCH_INVALID_ARGUMENT, "NULL argument");
        if (n == 0) return;
        DITCH_CHECK(act <= 5, DITCH_INVALID_ARGUMENT, "unknown activation");
        const int kind = glu_kind(gate->v, up->v, (int64_t)n);
        DITCH_CHECK(kind != 0, DITCH_UNSUPPORTED, "glu: the fused product does not take this pair or batch");
        DITCH_CHECK(frag_bytes >= ditch_hip_frag_bytes(gate, n) && out_bytes >= ditch_hip_glu_frag_bytes(gate, up, n),
                    DITCH_INVALID_ARGUMENT, "glu: fragment buffers shorter than n rows");
        hipStream_t s = stream ? (hipStream_t)stream : h->stream;
        const TileView &g = gate->v, &u = up->v;
        if (kind == 1)
            launch_mx_glu(g, u, act, nullptr, d_out_frags, g.rows / 128, d_frags, g.units_k, (int64_t)n, s);
        else
            launch_tile_glu(g, u, act, nullptr, d_out_frags, split_ldk(g.rows), d_frags, split_ldk(g.cols),
                            (int64_t)n, s);
    });
}

// ---------------------------------------------------------------------------
// Model

ditch_hip_model *ditch_hip_model_create(ditch_hip *h, const ditch_model_config *cfg) {
    ditch_hip_model *m = nullptr;
    int32_t rc = guarded(h, [&] {
        DITCH_CHECK(cfg, DITCH_INVALID_ARGUMENT, "NULL config");
        m = model_create(h, cfg);
    });
    return rc == DITCH_OK ? m : nullptr;
}

ditch_hip_model *ditch_hip_model_load(ditch_hip *h, const char *path, uint64_t expert_cache_bytes) {
    ditch_hip_model *m = nullptr;
    int32_t rc = guarded(h, [&] { m = model_load(h, path, expert_cache_bytes); });
    return rc == DITCH_OK ? m : nullptr;
}

int32_t ditch_hip_model_get_config(const ditch_hip_model *m, ditch_model_config *out) {
    if (!m || !out) return DITCH_INVALID_ARGUMENT;
    *out = m->c;
    out->rope_factors = nullptr;
    return DITCH_OK;
}

void ditch_hip_model_free(ditch_hip_model *m) {
    if (!m) return;
    (void)hipStreamSynchronize(m->h->stream);
    delete m;
}

int32_t ditch_hip_model_set(ditch_hip_model *m, int32_t layer, int32_t slot, int32_t expert, const ditch_weight *w) {
    if (!m) return DITCH_INVALID_ARGUMENT;
    return guarded(m->h, [&] {
        DITCH_CHECK(w, DITCH_INVALID_ARGUMENT, "NULL weight");
        model_set(m, layer, slot, expert, w);
    });
}

int32_t ditch_hip_model_set_delta(ditch_hip_model *m, int32_t layer, int32_t slot, int32_t expert, uint64_t rank,
                                  const float *a, const float *b) {
    if (!m) return DITCH_INVALID_ARGUMENT;
    return guarded(m->h, [&] {
        DITCH_CHECK(rank == 0 || (a && b), DITCH_INVALID_ARGUMENT, "NULL delta");
        model_set_delta(m, layer, slot, expert, rank, a, b);
    });
}

int32_t ditch_hip_model_set_expert_cache(ditch_hip_model *m, uint64_t bytes) {
    if (!m) return DITCH_INVALID_ARGUMENT;
    return guarded(m->h, [&] {
        for (const auto &L : m->layers)
            for (const auto *vec : {&L.eg, &L.eu, &L.ed})
                for (const auto &mt : *vec)
                    DITCH_CHECK(!mt.ok(), DITCH_INVALID_ARGUMENT, "expert cache: experts were registered before");
        DITCH_CHECK(!m->cache, DITCH_INVALID_ARGUMENT, "expert cache already built");
        m->expert_budget = bytes;
    });
}

int32_t ditch_hip_model_expert_cache_stats(const ditch_hip_model *m, ditch_expert_cache_stats *out) {
    if (!m || !out) return DITCH_INVALID_ARGUMENT;
    *out = ditch_expert_cache_stats{};
    out->capacity = m->expert_budget;
    if (const ditch::ExpertCache *c = m->cache) {
        out->slots = c->slots.size();
        for (const auto &sl : c->slots) out->resident += sl.layer >= 0;
        out->hits = c->hits;
        out->misses = c->misses;
        out->prefetched = c->prefetches;
        out->bytes_read = c->bytes_read;
        out->evictions = c->evictions;
        out->slot_bytes = c->slot_bytes;
        out->warmed = c->warmed;
        out->bytes_staged = c->bytes_staged;
    }
    return DITCH_OK;
}

int32_t ditch_hip_model_hot_experts(ditch_hip_model *m, ditch_hot_expert *out, uint64_t capacity,
                                    uint64_t *count) {
    if (!m) return DITCH_INVALID_ARGUMENT;
    return guarded(m->h, [&] {
        DITCH_CHECK(count && (out || capacity == 0), DITCH_INVALID_ARGUMENT, "hot_experts arguments");
        const std::vector<HotExpert> hot = cache_hot_experts(m);
        *count = hot.size();
        for (uint64_t k = 0; k < capacity && k < hot.size(); k++)
            out[k] = ditch_hot_expert{hot[k].layer, hot[k].expert, hot[k].uses};
    });
}

int32_t ditch_hip_model_warm_experts(ditch_hip_model *m, const ditch_hot_expert *hot, uint64_t n,
                                     uint64_t *warmed) {
    if (!m) return DITCH_INVALID_ARGUMENT;
    return guarded(m->h, [&] {
        DITCH_CHECK(hot || n == 0, DITCH_INVALID_ARGUMENT, "warm_experts arguments");
        DITCH_CHECK(m->expert_budget > 0, DITCH_INVALID_ARGUMENT, "warm_experts: the model streams no experts");
        std::vector<HotExpert> h((size_t)n);
        for (uint64_t k = 0; k < n; k++) h[k] = HotExpert{hot[k].layer, hot[k].expert, hot[k].uses};
        const uint64_t w = cache_warm(m, h.data(), n);
        if (warmed) *warmed = w;
    });
}

int32_t ditch_hip_model_reset_deltas(ditch_hip_model *m) {
    if (!m) return DITCH_INVALID_ARGUMENT;
    return guarded(m->h, [&] { model_reset_deltas(m); });
}

uint64_t ditch_hip_model_bytes(const ditch_hip_model *m) { return m ? model_bytes(m) : 0; }

int32_t ditch_hip_forward(ditch_hip_model *m, const uint32_t *tokens, const ditch_row *rows, uint64_t n,
                          const uint64_t *capture_rows, uint64_t n_capture, float *residuals,
                          const uint64_t *logit_rows, uint64_t n_logit, float *logits) {
    if (!m) return DITCH_INVALID_ARGUMENT;
    return guarded(m->h, [&] {
        DITCH_CHECK(tokens && rows, DITCH_INVALID_ARGUMENT, "NULL tokens/rows");
        DITCH_CHECK(n_capture == 0 || (capture_rows && residuals), DITCH_INVALID_ARGUMENT, "capture buffers");
        DITCH_CHECK(n_logit == 0 || (logit_rows && logits), DITCH_INVALID_ARGUMENT, "logit buffers");
        if (n == 0) return;
        const ditch_model_config &c = m->c;
        for (uint64_t i = 0; i < n; i++)
            DITCH_CHECK(tokens[i] < (m->embed.t ? (uint64_t)m->embed.t->v.rows : 0), DITCH_INVALID_ARGUMENT,
                        "token id outside the embedding table");
        for (uint64_t i = 0; i < n_capture; i++) DITCH_CHECK(capture_rows[i] < n, DITCH_INVALID_ARGUMENT, "capture row");
        for (uint64_t i = 0; i < n_logit; i++) DITCH_CHECK(logit_rows[i] < n, DITCH_INVALID_ARGUMENT, "logit row");
        hipStream_t s = m->h->stream;
        int64_t B = 0, T = 0;
        for (uint64_t i = 0; i < n; i++) {
            B = std::max<int64_t>(B, (int64_t)rows[i].b + 1);
            T = std::max<int64_t>(T, (int64_t)rows[i].pos + 1);
        }
        size_t res_bytes = (c.layers + 1) * n_capture * c.hidden * 4, log_bytes = n_logit * c.vocab * 4;
        Tmp dt(n * 4), dr(n * sizeof(ditch_row)), dc(n_capture * 8 + 8), dl(n_logit * 8 + 8), dres(res_bytes + 4),
            dlog(log_bytes + 4);
        h2d(dt.p, tokens, n * 4, s);
        h2d(dr.p, rows, n * sizeof(ditch_row), s);
        h2d(dc.p, capture_rows, n_capture * 8, s);
        h2d(dl.p, logit_rows, n_logit * 8, s);
        model_forward(m, dt.as<uint32_t>(), dr.as<ditch_row>(), (int64_t)n, B, T, dc.as<uint64_t>(),
                      (int64_t)n_capture, n_capture ? dres.as<float>() : nullptr, dl.as<uint64_t>(), (int64_t)n_logit,
                      n_logit ? dlog.as<float>() : nullptr);
        d2h(residuals, dres.p, n_capture ? res_bytes : 0, s);
        d2h(logits, dlog.p, n_logit ? log_bytes : 0, s);
        DITCH_TRY_HIP(hipStreamSynchronize(s));
    });
}

int32_t ditch_hip_forward_device(ditch_hip_model *m, const uint32_t *d_tokens, const ditch_row *d_rows, uint64_t n,
                                 uint32_t n_prompts, uint32_t max_len, const uint64_t *d_capture_rows,
                                 uint64_t n_capture, float *d_residuals, uint64_t residuals_bytes,
                                 const uint64_t *d_logit_rows, uint64_t n_logit, float *d_logits,
                                 uint64_t logits_bytes) {
    if (!m) return DITCH_INVALID_ARGUMENT;
    return guarded(m->h, [&] {
        DITCH_CHECK(d_tokens && d_rows, DITCH_INVALID_ARGUMENT, "NULL tokens/rows");
        if (n == 0) return;
        const ditch_model_config &c = m->c;
        DITCH_CHECK(n_prompts > 0 && max_len > 0, DITCH_INVALID_ARGUMENT, "forward_device: empty KV cache shape");
        DITCH_CHECK(n_capture == 0 || (d_capture_rows && d_residuals &&
                                       residuals_bytes >= (c.layers + 1) * n_capture * c.hidden * 4),
                    DITCH_INVALID_ARGUMENT, "forward_device: capture rows or residual buffer missing or too short");
        DITCH_CHECK(n_logit == 0 || (d_logit_rows && d_logits && logits_bytes >= n_logit * c.vocab * 4),
                    DITCH_INVALID_ARGUMENT, "forward_device: logit rows or logit buffer missing or too short");
        model_forward(m, d_tokens, d_rows, (int64_t)n, (int64_t)n_prompts, (int64_t)max_len, d_capture_rows,
                      (int64_t)n_capture, n_capture ? d_residuals : nullptr, d_logit_rows, (int64_t)n_logit,
                      n_logit ? d_logits : nullptr);
    });
}

ditch_hip_kv_cache *ditch_hip_kv_cache_create(ditch_hip_model *m, uint32_t n_prompts, uint32_t max_len) {
    if (!m) return nullptr;
    ditch_hip_kv_cache *c = nullptr;
    int32_t rc = guarded(m->h, [&] { c = kv_cache_create(m, (int64_t)n_prompts, (int64_t)max_len); });
    return rc == DITCH_OK ? c : nullptr;
}

void ditch_hip_kv_cache_free(ditch_hip_kv_cache *c) {
    if (!c) return;
    (void)hipStreamSynchronize(c->m->h->stream);
    delete c;
}

int32_t ditch_hip_forward_cached(ditch_hip_model *m, ditch_hip_kv_cache *c, const uint32_t *d_tokens,
                                 const ditch_row *d_rows, uint64_t n, const uint64_t *d_logit_rows, uint64_t n_logit,
                                 float *d_logits, uint64_t logits_bytes) {
    if (!m) return DITCH_INVALID_ARGUMENT;
    return guarded(m->h, [&] {
        DITCH_CHECK(c && c->m == m, DITCH_INVALID_ARGUMENT, "forward_cached: the KV cache belongs to another model");
        DITCH_CHECK(d_tokens && d_rows, DITCH_INVALID_ARGUMENT, "NULL tokens/rows");
        if (n == 0) return;
        DITCH_CHECK(n_logit == 0 || (d_logit_rows && d_logits && logits_bytes >= n_logit * m->c.vocab * 4),
                    DITCH_INVALID_ARGUMENT, "forward_cached: logit rows or logit buffer missing or too short");
        model_forward(m, d_tokens, d_rows, (int64_t)n, c->B, c->T, nullptr, 0, nullptr, d_logit_rows,
                      (int64_t)n_logit, n_logit ? d_logits : nullptr, c);
    });
}

int32_t ditch_hip_sampler_init(ditch_sampler *s, uint64_t seed, float temperature, uint64_t top_k, float top_p) {
    if (!s) return DITCH_INVALID_ARGUMENT;
    sampler_init(s, seed, temperature, top_k, top_p);
    return DITCH_OK;
}

int32_t ditch_hip_pick_tokens_device(ditch_hip *h, uint32_t *d_out, const float *d_logits, uint64_t n, uint64_t vocab,
                                     ditch_sampler *sampler, void *stream) {
    return guarded(h, [&] {
        DITCH_CHECK(d_out && d_logits, DITCH_INVALID_ARGUMENT, "NULL argument");
        launch_pick(d_out, d_logits, (int64_t)n, (int64_t)vocab, sampler, stream ? (hipStream_t)stream : h->stream);
    });
}

int32_t ditch_hip_generate(ditch_hip_model *m, ditch_hip_kv_cache *c, const uint32_t *tokens,
                           const uint64_t *prompt_lens, uint64_t n_prompts, uint64_t max_new_tokens,
                           const uint32_t *eos_ids, uint64_t n_eos, ditch_sampler *sampler, uint32_t *out_tokens,
                           uint64_t *out_lens, float *first_logits) {
    if (!m) return DITCH_INVALID_ARGUMENT;
    return guarded(m->h, [&] {
        DITCH_CHECK(tokens && prompt_lens && out_tokens && out_lens && (n_eos == 0 || eos_ids), DITCH_INVALID_ARGUMENT,
                    "NULL argument");
        generate(m, c, tokens, prompt_lens, (int64_t)n_prompts, (int64_t)max_new_tokens, eos_ids, (int64_t)n_eos,
                 sampler, out_tokens, out_lens, first_logits);
    });
}

int32_t ditch_hip_model_path_stats(const ditch_hip_model *m, ditch_model_path_stats *out) {
    if (!m || !out) return DITCH_INVALID_ARGUMENT;
    out->moe_device_planned = m->moe_device_planned;
    out->moe_host_planned = m->moe_host_planned;
    return DITCH_OK;
}

// ---------------------------------------------------------------------------
// Edit, log-softmax, KL

int32_t ditch_hip_edit_delta(ditch_hip *h, float *a, float *b, const ditch_weight *w, const float *v, uint64_t k,
                             float weight) {
    return guarded(h, [&] {
        DITCH_CHECK(a && b && w && v && k > 0, DITCH_INVALID_ARGUMENT, "edit_delta arguments");
        hipStream_t s = h->stream;
        WeightRef t;
        acquire_weight(h, w, s, t);
        Tmp dv(k * w->rows * 4), da(k * w->cols * 4);
        h2d(dv.p, v, k * w->rows * 4, s);
        launch_matvecT(da.as<float>(), t->v, dv.as<float>(), (int64_t)k, s);
        d2h(a, da.p, k * w->cols * 4, s);
        DITCH_TRY_HIP(hipStreamSynchronize(s));
        for (uint64_t i = 0; i < w->rows; i++)
            for (uint64_t j = 0; j < k; j++) b[i * k + j] = -weight * v[j * w->rows + i];
    });
}

int32_t ditch_hip_model_edit(ditch_hip_model *m, int32_t layer, int32_t slot, int32_t expert, const float *v,
                             uint64_t k, float weight) {
    if (!m) return DITCH_INVALID_ARGUMENT;
    return guarded(m->h, [&] {
        DITCH_CHECK(v && k > 0, DITCH_INVALID_ARGUMENT, "edit arguments");
        model_edit(m, layer, slot, expert, v, k, weight);
    });
}

int32_t ditch_hip_model_edit_batch(ditch_hip_model *m, const ditch_edit_target *targets, uint64_t n, uint64_t k) {
    if (!m) return DITCH_INVALID_ARGUMENT;
    return guarded(m->h, [&] {
        DITCH_CHECK(targets && n > 0 && k > 0, DITCH_INVALID_ARGUMENT, "edit batch arguments");
        model_edit_batch(m, targets, n, k);
    });
}

static void edit_opts_check(const ditch_edit_options *o) {
    DITCH_CHECK(o, DITCH_INVALID_ARGUMENT, "NULL edit options");
    DITCH_CHECK(o->row_normalization >= DITCH_ROWNORM_NONE && o->row_normalization <= DITCH_ROWNORM_FULL,
                DITCH_INVALID_ARGUMENT, "edit: unknown row normalisation");
}

uint64_t ditch_hip_edit_rank(uint64_t rows, uint64_t cols, uint64_t k, const ditch_edit_options *opts) {
    if (!opts) return 0;
    return (uint64_t)edit_rank((int64_t)rows, (int64_t)cols, (int64_t)k, opts->row_normalization,
                               (int64_t)opts->lora_rank, opts->ablate_inputs != 0);
}

int32_t ditch_hip_edit_delta_ex(ditch_hip *h, float *a, uint64_t a_len, float *b, uint64_t b_len,
                                const ditch_weight *w, const float *v, uint64_t k, float weight,
                                const ditch_edit_options *opts) {
    return guarded(h, [&] {
        DITCH_CHECK(a && b && w && v && k > 0, DITCH_INVALID_ARGUMENT, "edit_delta_ex arguments");
        edit_opts_check(opts);
        const uint64_t rank = ditch_hip_edit_rank(w->rows, w->cols, k, opts);
        DITCH_CHECK(a_len >= rank * w->cols && b_len >= w->rows * rank, DITCH_INVALID_ARGUMENT,
                    "edit_delta_ex: a or b shorter than the delta");
        hipStream_t s = h->stream;
        WeightRef t;
        acquire_weight(h, w, s, t);
        float *da = nullptr, *db = nullptr;
        int64_t r = 0;
        edit_delta_device(h, t->v, v, (int64_t)k, weight, opts->row_normalization, (int64_t)opts->lora_rank, opts->seed,
                          opts->ablate_inputs != 0, s, &da, &db, &r);
        try {
            d2h(a, da, r * w->cols * 4, s);
            d2h(b, db, w->rows * r * 4, s);
            DITCH_TRY_HIP(hipStreamSynchronize(s));
        } catch (...) {
            dev_free(da);
            dev_free(db);
            throw;
        }
        dev_free(da);
        dev_free(db);
    });
}

int32_t ditch_hip_model_edit_ex(ditch_hip_model *m, int32_t layer, int32_t slot, int32_t expert, const float *v,
                                uint64_t k, float weight, const ditch_edit_options *opts) {
    if (!m) return DITCH_INVALID_ARGUMENT;
    return guarded(m->h, [&] {
        DITCH_CHECK(v && k > 0, DITCH_INVALID_ARGUMENT, "edit arguments");
        edit_opts_check(opts);
        model_edit_ex(m, layer, slot, expert, v, k, weight, opts->row_normalization, (int64_t)opts->lora_rank,
                      opts->seed, opts->ablate_inputs != 0);
    });
}

void ditch_hip_edit_gaussian(float *out, uint64_t n, uint64_t seed) {
    if (out) edit_gaussian(out, (size_t)n, seed);
}

int32_t ditch_hip_logSoftmaxRows(ditch_hip *h, float *out, const float *x, uint64_t n, uint64_t len) {
    return guarded(h, [&] {
        DITCH_CHECK(out && x, DITCH_INVALID_ARGUMENT, "NULL argument");
        if (n == 0 || len == 0) return;
        hipStream_t s = h->stream;
        Tmp dx(n * len * 4), dout(n * len * 4);
        h2d(dx.p, x, n * len * 4, s);
        launch_log_softmax_rows(dout.as<float>(), dx.as<float>(), n, len, s, &h->rowred);
        d2h(out, dout.p, n * len * 4, s);
        DITCH_TRY_HIP(hipStreamSynchronize(s));
    });
}

int32_t ditch_hip_klRows(ditch_hip *h, double *kl, const float *base_logprobs, const float *trial_logits, uint64_t n,
                         uint64_t vocab) {
    return guarded(h, [&] {
        DITCH_CHECK(kl && base_logprobs && trial_logits, DITCH_INVALID_ARGUMENT, "NULL argument");
        if (n == 0) return;
        hipStream_t s = h->stream;
        Tmp db(n * vocab * 4), dt(n * vocab * 4), dk(n * 8);
        h2d(db.p, base_logprobs, n * vocab * 4, s);
        h2d(dt.p, trial_logits, n * vocab * 4, s);
        launch_kl_rows(dk.as<double>(), db.as<float>(), dt.as<float>(), n, vocab, s, &h->rowred);
        d2h(kl, dk.p, n * 8, s);
        DITCH_TRY_HIP(hipStreamSynchronize(s));
    });
}

int32_t ditch_hip_logSoftmaxRows_device(ditch_hip *h, float *d_out, const float *d_x, uint64_t n, uint64_t len,
                                        void *stream) {
    return guarded(h, [&] {
        DITCH_CHECK(d_out && d_x, DITCH_INVALID_ARGUMENT, "NULL argument");
        if (n == 0 || len == 0) return;
        launch_log_softmax_rows(d_out, d_x, (int64_t)n, (int64_t)len, stream ? (hipStream_t)stream : h->stream,
                                &h->rowred);
    });
}

int32_t ditch_hip_klRows_device(ditch_hip *h, double *d_kl, const float *d_base_logprobs,
                                const float *d_trial_logits, uint64_t n, uint64_t vocab, void *stream) {
    return guarded(h, [&] {
        DITCH_CHECK(d_kl && d_base_logprobs && d_trial_logits, DITCH_INVALID_ARGUMENT, "NULL argument");
        if (n == 0) return;
        launch_kl_rows(d_kl, d_base_logprobs, d_trial_logits, (int64_t)n, (int64_t)vocab,
                       stream ? (hipStream_t)stream : h->stream, &h->rowred);
    });
}

// ---------------------------------------------------------------------------
// Direction pipeline

static hipStream_t pick(ditch_hip *h, void *stream) { return stream ? (hipStream_t)stream : h->stream; }

int32_t ditch_hip_residual_reduce_device(ditch_hip *h, const float *d_residuals, uint64_t entries, uint64_t n_capture,
                                         uint64_t hidden, const uint32_t *d_first, const uint32_t *d_take,
                                         uint64_t prompts, float winsor_q, float *d_vout, double *d_sum, double *d_sq,
                                         void *stream) {
    return guarded(h, [&] {
        DITCH_CHECK(d_residuals && d_first && d_take && d_vout, DITCH_INVALID_ARGUMENT, "NULL argument");
        launch_residual_reduce(d_residuals, (int64_t)entries, (int64_t)n_capture, (int64_t)hidden, d_first, d_take,
                               (int64_t)prompts, winsor_q, d_vout, d_sum, d_sq, pick(h, stream));
    });
}

int32_t ditch_hip_residual_mean_device(ditch_hip *h, float *d_mean, const double *d_sum, uint64_t count, uint64_t n,
                                       void *stream) {
    return guarded(h, [&] {
        DITCH_CHECK(d_mean && d_sum, DITCH_INVALID_ARGUMENT, "NULL argument");
        launch_residual_mean(d_mean, d_sum, count, (int64_t)n, pick(h, stream));
    });
}

int32_t ditch_hip_directions_device(ditch_hip *h, float *d_dirs, const float *d_good_means, const float *d_bad_means,
                                    uint64_t entries, uint64_t hidden, int32_t orthogonalize, void *stream) {
    return guarded(h, [&] {
        DITCH_CHECK(d_dirs && d_good_means && d_bad_means, DITCH_INVALID_ARGUMENT, "NULL argument");
        DITCH_CHECK(entries <= 65535, DITCH_UNSUPPORTED, "directions: more than 65535 entries");
        launch_directions(d_dirs, d_good_means, d_bad_means, (int64_t)entries, (int64_t)hidden, orthogonalize,
                          pick(h, stream), &h->dirtmp);
    });
}

int32_t ditch_hip_sketch_add_device(ditch_hip *h, double *d_y, double *d_w, const float *d_omega, uint64_t m,
                                    const float *d_center, const float *d_v, uint64_t prompts, uint64_t entries,
                                    uint64_t hidden, void *stream) {
    return guarded(h, [&] {
        DITCH_CHECK(d_y && d_w && d_omega && d_center && d_v, DITCH_INVALID_ARGUMENT, "NULL argument");
        DITCH_CHECK(prompts <= 65535 && entries <= 65535, DITCH_UNSUPPORTED, "sketch: grid");
        launch_sketch_add(d_y, d_w, d_omega, (int64_t)m, d_center, d_v, (int64_t)prompts, (int64_t)entries,
                          (int64_t)hidden, pick(h, stream), &h->dirtmp);
    });
}

int32_t ditch_hip_basis_device(ditch_hip *h, float *d_dirs, const float *d_first, const float *d_good_means,
                               uint64_t entries, uint64_t hidden, uint64_t k, int32_t orthogonalize, const double *d_y,
                               const double *d_w, uint64_t m, void *stream) {
    return guarded(h, [&] {
        DITCH_CHECK(d_dirs && d_first && d_good_means && (k <= 1 || (d_y && d_w)), DITCH_INVALID_ARGUMENT,
                    "NULL argument");
        DITCH_CHECK(k >= 1, DITCH_INVALID_ARGUMENT, "basis: no directions");
        DITCH_CHECK(entries <= 65535, DITCH_UNSUPPORTED, "basis: more than 65535 entries");
        launch_basis(d_dirs, d_first, d_good_means, (int64_t)entries, (int64_t)hidden, (int64_t)k, orthogonalize, d_y,
                     d_w, (int64_t)m, pick(h, stream), &h->dirtmp);
    });
}

}  // extern "C"
