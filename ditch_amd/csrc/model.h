// model.h — host-side state of a resident model (not part of the ABI).
#pragma once
#include <cstdint>
#include <memory>
#include <unordered_map>
#include <vector>

#include "internal.h"

struct ditch_hip_model;

namespace ditch {

// A routed expert matrix kept in pinned host memory (expert streaming): its
// re-tiled parts back to back, and where each device pointer of its TileView
// lands in that blob (field_off: codes, scale, zero, side, mx, mx_scales; -1
// for none). `t` keeps the tensor's metadata with no device memory.
struct HostMat {
    uint8_t *host = nullptr;
    size_t bytes = 0;
    bool pinned = false;  // else pageable: copied to the device through the cache's pinned staging ring
    int64_t field_off[6] = {-1, -1, -1, -1, -1, -1};
};
void host_mat_free(HostMat &hm);

struct Mat {
    ditch_hip_tensor *t = nullptr;
    float *da = nullptr, *db = nullptr;  // delta A [rank][cols], B [rows][rank]
    bool joint = false;                   // db lies in da's allocation (one allocation for both)
    std::shared_ptr<void> arena;          // else: da and db lie in a batch edit's allocation, shared
    int rank = 0;
    HostMat hm;
    void clear_delta() {
        if (arena) arena.reset();  // the allocation goes with its last matrix
        else {
            dev_free(da);
            if (!joint) dev_free(db);
        }
        da = db = nullptr;
        joint = false;
        rank = 0;
    }
    void release() {
        free_tensor(t);
        t = nullptr;
        host_mat_free(hm);
        clear_delta();
    }
    bool ok() const { return t != nullptr; }
    bool streamed() const { return hm.host != nullptr; }
};

struct Vec {
    float *p = nullptr;
    int64_t len = 0;
    void release() {
        dev_free(p);
        p = nullptr;
        len = 0;
    }
};

// Moves a registered routed expert matrix to host memory (frees its device
// parts): pinned while its layer's pinned bytes stay under `pinned_limit`
// and the allocation succeeds, pageable after that (systems cap pinned
// memory; these GPU hosts pin about 65 GiB). The model's EXPERT_PINNED_LIMIT
// is shared evenly by its routed layers, so every layer has experts whose
// refill is one DMA.
constexpr uint64_t EXPERT_PINNED_LIMIT = (uint64_t)48 << 30;
void stream_out(Mat &mt, uint64_t &pinned_bytes, uint64_t pinned_limit, uint64_t &pinned_total, bool &pinned_exhausted);
// The matrix's TileView with its device pointers inside a copy of its host
// blob at `base`.
TileView view_at(const Mat &mt, const uint8_t *base);

// Device cache of routed experts (expert_cache.zig:108-607): fixed-size
// slots holding an expert's gate, up and down blobs, filled from pinned host
// memory by hipMemcpyAsync on a copy stream of its own. Keyed by (layer,
// expert); pinned while a chunk of a layer computes with them; victims are
// the unpinned entries whose layer comes back last in the layer cycle (the
// forward visits layers in order), among those one whose blobs sit in pinned
// host memory (a refill by DMA; a pageable blob goes through the host copy
// of the staging ring), least recently used among equals. Copies ahead
// spread the shortfall over the layers (a cap on each layer's missing
// experts).
struct ExpertCache {
    struct Slot {
        int64_t layer = -1, expert = -1;
        int pins = 0;
        uint64_t stamp = 0;
        bool prefetched = false;    // filled ahead of use (prefetch, warm): its first use counts as a miss
        bool cheap = false;         // its three blobs are in pinned host memory: a refill is DMA only
        uint64_t use_serial = 0;     // the release (chunk) that last used it, 0: none
        uint64_t load_serial = 0;    // the fill that last loaded it
        hipEvent_t loaded = nullptr; // the copy stream's last fill
    };
    // One event per released chunk, recorded on the compute stream, in a
    // ring: a slot's refill waits on its last chunk's event unless the host
    // has seen that release complete (a synchronisation of the compute
    // stream) or the copy stream already waits on a later one. An event the
    // ring re-records marks a later point of the same stream, so a late wait
    // on it is only longer, never short.
    static constexpr int USE_RING = 64;
    hipEvent_t use_ev[USE_RING] = {};
    uint64_t released = 0, released_done = 0, copy_waited = 0, loads = 0;
    uint64_t capacity = 0, slot_bytes = 0, clock = 0;
    uint8_t *arena = nullptr;
    std::vector<Slot> slots;
    hipStream_t copy = nullptr;
    uint64_t hits = 0, misses = 0, prefetches = 0, bytes_read = 0, evictions = 0;
    std::vector<std::vector<int32_t>> last_used;  // per layer: experts routed by the last forward
    std::unordered_map<uint64_t, uint64_t> uses;   // (layer << 32 | expert) -> acquisitions
    std::unordered_map<uint64_t, int> where;       // (layer << 32 | expert) -> its slot
    std::vector<int64_t> resident_layer;           // per layer: slots holding one of its experts
    uint64_t warmed = 0;
    // pinned staging ring for pageable blobs: a buffer is refilled once the
    // copy stream has passed its last copy
    static constexpr int NSTAGE = 4;
    static constexpr size_t STAGE_BYTES = (size_t)16 << 20;
    uint8_t *stage[NSTAGE] = {};
    hipEvent_t stage_done[NSTAGE] = {};
    bool stage_pending[NSTAGE] = {};
    int stage_next = 0;
    uint64_t bytes_staged = 0;
    ~ExpertCache();
};

struct Layer;
std::vector<int> cache_acquire(ditch_hip_model *m, int64_t layer, const std::vector<int32_t> &experts, size_t from,
                               hipStream_t s);
void cache_release(ditch_hip_model *m, const std::vector<int> &slots, hipStream_t s);
// The compute stream was synchronised: every chunk released on it is done.
void cache_synced(ditch_hip_model *m);
void cache_note_layer(ditch_hip_model *m, int64_t layer, const std::vector<int32_t> &experts);
void cache_prefetch_next(ditch_hip_model *m, int64_t layer);
struct HotExpert {
    uint32_t layer, expert;
    uint64_t uses;
};
std::vector<HotExpert> cache_hot_experts(ditch_hip_model *m);
uint64_t cache_warm(ditch_hip_model *m, const HotExpert *hot, uint64_t n);
void expert_views(ExpertCache &c, int slot, const Layer &L, int64_t e, TileView &g, TileView &u, TileView &d);

struct Layer {
    Vec attn_norm, q_bias, k_bias, v_bias, q_norm, k_norm, ffn_norm, corr, q_a_norm, kv_a_norm;
    Mat q, k, v, o, gate, up, down, router, sh_gate, sh_up, sh_down, q_a, q_b, kv_a, kv_b;
    std::vector<Mat> eg, eu, ed;
    // the device-planned routed products' segment tables (gate, up, down)
    // and the down deltas' A pointers, uploaded again only when what they
    // are built from changes (plan_key: the tensors, delta factors and
    // ranks, and the model's weights version)
    DevBuf plan_tab, plan_da;
    std::vector<uintptr_t> plan_key;
};

}  // namespace ditch

// KvCache.initFor(model, batch, max_len) (model.zig:2586-2724): every layer's
// keys and values for `B` prompt slots of `T` positions, f32, [layer][b][pos]
// [kv_dim], kept across forward calls (prefill, then decode steps).
struct ditch_hip_kv_cache {
    ditch_hip_model *m = nullptr;
    int64_t B = 0, T = 0, kvd = 0, layers = 0;
    float *k = nullptr, *v = nullptr;
    ~ditch_hip_kv_cache();
};

struct ditch_hip_model {
    ditch_hip *h = nullptr;
    ditch_model_config c{};
    std::vector<uint8_t> moe_layers;
    std::vector<ditch::Layer> layers;
    uint64_t weights_version = 0;  // bumped whenever a matrix slot gets a new tensor
    ditch::Mat embed, lm_head;
    ditch::Vec final_norm;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    // workspace
    ditch::DevBuf x, hbuf, q, k, v, att, o, g, u, kc, vc, rowsb, xa, logit_h, mla_a, mla_b, mla_c;
    ditch::DevBuf r_logits, r_sel, r_selw, r_ord, r_counts, r_offsets, r_pair_token, r_pair_of, e_gate, e_up, e_out, e_shared,
        segs, segd, e_xa, e_xa_part;
    ditch::DevBuf xsplit;  // split activations of the tiled GEMM
    ditch::DevBuf gmeta;   // row map and tile table of the grouped tiled GEMM
    ditch::DevBuf hs, atts, acts;  // A fragments written by the producers (norm, attention, gate/up)
    ditch::DevBuf attn_dense;      // the attention's dense-rows flag
    ditch::DevBuf edit_v, edit_part;  // the none-mode edits' directions and the edit batch's tables
    uint64_t expert_budget = 0;    // > 0: routed experts stream from pinned host memory
    uint64_t expert_pinned = 0;    // host bytes of routed experts held pinned
    std::vector<uint64_t> expert_pinned_layer;  // the same per layer
    bool expert_pinned_exhausted = false;
    // routed layers run with the grouped products planned on the device /
    // on the host (after reading the expert counts back), since creation
    uint64_t moe_device_planned = 0, moe_host_planned = 0;
    ditch::ExpertCache *cache = nullptr;
    ~ditch_hip_model();
};
