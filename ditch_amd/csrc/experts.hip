// experts.hip — routed-expert streaming (expert_cache.zig:108-607).
//
// With a budget set on the model (ditch_hip_model_set_expert_cache) every
// routed expert matrix is re-tiled on the device at registration as usual,
// then copied to pinned host memory (one blob per matrix) and its device
// memory freed. The forward keeps a device cache of fixed-size slots (one
// slot = an expert's gate, up and down blobs) within the budget; after a
// layer's router has picked its experts, the missing ones are copied host ->
// slot on the cache's own stream, the compute stream waits on those copies,
// and the grouped products run on views into the slots. A layer whose
// experts do not all fit runs in chunks that do. The experts the next routed
// layer used in the previous forward are copied ahead while this layer
// computes (prompts of a search share their routing from trial to trial).
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "model.h"

namespace ditch {

void host_mat_free(HostMat &hm) {
    if (hm.host) {
        if (hm.pinned) (void)hipHostFree(hm.host);
        else free(hm.host);
    }
    hm.host = nullptr;
    hm.bytes = 0;
    hm.pinned = false;
}

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

void stream_out(Mat &mt, uint64_t &pinned_bytes, uint64_t pinned_limit, uint64_t &pinned_total, bool &pinned_exhausted) {
    ditch_hip_tensor *t = mt.t;
    DITCH_CHECK(t, DITCH_INVALID_ARGUMENT, "stream_out of an empty slot");
    void *parts[6] = {t->codes, t->scale, t->zero, t->side, t->mx, t->mx_scales};
    size_t off[6], total = 0;
    for (int i = 0; i < 6; i++) {
        off[i] = total;
        if (parts[i]) total += align256(t->part_bytes[i]);
    }
    HostMat hm;
    const size_t alloc = total ? total : 256;
    if (!pinned_exhausted && pinned_bytes + alloc <= pinned_limit) {
        if (hipHostMalloc((void **)&hm.host, alloc, hipHostMallocDefault) == hipSuccess) {
            hm.pinned = true;
            pinned_bytes += alloc;
            pinned_total += alloc;
        } else {
            (void)hipGetLastError();
            hm.host = nullptr;
            pinned_exhausted = true;
        }
    }
    if (!hm.host) {
        void *p = nullptr;
        DITCH_CHECK(posix_memalign(&p, 4096, (alloc + 4095) / 4096 * 4096) == 0, DITCH_OUT_OF_MEMORY,
                    "expert streaming: host out of memory");
        hm.host = (uint8_t *)p;
    }
    hm.bytes = total;
    for (int i = 0; i < 6; i++)
        if (parts[i] && t->part_bytes[i]) DITCH_TRY_HIP(hipMemcpy(hm.host + off[i], parts[i], t->part_bytes[i], hipMemcpyDeviceToHost));
    // where each TileView pointer lands: inside one of the parts (MXFP4's side
    // words alias its scale array)
    const TileView &v = t->v;
    const void *fields[6] = {v.codes, v.scale, v.zero, v.side, v.mx, v.mx_scales};
    for (int f = 0; f < 6; f++) {
        hm.field_off[f] = -1;
        if (!fields[f]) continue;
        for (int i = 0; i < 6; i++) {
            const uint8_t *b = (const uint8_t *)parts[i];
            if (b && (const uint8_t *)fields[f] >= b && (const uint8_t *)fields[f] < b + t->part_bytes[i]) {
                hm.field_off[f] = (int64_t)(off[i] + ((const uint8_t *)fields[f] - b));
                break;
            }
        }
        DITCH_CHECK(hm.field_off[f] >= 0, DITCH_DEVICE_FAILED, "stream_out: a view pointer outside the tensor's parts");
    }
    for (int i = 0; i < 6; i++) dev_free(parts[i]);
    t->codes = t->scale = t->zero = t->side = t->mx = t->mx_scales = nullptr;
    t->v.codes = nullptr;
    t->v.scale = nullptr;
    t->v.zero = nullptr;
    t->v.side = nullptr;
    t->v.mx = nullptr;
    t->v.mx_scales = nullptr;
    host_mat_free(mt.hm);
    mt.hm = hm;
}

TileView view_at(const Mat &mt, const uint8_t *base) {
    TileView v = mt.t->v;
    auto at = [&](int f) { return mt.hm.field_off[f] < 0 ? nullptr : base + mt.hm.field_off[f]; };
    v.codes = at(0);
    v.scale = at(1);
    v.zero = at(2);
    v.side = (const uint32_t *)at(3);
    v.mx = at(4);
    v.mx_scales = at(5);
    return v;
}

ExpertCache::~ExpertCache() {
    if (copy) (void)hipStreamSynchronize(copy);
    for (Slot &sl : slots)
        if (sl.loaded) (void)hipEventDestroy(sl.loaded);
    for (hipEvent_t ev : use_ev)
        if (ev) (void)hipEventDestroy(ev);
    for (int b = 0; b < NSTAGE; b++) {
        if (stage[b]) (void)hipHostFree(stage[b]);
        if (stage_done[b]) (void)hipEventDestroy(stage_done[b]);
    }
    dev_free(arena);
    if (copy) (void)hipStreamDestroy(copy);
}

// Slot layout: gate blob, up blob, down blob (256-byte aligned).
static uint64_t expert_bytes(const Layer &L, int64_t e) {
    return align256(L.eg[e].hm.bytes) + align256(L.eu[e].hm.bytes) + align256(L.ed[e].hm.bytes);
}

// Builds the cache at the first forward: the slot size is the largest
// expert of the model, the slot count what the budget holds.
static ExpertCache &cache_of(ditch_hip_model *m) {
    if (m->cache) return *m->cache;
    uint64_t slot = 0, count = 0;
    for (const Layer &L : m->layers)
        for (size_t e = 0; e < L.eg.size(); e++)
            if (L.eg[e].streamed() && L.eu[e].streamed() && L.ed[e].streamed()) {
                slot = std::max(slot, expert_bytes(L, (int64_t)e));
                count++;
            }
    DITCH_CHECK(slot > 0, DITCH_INVALID_ARGUMENT, "expert cache: no streamed experts");
    const uint64_t n = std::min(m->expert_budget / slot, count);  // no more slots than experts
    DITCH_CHECK(n >= 1, DITCH_INVALID_ARGUMENT, "expert cache budget below one expert's gate + up + down");
    auto *c = new ExpertCache();
    try {
        c->capacity = m->expert_budget;
        c->slot_bytes = slot;
        c->arena = (uint8_t *)dev_alloc(n * slot);
        c->slots.resize(n);
        for (auto &sl : c->slots) DITCH_TRY_HIP(hipEventCreateWithFlags(&sl.loaded, hipEventDisableTiming));
        for (hipEvent_t &ev : c->use_ev) DITCH_TRY_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
        DITCH_TRY_HIP(hipStreamCreateWithFlags(&c->copy, hipStreamNonBlocking));
        c->last_used.resize(m->layers.size());
        c->resident_layer.assign(m->layers.size(), 0);
    } catch (...) {
        delete c;
        throw;
    }
    m->cache = c;
    return *c;
}

static uint64_t slot_key(int64_t layer, int64_t e) { return (uint64_t)layer << 32 | (uint64_t)e; }

static int find_slot(const ExpertCache &c, int64_t layer, int64_t e) {
    const auto it = c.where.find(slot_key(layer, e));
    return it == c.where.end() ? -1 : it->second;
}

// Routed layers copied ahead after each routed layer (see cache_prefetch_next).
constexpr int PREFETCH_LAYERS = 2;

// Experts layer `l` routed in the last forward that are not resident.
static int64_t hole_of(const ExpertCache &c, int64_t l) {
    return (int64_t)c.last_used[l].size() - c.resident_layer[l];
}

// The most experts a layer may be missing once the copies ahead have made
// room: the shortfall (experts the routed layers used last minus slots)
// spread over the routed layers that are not being copied ahead. A cache
// short by D experts then refills about D / (routed - PREFETCH_LAYERS) of
// them for each routed layer, a steady stream of copies under the compute,
// where letting the whole shortfall sit in one layer makes that layer wait
// for all of it. 0: no shortfall, no cap.
static int64_t hole_cap(const ExpertCache &c, const ditch_hip_model *m) {
    int64_t want = 0, routed = 0;
    for (size_t l = 0; l < c.last_used.size(); l++)
        if (m->moe_layers[l]) {
            routed++;
            want += (int64_t)c.last_used[l].size();
        }
    const int64_t short_by = want - (int64_t)c.slots.size(), spread = routed - PREFETCH_LAYERS;
    if (short_by <= 0 || spread <= 0) return 0;
    return (short_by + spread - 1) / spread;
}

// Victim for a fill during layer `cur`: an unpinned slot, empty first; then
// the slot whose layer the forward reaches last from `cur` (the layers just
// computed), among that layer's slots one whose expert reloads by DMA from
// pinned host memory (so the pageable ones stay resident), then the least
// recently used. A copy ahead for a layer `ahead` routed layers on passes
// `cap` > 0: layers further than that whose missing experts are below the
// cap come first, so the shortfall spreads over the layers.
static int victim(const ExpertCache &c, int64_t cur, int64_t nlayers, int64_t cap = 0, int64_t ahead = -1) {
    int best = -1;
    int64_t best_d = -1;
    uint64_t best_stamp = 0;
    bool best_cheap = false, best_open = false;
    for (size_t i = 0; i < c.slots.size(); i++) {
        const auto &sl = c.slots[i];
        if (sl.pins > 0) continue;
        if (sl.layer < 0) return (int)i;
        const int64_t d = ((sl.layer - cur - 1) % nlayers + nlayers) % nlayers;
        const bool open = cap > 0 && d > ahead && hole_of(c, sl.layer) < cap;
        bool better;
        if (best < 0) better = true;
        else if (open != best_open) better = open;
        else if (d != best_d) better = d > best_d;
        else if (sl.cheap != best_cheap) better = sl.cheap;
        else better = sl.stamp < best_stamp;
        if (better) {
            best = (int)i;
            best_d = d;
            best_stamp = sl.stamp;
            best_cheap = sl.cheap;
            best_open = open;
        }
    }
    return best;
}

// A pageable blob to the device through the pinned staging ring (the role of
// stream.zig's pinned buffers): each piece is copied on the host into the
// next staging buffer once the copy stream has finished with it, then sent
// on the copy stream.
static void stage_copy(ExpertCache &c, uint8_t *dst, const uint8_t *src, size_t bytes) {
    for (size_t off = 0; off < bytes;) {
        const int b = c.stage_next;
        c.stage_next = (b + 1) % ExpertCache::NSTAGE;
        if (!c.stage[b]) {
            DITCH_TRY_HIP(hipHostMalloc((void **)&c.stage[b], ExpertCache::STAGE_BYTES, hipHostMallocDefault));
            DITCH_TRY_HIP(hipEventCreateWithFlags(&c.stage_done[b], hipEventDisableTiming));
        }
        if (c.stage_pending[b]) DITCH_TRY_HIP(hipEventSynchronize(c.stage_done[b]));
        const size_t n = std::min(ExpertCache::STAGE_BYTES, bytes - off);
        memcpy(c.stage[b], src + off, n);
        DITCH_TRY_HIP(hipMemcpyAsync(dst + off, c.stage[b], n, hipMemcpyHostToDevice, c.copy));
        DITCH_TRY_HIP(hipEventRecord(c.stage_done[b], c.copy));
        c.stage_pending[b] = true;
        c.bytes_staged += n;
        off += n;
    }
}

// Fills slot `i` with expert (layer, e): the copy stream waits for the
// compute stream's last use of the slot, then copies the three blobs.
static void fill(ExpertCache &c, ditch_hip_model *m, int i, int64_t layer, int64_t e) {
    auto &sl = c.slots[i];
    if (sl.layer >= 0) c.evictions++;
    if (sl.use_serial > c.released_done && sl.use_serial > c.copy_waited) {
        DITCH_TRY_HIP(hipStreamWaitEvent(c.copy, c.use_ev[sl.use_serial % ExpertCache::USE_RING], 0));
        c.copy_waited = sl.use_serial;
    }
    const Layer &L = m->layers[layer];
    uint8_t *base = c.arena + (uint64_t)i * c.slot_bytes;
    uint64_t off = 0;
    for (const Mat *mt : {&L.eg[e], &L.eu[e], &L.ed[e]}) {
        if (mt->hm.pinned) DITCH_TRY_HIP(hipMemcpyAsync(base + off, mt->hm.host, mt->hm.bytes, hipMemcpyHostToDevice, c.copy));
        else stage_copy(c, base + off, mt->hm.host, mt->hm.bytes);
        c.bytes_read += mt->hm.bytes;
        off += align256(mt->hm.bytes);
    }
    DITCH_TRY_HIP(hipEventRecord(sl.loaded, c.copy));
    if (sl.layer >= 0) {
        c.where.erase(slot_key(sl.layer, sl.expert));
        c.resident_layer[sl.layer]--;
    }
    sl.layer = layer;
    sl.expert = e;
    c.where[slot_key(layer, e)] = i;
    c.resident_layer[layer]++;
    sl.cheap = L.eg[e].hm.pinned && L.eu[e].hm.pinned && L.ed[e].hm.pinned;
    sl.load_serial = ++c.loads;
    sl.prefetched = false;
    sl.stamp = ++c.clock;
}

void expert_views(ExpertCache &c, int i, const Layer &L, int64_t e, TileView &g, TileView &u, TileView &d) {
    const uint8_t *base = c.arena + (uint64_t)i * c.slot_bytes;
    g = view_at(L.eg[e], base);
    u = view_at(L.eu[e], base + align256(L.eg[e].hm.bytes));
    d = view_at(L.ed[e], base + align256(L.eg[e].hm.bytes) + align256(L.eu[e].hm.bytes));
}

// Makes as many of `experts` (from `from` on) resident and pinned as the
// slots allow; the compute stream `s` waits for their copies. Returns the
// slots in the order of `experts` (chunk = the prefix that fits). The
// resident ones are pinned first, so that a miss never takes the slot of an
// expert the same chunk is about to use (the victim rule counts the current
// layer's other slots as the farthest in the cycle).
std::vector<int> cache_acquire(ditch_hip_model *m, int64_t layer, const std::vector<int32_t> &experts, size_t from,
                               hipStream_t s) {
    ExpertCache &c = cache_of(m);
    std::vector<int> got;
    const int64_t nl = (int64_t)m->layers.size();
    std::vector<int> resident(experts.size(), -1);
    for (size_t k = from; k < experts.size(); k++) {
        const int i = find_slot(c, layer, experts[k]);
        if (i >= 0) {
            resident[k] = i;
            c.slots[i].pins++;
        }
    }
    uint64_t newest = 0;
    int newest_slot = -1;
    size_t k = from;
    for (; k < experts.size(); k++) {
        const int64_t e = experts[k];
        int i = resident[k];
        c.uses[(uint64_t)layer << 32 | (uint64_t)e]++;
        if (i >= 0) {
            // an expert filled ahead of use was still a read (expert_cache.zig:403-410)
            if (c.slots[i].prefetched) c.misses++;
            else c.hits++;
            c.slots[i].prefetched = false;
        } else {
            i = victim(c, layer, nl);
            // every slot holds an expert this chunk uses later and none is
            // acquired yet: give those up from the last, so the chunk starts
            for (size_t j = experts.size(); i < 0 && got.empty() && j-- > k + 1;) {
                if (resident[j] < 0) continue;
                c.slots[resident[j]].pins--;
                resident[j] = -1;
                i = victim(c, layer, nl);
            }
            if (i < 0) {
                c.uses[(uint64_t)layer << 32 | (uint64_t)e]--;
                break;  // every slot pinned by this chunk
            }
            fill(c, m, i, layer, e);
            c.misses++;
            c.slots[i].pins++;
        }
        auto &sl = c.slots[i];
        sl.stamp = ++c.clock;
        if (sl.load_serial > newest) {
            newest = sl.load_serial;
            newest_slot = i;
        }
        got.push_back(i);
    }
    // the copy stream is in order: its newest fill among the chunk's slots
    // done means all of them are
    if (newest_slot >= 0) DITCH_TRY_HIP(hipStreamWaitEvent(s, c.slots[newest_slot].loaded, 0));
    // the resident experts past the chunk: unpinned again (a later chunk
    // takes them)
    for (; k < experts.size(); k++)
        if (resident[k] >= 0) c.slots[resident[k]].pins--;
    DITCH_CHECK(!got.empty(), DITCH_DEVICE_FAILED, "expert cache: no slot free for a chunk");
    return got;
}

// The chunk's products are enqueued on `s`: the slots may be refilled once
// the stream has passed this point.
void cache_release(ditch_hip_model *m, const std::vector<int> &slots, hipStream_t s) {
    ExpertCache &c = *m->cache;
    const uint64_t k = ++c.released;
    DITCH_TRY_HIP(hipEventRecord(c.use_ev[k % ExpertCache::USE_RING], s));
    for (int i : slots) {
        auto &sl = c.slots[i];
        sl.use_serial = k;
        sl.pins--;
    }
}

void cache_synced(ditch_hip_model *m) {
    if (m->cache) m->cache->released_done = m->cache->released;
}

// After layer `layer`: copy ahead the experts the next routed layers (up to
// PREFETCH_LAYERS of them, nearest first) used in the previous forward, into
// slots that hold nothing nearer in the cycle than the layer copied for,
// taking them from the layers whose missing experts are under hole_cap().
// Two layers ahead: a copy into a slot of the layer just computed starts
// once that layer's products are done with it, which leaves it about one
// layer's compute.
void cache_prefetch_next(ditch_hip_model *m, int64_t layer) {
    if (!m->cache) return;
    ExpertCache &c = *m->cache;
    const int64_t nl = (int64_t)m->layers.size();
    const int64_t cap = hole_cap(c, m);
    int done = 0;
    for (int64_t d = 1; d < nl && done < PREFETCH_LAYERS; d++) {
        const int64_t next = (layer + d) % nl;
        if (m->layers[next].eg.empty() || !m->moe_layers[next] || !m->layers[next].eg[0].streamed()) continue;
        done++;
        if ((size_t)next >= c.last_used.size()) continue;
        const int64_t dist_next = d - 1;
        for (int32_t e : c.last_used[next]) {
            if (find_slot(c, next, e) >= 0) continue;
            const int i = victim(c, layer, nl, cap, dist_next);
            if (i < 0) return;
            const auto &sl = c.slots[i];
            // never displace an expert the forward needs before `next`
            if (sl.layer >= 0 && ((sl.layer - layer - 1) % nl + nl) % nl <= dist_next) return;
            fill(c, m, i, next, e);
            c.slots[i].prefetched = true;
            c.prefetches++;
        }
    }
}

// ExpertCache.hotExperts (expert_cache.zig:501-523): every (layer, expert)
// acquired so far with its count, most used first, ties by layer then expert.
std::vector<HotExpert> cache_hot_experts(ditch_hip_model *m) {
    std::vector<HotExpert> out;
    if (!m->cache) return out;
    for (const auto &kv : m->cache->uses)
        out.push_back(HotExpert{(uint32_t)(kv.first >> 32), (uint32_t)(kv.first & 0xffffffffu), kv.second});
    std::sort(out.begin(), out.end(), [](const HotExpert &a, const HotExpert &b) {
        if (a.uses != b.uses) return a.uses > b.uses;
        if (a.layer != b.layer) return a.layer < b.layer;
        return a.expert < b.expert;
    });
    return out;
}

// ExpertCache.warm (expert_cache.zig:567-607): copies in the hottest experts
// of `hot` (most used first) that exist in the model as streamed routed
// experts and fit the free slots, before a run starts. Stops at the first
// entry with no uses or when no slot is free; resident ones are skipped.
// Returns the number copied in.
uint64_t cache_warm(ditch_hip_model *m, const HotExpert *hot, uint64_t n) {
    ExpertCache &c = cache_of(m);
    uint64_t warmed = 0;
    for (uint64_t k = 0; k < n; k++) {
        const HotExpert &h = hot[k];
        if (h.uses == 0) break;
        if (h.layer >= m->layers.size()) continue;
        const Layer &L = m->layers[h.layer];
        if (!m->moe_layers[h.layer] || h.expert >= L.eg.size()) continue;
        if (!(L.eg[h.expert].streamed() && L.eu[h.expert].streamed() && L.ed[h.expert].streamed())) continue;
        if (find_slot(c, h.layer, h.expert) >= 0) continue;
        int free = -1;
        for (size_t i = 0; i < c.slots.size(); i++)
            if (c.slots[i].layer < 0) {
                free = (int)i;
                break;
            }
        if (free < 0) break;
        fill(c, m, free, h.layer, h.expert);
        c.slots[free].prefetched = true;
        warmed++;
    }
    c.warmed += warmed;
    return warmed;
}

void cache_note_layer(ditch_hip_model *m, int64_t layer, const std::vector<int32_t> &experts) {
    if (m->cache && (size_t)layer < m->cache->last_used.size()) m->cache->last_used[layer] = experts;
}

}  // namespace ditch
