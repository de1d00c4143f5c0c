// edit_batch.hip — the edit's product with the resident weights,
// out[q][cols] = y[q][rows] . W (tensor.matvecTMulti, tensor.zig:1056-1094),
// for one matrix or for every matrix of an edit in one launch
// (abliterate.apply's loop over layers, components and experts,
// abliterate.zig:148-210), and the batch of none-mode deltas built on it
// (computeOutputDelta, abliterate.zig:264-280: a = V^T W, b = -weight V).
//
// One workgroup per (matrix, 128/64/32-column unit): its waves walk the
// matrix's 16-row groups, each lane loading the unit's 16-byte tile word of
// its row (row l % 16, columns 8 (l / 16) + 32 t .. +8 of each k tile t),
// four row groups' words and side data in flight at a time, decoding them
// to the reference's values and multiply-adding y[row] into q accumulators
// per column. The 16 rows a wave's lanes hold are summed by DPP moves, the
// waves' sums in LDS in wave order: every weight byte is read once per
// launch, and the result does not depend on timing. Like the reference, a
// row whose y is 0 contributes nothing (0 times a non-finite weight
// included).
#include <map>

#include "gemm_common.h"
#include "model.h"
#include "tile_decode.h"

namespace ditch {

struct WtySeg {
    TileView w;
    const float *y;  // [q][rows]
    float *out;      // [q][cols]
};

struct WtyArgs {
    const WtySeg *segs;     // device table, or NULL: the one segment `one`
    const int64_t *items;   // per workgroup: segment << 32 | unit (with segs)
    WtySeg one;
    int64_t q0, q;          // directions q0 .. q0 + q (q <= the kernel's QB)
};

constexpr int WTY_WAVES = 4;
constexpr int WTY_STEP = 4;  // row groups whose loads are in flight together


// Side data of one (row, unit): the Q8 / MXFP4 scale word, or the FP8 /
// INT4 scale (and INT4 zero point) of each k tile.
template <int TF> struct WtySide {
    uint32_t word;
    float s[Fmt<TF>::tiles];
    int zp[Fmt<TF>::tiles];
};

// (kq: the lane's 8-column quarter of each 32-column k tile; a scale block
// of FP8 / INT4 narrower than the unit covers the lane's 8 columns whole)
template <int TF>
__device__ __forceinline__ void wty_side(const TileView &w, int64_t row, int64_t unit, int kq, WtySide<TF> &sd) {
    constexpr int TL = Fmt<TF>::tiles, UK = 32 * TL;
    if constexpr (TF == TF_Q8 || TF == TF_MX4) {
        sd.word = load_side<TF>(w, row, unit).word;
    } else if constexpr (TF == TF_FP8 || TF == TF_INT4) {
        const int64_t span = TF == TF_FP8 ? w.block_cols : w.group;
        if (span % UK == 0) {  // one scale block covers the unit
            int zp = 0;
            const float s = tile_scale_of<TF>(w, row, unit * UK, &zp);
#pragma unroll
            for (int t = 0; t < TL; t++) {
                sd.s[t] = s;
                sd.zp[t] = zp;
            }
        } else {
#pragma unroll
            for (int t = 0; t < TL; t++) {
                sd.zp[t] = 0;
                sd.s[t] = tile_scale_of<TF>(w, row, unit * UK + 32 * t + 8 * kq, &sd.zp[t]);
            }
        }
    }
}

// The 8 weights of k tile t in the lane's word, as the reference decodes
// them (tiled_element_f32's values).
template <int TF>
__device__ __forceinline__ void wty_decode(const TileView &w, const Raw &raw, const WtySide<TF> &sd, int t,
                                           float (&f)[8]) {
    if constexpr (TF == TF_F32) {
        const uint4 &v = raw.a, &h = raw.b;
        f[0] = u2f(v.x); f[1] = u2f(v.y); f[2] = u2f(v.z); f[3] = u2f(v.w);
        f[4] = u2f(h.x); f[5] = u2f(h.y); f[6] = u2f(h.z); f[7] = u2f(h.w);
    } else if constexpr (TF == TF_F16) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t wd = word_of(raw.a, j / 2);
            f[j] = f16_to_f32((uint16_t)((j & 1) ? (wd >> 16) : (wd & 0xffffu)));
        }
    } else if constexpr (TF == TF_Q8) {
        const uint32_t w0 = word_of(raw.a, 2 * t), w1 = word_of(raw.a, 2 * t + 1);
        const float d = f16_to_f32((uint16_t)((sd.word >> (16 * t)) & 0xffffu));
#pragma unroll
        for (int j = 0; j < 4; j++) {
            f[j] = __fmul_rn((float)(int8_t)((w0 >> (8 * j)) & 0xffu), d);
            f[4 + j] = __fmul_rn((float)(int8_t)((w1 >> (8 * j)) & 0xffu), d);
        }
    } else {
        u32x4 bh;
        if constexpr (TF == TF_BF16) bh = u32x4{raw.a.x, raw.a.y, raw.a.z, raw.a.w};
        else if constexpr (TF == TF_FP8) decode_fp8(w, raw, t, sd.s[t], bh);
        else if constexpr (TF == TF_MX4) decode_mx4(raw, sd.word, t, bh);
        else decode_int4(raw, t, sd.s[t], sd.zp[t], bh);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            f[2 * q] = u2f(bh[q] << 16);
            f[2 * q + 1] = u2f(bh[q] & 0xffff0000u);
        }
    }
}

// FAST (FP8, MXFP4, INT4 tensors whose every element the conversion
// instructions decode exactly, TileView::fast): the tiled GEMM's decode from
// the per-row side words, and every weight finite, so a row whose y is 0
// adds exactly 0 without a test.
template <int TF> constexpr bool wty_has_fast() { return TF == TF_FP8 || TF == TF_MX4 || TF == TF_INT4; }
template <int TF, bool FAST> constexpr int wty_side_words() {
    if constexpr (FAST) return TileCfg<TF>::NS;
    else return 1;
}

template <int TF, int QB, bool FAST>
__global__ __launch_bounds__(WTY_WAVES * 64) void wty_kernel(WtyArgs a) {
    constexpr int TL = Fmt<TF>::tiles, UK = 32 * TL, NV = 8 * TL;
    constexpr int NS = wty_side_words<TF, FAST>();
    __shared__ float red[WTY_WAVES][QB][UK];
    int64_t unit;
    const WtySeg *sp = &a.one;
    if (a.segs) {
        const int64_t it = a.items[blockIdx.x];
        sp = a.segs + (it >> 32);
        unit = it & 0xffffffffll;
    } else {
        unit = blockIdx.x;
    }
    const TileView w = sp->w;
    const float *y = sp->y;
    float *out = sp->out;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, kq = lane >> 4;
    const int64_t groups = (w.rows + 15) / 16;
    float acc[QB][NV];
#pragma unroll
    for (int j = 0; j < QB; j++)
#pragma unroll
        for (int v = 0; v < NV; v++) acc[j][v] = 0.f;

    SideStep st{1u, 0};
    if constexpr (FAST) st = side_step<TF>(w);
    for (int64_t g0 = (int64_t)wave * WTY_STEP; g0 < groups; g0 += WTY_WAVES * WTY_STEP) {
        Raw raw[WTY_STEP];
        WtySide<TF> sd[WTY_STEP];
        uint32_t sw[WTY_STEP][NS];
        float yv[WTY_STEP][QB];
        // every load of the step first
#pragma unroll
        for (int i = 0; i < WTY_STEP; i++) {
            const int64_t g = g0 + i < groups ? g0 + i : groups - 1;
            const int64_t row = g * 16 + r16;
            raw[i] = load_raw<TF>(w, g, unit, lane);
            if constexpr (FAST) {
                const uint32_t *base = w.side + side_row(w, g, lane);
#pragma unroll
                for (int j = 0; j < NS; j++) sw[i][j] = gload<uint32_t>(side_word<TF>(st, base, unit, j));
            } else {
                wty_side<TF>(w, row, unit, kq, sd[i]);
            }
#pragma unroll
            for (int j = 0; j < QB; j++)
                yv[i][j] = (g0 + i < groups && row < w.rows && j < a.q) ? y[(a.q0 + j) * w.rows + row] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < WTY_STEP; i++) {
#pragma unroll
            for (int t = 0; t < TL; t++) {
                float f[8];
                if constexpr (FAST) {
                    const u32x4 c[1] = {u32x4{raw[i].a.x, raw[i].a.y, raw[i].a.z, raw[i].a.w}};
                    const u32x4 bh = decode_tile_lds<TF>(w, c, sw[i], t, true);
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        f[2 * q] = u2f(bh[q] << 16);
                        f[2 * q + 1] = u2f(bh[q] & 0xffff0000u);
                    }
#pragma unroll
                    for (int j = 0; j < QB; j++)
#pragma unroll
                        for (int e = 0; e < 8; e++) acc[j][8 * t + e] = __builtin_fmaf(yv[i][j], f[e], acc[j][8 * t + e]);
                } else {
                    wty_decode<TF>(w, raw[i], sd[i], t, f);
#pragma unroll
                    for (int j = 0; j < QB; j++)
#pragma unroll
                        for (int e = 0; e < 8; e++)
                            acc[j][8 * t + e] = yv[i][j] != 0.f ? __builtin_fmaf(yv[i][j], f[e], acc[j][8 * t + e])
                                                                : acc[j][8 * t + e];
                }
            }
        }
    }
    // the wave's 16 rows, then the waves in order
#pragma unroll
    for (int j = 0; j < QB; j++)
#pragma unroll
        for (int v = 0; v < NV; v++) {
            const float s = row16_sum(acc[j][v]);
            if (r16 == 0) red[wave][j][32 * (v / 8) + 8 * kq + (v % 8)] = s;
        }
    __syncthreads();
    for (int i = threadIdx.x; i < QB * UK; i += WTY_WAVES * 64) {
        const int j = i / UK, c = i % UK;
        const int64_t col = unit * UK + c;
        if (j >= a.q || col >= w.cols) continue;
        float s = red[0][j][c];
#pragma unroll
        for (int wv = 1; wv < WTY_WAVES; wv++) s = __fadd_rn(s, red[wv][j][c]);
        out[(a.q0 + j) * w.cols + col] = s;
    }
}

template <int TF, bool FAST>
static void wty_launch_q(const WtyArgs &a, unsigned blocks, hipStream_t s) {
    if (a.q == 1) hipLaunchKernelGGL((wty_kernel<TF, 1, FAST>), dim3(blocks), dim3(WTY_WAVES * 64), 0, s, a);
    else if (a.q == 2) hipLaunchKernelGGL((wty_kernel<TF, 2, FAST>), dim3(blocks), dim3(WTY_WAVES * 64), 0, s, a);
    else hipLaunchKernelGGL((wty_kernel<TF, 4, FAST>), dim3(blocks), dim3(WTY_WAVES * 64), 0, s, a);
}

template <int TF>
static void wty_launch_fast(const WtyArgs &a, bool fast, unsigned blocks, hipStream_t s) {
    if constexpr (wty_has_fast<TF>()) {
        if (fast) return wty_launch_q<TF, true>(a, blocks, s);
    }
    wty_launch_q<TF, false>(a, blocks, s);
}

// The kind of kernel a tensor takes: its tile format, and whether it takes
// the side-word decode.
static int wty_kind(const TileView &w) {
    const bool fast = w.fast && w.side && (w.tf == TF_FP8 || w.tf == TF_MX4 || w.tf == TF_INT4);
    return w.tf * 2 + (fast ? 1 : 0);
}

// q directions in passes of at most 4 (the accumulators of one pass stay in
// registers)
static void wty_launch(int kind, WtyArgs a, int64_t q, unsigned blocks, hipStream_t s) {
    const int tf = kind / 2;
    const bool fast = kind % 2;
    for (int64_t q0 = 0; q0 < q; q0 += 4) {
        a.q0 = q0;
        a.q = q - q0 < 4 ? q - q0 : 4;
        switch (tf) {
        case TF_BF16: wty_launch_fast<TF_BF16>(a, fast, blocks, s); break;
        case TF_F16: wty_launch_fast<TF_F16>(a, fast, blocks, s); break;
        case TF_F32: wty_launch_fast<TF_F32>(a, fast, blocks, s); break;
        case TF_Q8: wty_launch_fast<TF_Q8>(a, fast, blocks, s); break;
        case TF_FP8: wty_launch_fast<TF_FP8>(a, fast, blocks, s); break;
        case TF_MX4: wty_launch_fast<TF_MX4>(a, fast, blocks, s); break;
        case TF_INT4: wty_launch_fast<TF_INT4>(a, fast, blocks, s); break;
        default: throw Error{DITCH_UNSUPPORTED, "matvecTMulti: tile format"};
        }
        DITCH_TRY_HIP(hipGetLastError());
    }
}

void launch_matvecT(float *out, const TileView &w, const float *y, int64_t q, hipStream_t s) {
    DITCH_CHECK(q >= 1, DITCH_INVALID_ARGUMENT, "matvecTMulti: q must be at least 1");
    if (w.rows <= 0 || w.cols <= 0) return;
    WtyArgs a{};
    a.one = WtySeg{w, y, out};
    wty_launch(wty_kind(w), a, q, (unsigned)w.units_k, s);
}

// ---------------------------------------------------------------------------
// The batch edit

// b = -weight * V^T per matrix: b[i][j] = -weight v[j][i]
struct EditB {
    float *b;
    const float *v;
    int64_t rows;
    float weight;
};

__global__ void edit_b_kernel(const EditB *t, int64_t k) {
    const EditB e = t[blockIdx.y];
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < e.rows * k;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / k, j = i % k;
        e.b[i] = -e.weight * e.v[j * e.rows + r];
    }
}

Mat *mat_slot_of(ditch_hip_model *m, int layer, int slot, int expert);  // model.hip
void check_edit_slot(int slot);                                          // model.hip
void model_edit(ditch_hip_model *m, int layer, int slot, int expert, const float *v, uint64_t k, float weight);

void model_edit_batch(ditch_hip_model *m, const ditch_edit_target *targets, uint64_t n, uint64_t k) {
    DITCH_CHECK(targets && n > 0 && k >= 1 && k <= (uint64_t)INT32_MAX, DITCH_INVALID_ARGUMENT, "edit batch arguments");
    hipStream_t s = m->h->stream;
    // the resident matrices go through the grouped product; a streamed
    // expert's blob is staged on the device one matrix at a time
    std::vector<uint64_t> resident;
    std::vector<Mat *> mats(n);
    for (uint64_t i = 0; i < n; i++) {
        const ditch_edit_target &t = targets[i];
        DITCH_CHECK(t.v != nullptr, DITCH_INVALID_ARGUMENT, "edit batch: NULL directions");
        check_edit_slot(t.slot);
        mats[i] = mat_slot_of(m, t.layer, t.slot, t.expert);
        DITCH_CHECK(mats[i]->ok(), DITCH_INVALID_ARGUMENT, "edit batch: an empty slot");
        if (!mats[i]->streamed()) resident.push_back(i);
    }
    for (uint64_t i = 0; i < n; i++)
        if (mats[i]->streamed()) model_edit(m, targets[i].layer, targets[i].slot, targets[i].expert, targets[i].v, k,
                                            targets[i].weight);
    if (resident.empty()) return;
    // the distinct direction sets, each copied to the device once
    std::unordered_map<const float *, int64_t> vslot;
    std::vector<const float *> vlist;
    std::vector<int64_t> vrows;
    for (uint64_t i : resident) {
        const int64_t rows = mats[i]->t->v.rows;
        auto it = vslot.find(targets[i].v);
        if (it == vslot.end()) {
            vslot[targets[i].v] = (int64_t)vlist.size();
            vlist.push_back(targets[i].v);
            vrows.push_back(rows);
        } else {
            DITCH_CHECK(vrows[it->second] == rows, DITCH_INVALID_ARGUMENT,
                        "edit batch: one direction set given to matrices of different row counts");
        }
    }
    std::vector<int64_t> voff(vlist.size());
    int64_t vtotal = 0;
    for (size_t i = 0; i < vlist.size(); i++) {
        voff[i] = vtotal;
        vtotal += (int64_t)k * vrows[i];
    }
    float *dv = m->edit_v.get<float>((size_t)vtotal);
    for (size_t i = 0; i < vlist.size(); i++)
        DITCH_TRY_HIP(hipMemcpyAsync(dv + voff[i], vlist[i], k * vrows[i] * 4, hipMemcpyHostToDevice, s));
    // every delta in one allocation shared by the matrices (freed when the
    // last of them drops its delta)
    std::vector<int64_t> doff(resident.size());
    int64_t dtotal = 0, items = 0, max_rows = 0;
    for (size_t r = 0; r < resident.size(); r++) {
        const TileView &w = mats[resident[r]]->t->v;
        doff[r] = dtotal;
        dtotal += (int64_t)k * (w.cols + w.rows);
        items += w.units_k;
        max_rows = std::max<int64_t>(max_rows, w.rows);
    }
    std::shared_ptr<void> arena(dev_alloc((size_t)dtotal * 4), [](void *p) { dev_free(p); });
    float *base = (float *)arena.get();
    std::vector<WtySeg> segs(resident.size());
    std::vector<EditB> eb(resident.size());
    std::vector<int64_t> item(items);
    int64_t it = 0;
    int kind = -1;
    bool one_kind = true;
    for (size_t r = 0; r < resident.size(); r++) {
        const ditch_edit_target &t = targets[resident[r]];
        const TileView &w = mats[resident[r]]->t->v;
        const float *v = dv + voff[vslot[t.v]];
        float *da = base + doff[r], *db = da + k * w.cols;
        segs[r] = WtySeg{w, v, da};
        eb[r] = EditB{db, v, w.rows, t.weight};
        for (int64_t u = 0; u < w.units_k; u++) item[it++] = ((int64_t)r << 32) | u;
        if (kind < 0) kind = wty_kind(w);
        one_kind = one_kind && wty_kind(w) == kind;
    }
    // the tables in one staging allocation, freed when the work has run
    const size_t seg_b = segs.size() * sizeof(WtySeg), eb_b = eb.size() * sizeof(EditB), it_b = item.size() * 8;
    uint8_t *tab = m->edit_part.get<uint8_t>(seg_b + eb_b + it_b + 64);
    WtySeg *dsegs = (WtySeg *)tab;
    EditB *deb = (EditB *)(tab + (seg_b + 15) / 16 * 16);
    int64_t *ditems = (int64_t *)(tab + (seg_b + 15) / 16 * 16 + (eb_b + 15) / 16 * 16);
    DITCH_TRY_HIP(hipMemcpyAsync(dsegs, segs.data(), seg_b, hipMemcpyHostToDevice, s));
    DITCH_TRY_HIP(hipMemcpyAsync(deb, eb.data(), eb_b, hipMemcpyHostToDevice, s));
    DITCH_TRY_HIP(hipMemcpyAsync(ditems, item.data(), it_b, hipMemcpyHostToDevice, s));
    if (one_kind) {
        WtyArgs a{};
        a.segs = dsegs;
        a.items = ditems;
        wty_launch(kind, a, (int64_t)k, (unsigned)items, s);
    } else {
        // matrices of several tile formats (or decodes): one launch per kind
        // over its items (the segment table is shared)
        std::map<int, std::vector<int64_t>> by_kind;
        for (int64_t i = 0; i < items; i++) by_kind[wty_kind(segs[item[i] >> 32].w)].push_back(item[i]);
        int64_t *dst = ditems;
        for (auto &kv : by_kind) {
            DITCH_TRY_HIP(hipMemcpyAsync(dst, kv.second.data(), kv.second.size() * 8, hipMemcpyHostToDevice, s));
            WtyArgs a{};
            a.segs = dsegs;
            a.items = dst;
            wty_launch(kv.first, a, (int64_t)k, (unsigned)kv.second.size(), s);
            dst += kv.second.size();
        }
    }
    const unsigned bx = (unsigned)std::min<int64_t>((max_rows * (int64_t)k + 255) / 256, 64);
    for (size_t r0 = 0; r0 < resident.size(); r0 += 65535) {
        const unsigned ny = (unsigned)std::min<size_t>(resident.size() - r0, 65535);
        hipLaunchKernelGGL(edit_b_kernel, dim3(bx, ny), dim3(256), 0, s, deb + r0, (int64_t)k);
        DITCH_TRY_HIP(hipGetLastError());
    }
    // the host tables above are read by the copies: wait before they go
    DITCH_TRY_HIP(hipStreamSynchronize(s));
    for (size_t r = 0; r < resident.size(); r++) {
        Mat *mt = mats[resident[r]];
        mt->clear_delta();
        mt->da = (float *)segs[r].out;
        mt->db = eb[r].b;
        mt->arena = arena;
        mt->rank = (int)k;
    }
}

}  // namespace ditch
