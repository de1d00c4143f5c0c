// internal.h — shared declarations of libditch_hip (not part of the ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/ditch_hip.h"

namespace ditch {

// ---------------------------------------------------------------------------
// Errors: every entry point returns a status and records a message.

struct Error {
    int32_t code;
    std::string msg;
};

#define DITCH_TRY_HIP(expr)                                                          \
    do {                                                                             \
        hipError_t e_ = (expr);                                                      \
        if (e_ != hipSuccess)                                                        \
            throw ::ditch::Error{e_ == hipErrorOutOfMemory ? DITCH_OUT_OF_MEMORY     \
                                                           : DITCH_DEVICE_FAILED,    \
                                 std::string(#expr) + ": " + hipGetErrorString(e_)}; \
    } while (0)

#define DITCH_CHECK(cond, code, msg)                                  \
    do {                                                              \
        if (!(cond)) throw ::ditch::Error{(code), std::string(msg)}; \
    } while (0)

// ---------------------------------------------------------------------------
// Weight tiles in HBM.
//
// Codes are re-tiled at upload so that one 16-byte load per lane yields the
// lane's B operand of v_mfma_f32_16x16x32_bf16 (weight row n = lane % 16,
// k = 8 * (lane / 16) .. +8 within a 32-wide k tile). A "unit" is 16 weight
// rows by unit_k columns, 64 lanes x 16 bytes (32 for f32):
//   TF_BF16, TF_F16 : unit_k 32,  one k tile per 16 B
//   TF_F32          : unit_k 32,  32 B per lane (two 16 B halves)
//   TF_Q8, TF_FP8   : unit_k 64,  8 codes for each of 2 k tiles
//   TF_MX4, TF_INT4 : unit_k 128, 8 nibbles for each of 4 k tiles
// Units are stored [n / 16][k / unit_k] (k fastest). Rows pad to 16 and
// columns to unit_k with zero codes. Scales stay in plain row-major arrays.
enum TileFormat : int32_t {
    TF_BF16 = 0,
    TF_F16 = 1,
    TF_F32 = 2,
    TF_Q8 = 3,    // GGUF Q8_0: int8 codes, f16 scale per (row, 32 columns)
    TF_FP8 = 4,   // E4M3/E5M2 codes, scale grid
    TF_MX4 = 5,   // E2M1 codes, E8M0 scale per (row, 32 columns)
    TF_INT4 = 6,  // 4-bit pack-quantized: (q - zp) * scale per group
};

__host__ __device__ inline int unit_k_of(int tf) {
    return (tf == TF_Q8 || tf == TF_FP8) ? 64 : (tf == TF_MX4 || tf == TF_INT4) ? 128 : 32;
}
__host__ __device__ inline int unit_bytes_of(int tf) { return tf == TF_F32 ? 2048 : 1024; }

// Kernel-side view of a resident weight (passed by value).
struct TileView {
    const uint8_t *codes;
    const void *scale;      // Q8: f16 [rows][kt]; MX4: u8 [rows][kt]; FP8: grid; INT4: [rows][groups]
    const uint8_t *zero;    // INT4: zero point (field value) [rows][groups], or null
    int32_t tf;
    int32_t scale_type;     // decode.h ScaleType
    int64_t rows, cols;     // logical
    int64_t units_k;        // units per 16-row group
    int64_t scale_cols;     // row stride of the scale array (FP8: grid cols)
    int64_t block_rows, block_cols, row_shard;  // FP8 grid
    int64_t group;          // INT4 group size
    int32_t e5m2;
    int32_t orig_dtype;     // ditch_weight dtype the tensor came from
    // 1 when the gfx950 conversion instructions decode every element of this
    // tensor exactly as the reference does: no E8M0 scale byte 255 (MXFP4),
    // no NaN/Inf codes and finite scales (FP8), finite scales (INT4), and
    // scale blocks that cover whole 64-column stages (FP8 block_cols and
    // INT4 group multiples of 64). Set at upload; the tiled GEMM requires it.
    int32_t fast;
    // per-row side words of the tiled GEMM (fast tensors), one 32-bit word
    // per (row, stage entry): MXFP4 the unit's four E8M0 bytes (aliases
    // `scale`), FP8 the scale grid as f32, INT4 the 16-bit scale bits | the
    // zero field << 16 per group
    const uint32_t *side;
    int64_t side_cols;
    // MXFP4 (fast tensors): the codes once more in the operand order of the
    // scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4): per 16-row group and
    // 128-column unit, lane l holds the 16 source bytes of row l % 16,
    // columns 32 * (l / 16) .. +32 (one E8M0 block), followed by the scales in
    // the same order: per group and unit 64 bytes, byte l = the E8M0 of that
    // lane's block (mx_scales)
    const uint8_t *mx;
    const uint8_t *mx_scales;
};

// Device memory helpers (all on the context stream).
void *dev_alloc(size_t bytes);
void dev_free(void *p);

// A device buffer that grows on demand (contents are not kept on growth).
// A borrowed buffer wraps memory owned elsewhere (the library's static
// scratch array): it never allocates, grows or frees, and a request beyond
// its size is refused before anything is launched on it.
struct DevBuf {
    void *p = nullptr;
    size_t bytes = 0;
    bool borrowed = false;
    DevBuf() = default;
    DevBuf(void *mem, size_t cap) : p(mem), bytes(cap), borrowed(true) {}
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    DevBuf(DevBuf &&o) noexcept : p(o.p), bytes(o.bytes), borrowed(o.borrowed) {
        o.p = nullptr;
        o.bytes = 0;
    }
    DevBuf &operator=(DevBuf &&o) noexcept {
        if (this != &o) {
            if (!borrowed) dev_free(p);
            p = o.p;
            bytes = o.bytes;
            borrowed = o.borrowed;
            o.p = nullptr;
            o.bytes = 0;
        }
        return *this;
    }
    ~DevBuf() {
        if (!borrowed) dev_free(p);
    }
    template <typename T>
    T *get(size_t count) {
        size_t need = count * sizeof(T);
        if (need > bytes) {
            if (borrowed)
                throw Error{DITCH_INVALID_ARGUMENT, "scratch: the call needs " + std::to_string(need) +
                                                        " bytes of scratch, the static scratch holds " +
                                                        std::to_string(bytes)};
            dev_free(p);
            p = nullptr;
            bytes = 0;
            p = dev_alloc(need < 256 ? 256 : need);
            bytes = need;
        }
        return (T *)p;
    }
};

}  // namespace ditch

struct ditch_hip_tensor {
    ditch::TileView v;
    void *codes = nullptr;
    void *scale = nullptr;
    void *zero = nullptr;
    void *side = nullptr;  // owned side words (FP8, INT4); MXFP4 aliases scale
    void *mx = nullptr;    // MXFP4 codes in scaled-MFMA order
    void *mx_scales = nullptr;
    // bytes of codes, scale, zero, side, mx, mx_scales (the owned allocations)
    size_t part_bytes[6] = {0, 0, 0, 0, 0, 0};
    uint64_t bytes = 0;
};

struct ditch_hip {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string name;
    std::string last_error;
    std::mutex mu;
    // scratch buffers reused by the host-memory entry points
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
    int cu_count = 0;
    // activation fragments of the tiled GEMM for the context's own products
    ditch::DevBuf split;
    // per-chunk partials of the row-split log-softmax / KL
    ditch::DevBuf rowred;
    // scratch of the direction pipeline (projections, basis columns)
    ditch::DevBuf dirtmp;
    // the edit's workspace (edit.hip), kept across calls: an edit of
    // thousands of matrices allocates and frees nothing per matrix
    std::shared_ptr<void> edit_work;
    // this device's copy of the static scratch array (api.hip), resolved
    // with hipGetSymbolAddress when the context opens
    void *static_scratch = nullptr;
    std::string scratch_error;
    // registered copies of the weights the per-call entry points receive
    // (tiles.hip, residency_*)
    struct ResidencyEntry {
        const void *data;
        size_t len;
        uint64_t desc;  // hash of the rest of the descriptor
        uint64_t sig;   // hash of sampled bytes of the weight's buffers
        uint64_t bytes; // device bytes of the registered copy
        ditch_hip_tensor *t;
        uint64_t used_at;
    };
    struct Residency {
        uint64_t budget = 0;
        bool stable = false;
        uint64_t used = 0, clock = 0, hits = 0, misses = 0, evictions = 0;
        std::vector<ResidencyEntry> entries;
    } res;
};

namespace ditch {

// tiles.hip
ditch_hip_tensor *upload_weight(ditch_hip *h, const ditch_weight *w, hipStream_t s);
// The bytes an upload of w reads from each of its host pieces (refused when
// the description is inconsistent or its sizes overflow).
struct RawSizes {
    size_t data, scale, zero, gidx;
};
RawSizes raw_sizes(const ditch_weight *w);
void free_tensor(ditch_hip_tensor *t);
// A per-call weight: the residency cache's copy (owned = false) or a fresh
// upload the caller frees (owned = true).
struct WeightRef {
    ditch_hip_tensor *t = nullptr;
    bool owned = false;
    WeightRef() = default;
    WeightRef(const WeightRef &) = delete;
    WeightRef &operator=(const WeightRef &) = delete;
    ditch_hip_tensor *operator->() const { return t; }
    ~WeightRef() {
        if (owned) free_tensor(t);
    }
};
void acquire_weight(ditch_hip *h, const ditch_weight *w, hipStream_t s, WeightRef &ref);
void residency_configure(ditch_hip *h, uint64_t budget, bool stable);
void residency_clear(ditch_hip *h);
void launch_dequant(const TileView &v, void *out, int64_t row0, int64_t nrows, hipStream_t s);
bool is_bf16_virtual(int32_t dtype);

// gemm.hip
struct MatmulEpilogue {
    const float *bias = nullptr;  // [rows]
    int accumulate = 0;           // out += result
    // low-rank delta: out[i][r] += sum_j b[r][j] * xa[i][j]
    const float *delta_b = nullptr;  // [rows][rank]
    const float *delta_xa = nullptr; // [n][rank]
    int delta_rank = 0;
    // three bf16 activation terms instead of two: products exact to f32
    // rounding (the VTable entry point, checked at the reference's
    // device-contract tolerance); the resident forward uses two
    int exact = 0;
};
// `ws` (optional) holds the split activations of the tiled GEMM; without it
// the product runs on the small-batch kernels.
void launch_matmul(const TileView &w, float *out, const float *x, int64_t n, const MatmulEpilogue &ep,
                   hipStream_t s, const int32_t *row_index = nullptr, DevBuf *ws = nullptr);

// gemm_tile.hip: large-batch product on pre-split activation fragments.
// Fragments of an activation [n][K] are stored [n/16][ldk][xt][64 lanes] x
// 16 bytes; split_ldk(K) tiles per block serve every weight format with K
// columns.
bool tile_gemm_takes(const TileView &w, int64_t n);
int64_t split_k_tiles(const TileView &w);  // k tiles a product over w runs
inline int64_t split_ldk(int64_t K) { return (K + 127) / 128 * 4; }
inline size_t split_bytes_ldk(int64_t n, int64_t ldk, int xt) { return (size_t)((n + 15) / 16) * ldk * xt * 1024; }
void launch_split(void *xs, const float *x, const int32_t *row_index, int64_t n, int64_t ldx, int64_t K,
                  int64_t ldk, int xt, hipStream_t s);
// The tiled product over f32 rows x with a delta (ep.delta_b, ep.delta_rank)
// whose x . A^T the activation split forms on the way (one partial sum per
// 32-column k tile, added by a wave per token into xa [n][rank]): one pass
// over x instead of two. False
// (nothing launched) when the tiled product does not take w.
bool launch_matmul_delta_split(const TileView &w, float *out, const float *x, int64_t n, const MatmulEpilogue &ep,
                               const float *da, int rank, float *xa, hipStream_t s, DevBuf *ws);
// part: f32 scratch of tile_part_bytes(w, n, xt) bytes for split-K partial
// sums (NULL: no split)
size_t tile_part_bytes(const TileView &w, int64_t n, int xt);
void launch_tile_gemm(const TileView &w, float *out, int64_t ldo, const void *xs, int64_t ldk, int64_t n, int xt,
                      const MatmulEpilogue &ep, hipStream_t s, float *part = nullptr);
// gate/up in one product: act(x gate^T) * (x up^T) into f32 rows [n][rows]
// (out, may be NULL) and/or the A fragments of the next product (xs_out)
// MXFP4 large batches on the scaled MFMA (fp6 activation terms x the fp4
// codes): fragments [ceil(n/16)][ldst] x 6400 B, ldst >= cols / 128.
bool mx_gemm_takes(const TileView &w, int64_t n);
size_t mx_frag_bytes(int64_t n, int64_t ldst);
void launch_split_mx(void *xm, const float *x, const int32_t *row_index, int64_t n, int64_t ldx, int64_t K,
                     int64_t ldst, hipStream_t s);
void launch_mx_gemm(const TileView &w, float *out, int64_t ldo, const void *xm, int64_t ldst, int64_t n,
                    const MatmulEpilogue &ep, hipStream_t s);
// act(x gate^T) * (x up^T) in one scaled-MFMA pass: f32 rows [n][rows] (out,
// optional) and/or the MX fragments of a product over them (xm_out, ldst_out
// stages of 128 columns; optional).
bool mx_glu_takes(const TileView &gate, const TileView &up, int64_t n);
void launch_mx_glu(const TileView &gate, const TileView &up, uint32_t act, float *out, void *xm_out, int64_t ldst_out,
                   const void *xm, int64_t ldst, int64_t n, hipStream_t s);
bool tile_glu_takes(const TileView &gate, const TileView &up, int64_t n);
void launch_tile_glu(const TileView &gate, const TileView &up, uint32_t act, float *out, void *xs_out,
                     int64_t ldk_out, const void *xs, int64_t ldk, int64_t n, hipStream_t s);

// An activation [n][K] handed to a product: f32 rows, pre-split fragments
// (xt = 2 terms, stride ldk), or both.
struct Act {
    const float *f32 = nullptr;
    const void *xs = nullptr;  // bf16-term fragments, ldk k tiles per 16 tokens
    int64_t ldk = 0;
    const void *xm = nullptr;  // MX fragments, ldst stages per 16 tokens
    int64_t ldst = 0;
};
void launch_matmul_act(const TileView &w, float *out, const Act &x, int64_t n, const MatmulEpilogue &ep,
                       hipStream_t s, DevBuf *ws);
// One product per segment (routed experts): segment z multiplies rows
// [off, off + cnt) of x (through row_index when given) by its own weight
// into rows [off, off + cnt) of out. Every segment has rows x cols weights
// of tile format tf.
struct GroupSeg {
    TileView w;
    int64_t off, cnt;
    const float *delta_b;
    int delta_rank;
};
// h_segs: the same table on the host (counts and offsets decide the path);
// ws and meta: workspaces for activation fragments and the tile table
void launch_matmul_grouped(const GroupSeg *d_segs, const GroupSeg *h_segs, unsigned nseg, int tf, int64_t rows,
                           int64_t cols, int64_t max_cnt, float *out, const float *x, const int32_t *row_index,
                           const float *delta_xa, int delta_stride, hipStream_t s, DevBuf *ws, DevBuf *meta);
bool tile_grouped_takes(const GroupSeg *h_segs, unsigned nseg, int64_t max_cnt);
// xs_pre: the activation fragments already split in the grouped row order
// (grouped_blocks(h_segs) 16-token blocks of split_k_tiles(w) k tiles);
// NULL: split x here
void launch_tile_gemm_grouped(const GroupSeg *d_segs, const GroupSeg *h_segs, unsigned nseg, float *out, int64_t ldo,
                              const float *x, int64_t ldx, const int32_t *row_index, const float *delta_xa,
                              int delta_stride, DevBuf *ws, DevBuf *meta, hipStream_t s, const void *xs_pre = nullptr);
int64_t grouped_blocks(const GroupSeg *h_segs, unsigned nseg);
// A grouped call planned on the device: prow [max_blocks * 16] (fragment row
// -> gathered row, -1 for zero rows), desc [max_desc][4] (segment, first
// block, segment's block end, first token within the segment), *count tile
// rows in use; the segment table's off/cnt written on the device too.
struct GroupedDevPlan {
    int32_t *prow, *desc, *count;
    int64_t max_blocks, max_desc;
};
// The routed down projections' delta products, formed by the grouped GLU:
// xa [pairs][max_rank] = act(gate) * up . A_z^T for each pair's segment z
// (a[z] the down projection's delta A, segs[z].delta_rank its rank, 0: no
// delta); ws holds the per-wave partial sums.
struct GroupedDeltaXa {
    const float *const *a;
    const GroupSeg *segs;
    float *xa;
    int64_t pairs;
    int max_rank;
    DevBuf *ws;
};
// out (may be NULL): act(gate) * up as f32 rows in the grouped row order;
// dx (may be NULL): the delta products as well; n_tok > 0: x holds n_tok
// token rows split once token-major and gathered by the tiles (row_index:
// pair -> token), else the pairs' rows are split in fragment order
void launch_tile_glu_grouped_dev(const GroupSeg *d_gate, const GroupSeg *d_up, const TileView &gate0,
                                 const TileView &up0, uint32_t act, float *out, void *xs_out, int64_t ldk_out,
                                 const float *x, int64_t ldx, const int32_t *row_index, const GroupedDevPlan &plan,
                                 DevBuf *ws, hipStream_t s, const GroupedDeltaXa *dx = nullptr, int64_t n_tok = 0);
// delta_xa [rows][delta_stride]: the x . A^T of the segments' deltas (their
// B and rank in the segment table), or NULL
void launch_tile_gemm_grouped_dev(const GroupSeg *d_segs, const TileView &w0, float *out, int64_t ldo,
                                  const void *xs, const GroupedDevPlan &plan, hipStream_t s,
                                  const float *delta_xa = nullptr, int delta_stride = 0);
// Routed gate/up in one tiled product: act(x gate_z^T) * (x up_z^T) per
// segment z, as f32 rows of out (may be NULL) and as the down product's
// activation fragments xs_out (ldk_out k tiles, grouped row order). n_tok >
// 0: x holds n_tok token rows, split once token-major and gathered per pair
// by the tiles (cheaper than splitting every pair's row when the segments
// cover at least n_tok pairs).
void launch_tile_glu_grouped(const GroupSeg *d_gate, const GroupSeg *d_up, const GroupSeg *h_gate,
                             const GroupSeg *h_up, unsigned nseg, uint32_t act, float *out, void *xs_out,
                             int64_t ldk_out, const float *x, int64_t ldx, const int32_t *row_index, DevBuf *ws,
                             DevBuf *meta, hipStream_t s, int64_t n_tok = 0);

// attention.hip: prompt attention (model.zig:2935-2986) on the fp32 MFMA for
// the head shapes it takes; q [n][heads][hd], caches [prompt][T][kvd], out
// [n][heads][vd]
struct AttnArgs {
    const float *q, *kc, *vc;
    float *out;
    const ditch_row *rows;
    int64_t n, heads, groups, hd, vd, T, kvd;
    float scale;
    // optional: the output also as the tiled GEMM's A fragments (k = head *
    // vd + dim; heads * vd a multiple of 128)
    void *xs;
    int64_t ldk;
    int64_t nb;  // prompt slots of the KV cache: rows with b >= nb or pos >= T are skipped
    // optional: the flag launch_attention_dense_check wrote for these rows
    // (1: dense, row r = prompt r / T at position r % T); the whole-prompt
    // kernel then takes them and the per-block kernel's workgroups exit
    const int *dense;
};
bool attention_mfma_takes(int64_t hd, int64_t vd, int64_t groups);
bool attention_prompt_takes(int64_t hd, int64_t vd, int64_t T);
void launch_attention_dense_check(const ditch_row *rows, int64_t n, int64_t T, int64_t nb, int *flag, hipStream_t s);
void launch_attention_mfma(const AttnArgs &a, int64_t kv_heads, hipStream_t s);

// ops.hip
// row_index (optional) gathers input rows out of n_src rows
void launch_rmsnorm(float *out, const float *x, const float *w, int64_t wlen, int64_t n, int64_t len,
                    float eps, int gemma, hipStream_t s, const int64_t *row_index = nullptr, int64_t n_src = 0);
// RMS norm into the tiled GEMM's A fragments (and f32 rows when out != NULL)
void launch_rmsnorm_split_mx(void *xm, int64_t ldst, float *out, const float *x, const float *w, int64_t wlen,
                             int64_t n, int64_t len, float eps, int gemma, hipStream_t s);
void launch_rmsnorm_split(void *xs, int64_t ldk, float *out, const float *x, const float *w, int64_t wlen, int64_t n,
                          int64_t len, float eps, int gemma, hipStream_t s);
void launch_rmsnorm_strided(float *out, const float *x, const float *w, int64_t wlen, int64_t n, int64_t len,
                            int64_t in_stride, int64_t out_stride, float eps, hipStream_t s);
void launch_layernorm(float *out, const float *x, const float *w, int64_t wlen, const float *bias, int64_t n,
                      int64_t len, float eps, int one_plus, hipStream_t s);
void launch_softmax_rows(float *x, int64_t n, int64_t len, hipStream_t s);
// generate.hip
void launch_pick(uint32_t *out, const float *logits, int64_t n, int64_t vocab, ditch_sampler *smp, hipStream_t s);
void sampler_init(ditch_sampler *smp, uint64_t seed, float temperature, uint64_t top_k, float top_p);

// edit.hip
void edit_gaussian(float *out, size_t n, uint64_t seed);
int64_t edit_rank(int64_t rows, int64_t cols, int64_t k, int mode, int64_t lora_rank, int ablate);
// (h: the context whose edit workspace the passes use)
void edit_delta_device(ditch_hip *h, const TileView &w, const float *hv, int64_t k, float weight, int mode,
                       int64_t lora_rank, uint64_t seed, int ablate, hipStream_t s, float **da_out, float **db_out,
                       int64_t *rank_out);

// directions.hip
void launch_residual_reduce(const float *res, int64_t entries, int64_t n_capture, int64_t hidden,
                            const uint32_t *first, const uint32_t *take, int64_t prompts, float q, float *vout,
                            double *sum, double *sq, hipStream_t s);
void launch_residual_mean(float *mean, const double *sum, uint64_t count, int64_t n, hipStream_t s);
void launch_directions(float *dirs, const float *good, const float *bad, int64_t entries, int64_t hidden,
                       int orthogonalize, hipStream_t s, DevBuf *tmp);
void launch_sketch_add(double *y, double *w, const float *omega, int64_t m, const float *center, const float *v,
                       int64_t prompts, int64_t entries, int64_t hidden, hipStream_t s, DevBuf *tmp);
void launch_basis(float *dirs, const float *first, const float *good, int64_t entries, int64_t hidden, int64_t k,
                  int orthogonalize, const double *y, const double *w, int64_t m, hipStream_t s, DevBuf *tmp);

// `tmp` holds the per-chunk partials (3 * n * chunks doubles)
void launch_log_softmax_rows(float *out, const float *x, int64_t n, int64_t len, hipStream_t s, DevBuf *tmp);
void launch_kl_rows(double *kl, const float *base, const float *trial, int64_t n, int64_t vocab, hipStream_t s,
                    DevBuf *tmp);
void launch_gated_act(uint32_t act, float *out, const float *gate, const float *up, int64_t n, int64_t len,
                      int64_t in_stride, int64_t out_stride, hipStream_t s);
void launch_rope_rows(float *x, int64_t n, int64_t dim, const float *cos_t, const float *sin_t, int64_t half,
                      const uint32_t *pos, uint32_t style, hipStream_t s);
void launch_attention_scores(float *scores, int64_t n_keys, const float *q, int64_t hd, const float *k,
                             int64_t stride, float scale, hipStream_t s);
void launch_attention_values(float *out, int64_t vd, const float *scores, int64_t n_keys, const float *v,
                             int64_t stride, hipStream_t s);
void launch_row_norms(float *out, const TileView &w, hipStream_t s);
// out[q][cols] = y[q][rows] . W over the resident tiles (edit_batch.hip)
void launch_matvecT(float *out, const TileView &w, const float *y, int64_t q, hipStream_t s);
void launch_delta_xa(float *xa, const float *x, const float *a, int64_t n, int64_t cols, int64_t rank,
                     hipStream_t s);

}  // namespace ditch
