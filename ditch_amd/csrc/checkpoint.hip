// checkpoint.hip — reads a checkpoint from disk into a resident model: a
// Hugging Face directory (config.json + *.safetensors shards, safetensors.zig;
// quantised tensors kept packed: FP8 with block scales, compressed-tensors
// pack-quantized INT and mxfp4-pack-quantized, dequant.zig:108-233,
// 855-947, 1072-1187) or a GGUF v3 file (gguf.zig, gguf_model.zig; block
// types kept packed). Files are memory-mapped; each weight's pieces (codes,
// scales, zero points, g_idx) are copied into pinned host memory and handed
// to the device registration, which copies them to HBM and re-tiles them.
// The families are those of the benchmark configurations: llama, qwen2,
// qwen3 / qwen3_moe and deepseek_v3 (config keys as models/*.lua read them).
#include <fcntl.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <dirent.h>

#include <algorithm>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "internal.h"
#include "model.h"

namespace ditch {

ditch_hip_model *model_create(ditch_hip *h, const ditch_model_config *cfg);
void model_set(ditch_hip_model *m, int layer, int slot, int expert, const ditch_weight *w);

// ---------------------------------------------------------------------------
// JSON (config.json and safetensors headers)

struct JVal {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    double num = 0;
    std::string str;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;

    const JVal *get(const std::string &k) const {
        if (kind != OBJ) return nullptr;
        for (const auto &kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
    bool has(const std::string &k) const {
        const JVal *v = get(k);
        return v && v->kind != NUL;
    }
    double num_or(const std::string &k, double dflt) const {
        const JVal *v = get(k);
        if (!v || v->kind == NUL) return dflt;
        if (v->kind == BOOL) return v->b ? 1 : 0;
        return v->kind == NUM ? v->num : dflt;
    }
    std::string str_or(const std::string &k, const std::string &dflt) const {
        const JVal *v = get(k);
        return v && v->kind == STR ? v->str : dflt;
    }
};

struct JParser {
    const char *p, *end;
    [[noreturn]] void fail(const char *what) { throw Error{DITCH_INVALID_ARGUMENT, std::string("json: ") + what}; }
    void ws() {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++;
    }
    static void put_utf8(std::string &s, uint32_t c) {
        if (c < 0x80) s += (char)c;
        else if (c < 0x800) {
            s += (char)(0xC0 | (c >> 6));
            s += (char)(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            s += (char)(0xE0 | (c >> 12));
            s += (char)(0x80 | ((c >> 6) & 0x3F));
            s += (char)(0x80 | (c & 0x3F));
        } else {
            s += (char)(0xF0 | (c >> 18));
            s += (char)(0x80 | ((c >> 12) & 0x3F));
            s += (char)(0x80 | ((c >> 6) & 0x3F));
            s += (char)(0x80 | (c & 0x3F));
        }
    }
    uint32_t hex4() {
        if (end - p < 4) fail("short \\u escape");
        uint32_t v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else fail("bad \\u escape");
        }
        return v;
    }
    std::string string() {
        if (p >= end || *p != '"') fail("string expected");
        p++;
        std::string s;
        while (p < end && *p != '"') {
            if (*p == '\\') {
                if (++p >= end) fail("bad escape");
                const char e = *p++;
                switch (e) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    uint32_t c = hex4();
                    if (c >= 0xD800 && c < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                        p += 2;
                        const uint32_t lo = hex4();
                        c = 0x10000 + ((c - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(s, c);
                    break;
                }
                default: fail("bad escape");
                }
            } else {
                s += *p++;
            }
        }
        if (p >= end) fail("unterminated string");
        p++;
        return s;
    }
    JVal value(int depth = 0) {
        if (depth > 64) fail("nesting too deep");
        ws();
        if (p >= end) fail("unexpected end");
        JVal v;
        if (*p == '{') {
            v.kind = JVal::OBJ;
            p++;
            ws();
            if (p < end && *p == '}') {
                p++;
                return v;
            }
            for (;;) {
                ws();
                std::string k = string();
                ws();
                if (p >= end || *p != ':') fail("':' expected");
                p++;
                v.obj.emplace_back(std::move(k), value(depth + 1));
                ws();
                if (p < end && *p == ',') {
                    p++;
                    continue;
                }
                if (p < end && *p == '}') {
                    p++;
                    return v;
                }
                fail("',' or '}' expected");
            }
        }
        if (*p == '[') {
            v.kind = JVal::ARR;
            p++;
            ws();
            if (p < end && *p == ']') {
                p++;
                return v;
            }
            for (;;) {
                v.arr.push_back(value(depth + 1));
                ws();
                if (p < end && *p == ',') {
                    p++;
                    continue;
                }
                if (p < end && *p == ']') {
                    p++;
                    return v;
                }
                fail("',' or ']' expected");
            }
        }
        if (*p == '"') {
            v.kind = JVal::STR;
            v.str = string();
            return v;
        }
        if (end - p >= 4 && !strncmp(p, "true", 4)) {
            v.kind = JVal::BOOL;
            v.b = true;
            p += 4;
            return v;
        }
        if (end - p >= 5 && !strncmp(p, "false", 5)) {
            v.kind = JVal::BOOL;
            p += 5;
            return v;
        }
        if (end - p >= 4 && !strncmp(p, "null", 4)) {
            p += 4;
            return v;
        }
        // number
        std::string t;
        while (p < end && (isdigit((unsigned char)*p) || *p == '-' || *p == '+' || *p == '.' || *p == 'e' || *p == 'E'))
            t += *p++;
        if (t.empty()) fail("value expected");
        v.kind = JVal::NUM;
        v.num = strtod(t.c_str(), nullptr);
        return v;
    }
};

static JVal parse_json(const char *p, size_t n) {
    JParser jp{p, p + n};
    JVal v = jp.value();
    return v;
}

// ---------------------------------------------------------------------------
// mapped files and pinned staging

struct Mapped {
    int fd = -1;
    const uint8_t *base = nullptr;
    size_t size = 0;
    std::string path;
    explicit Mapped(const std::string &p) : path(p) {
        fd = open(p.c_str(), O_RDONLY);
        DITCH_CHECK(fd >= 0, DITCH_INVALID_ARGUMENT, "checkpoint: cannot open " + p);
        struct stat st;
        if (fstat(fd, &st) != 0) {
            close(fd);
            throw Error{DITCH_INVALID_ARGUMENT, "checkpoint: cannot stat " + p};
        }
        size = (size_t)st.st_size;
        if (size) {
            void *m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
            if (m == MAP_FAILED) {
                close(fd);
                throw Error{DITCH_INVALID_ARGUMENT, "checkpoint: cannot map " + p};
            }
            base = (const uint8_t *)m;
        }
    }
    ~Mapped() {
        if (base) munmap((void *)base, size);
        if (fd >= 0) close(fd);
    }
    Mapped(const Mapped &) = delete;
    Mapped &operator=(const Mapped &) = delete;
};

// Pinned host memory for one weight's pieces at a time (reset per weight).
struct PinnedStage {
    uint8_t *buf = nullptr;
    size_t cap = 0, used = 0;
    ~PinnedStage() {
        if (buf) (void)hipHostFree(buf);
    }
    void reserve(size_t bytes) {
        if (bytes <= cap) return;
        if (buf) DITCH_TRY_HIP(hipHostFree(buf));
        buf = nullptr;
        cap = 0;
        DITCH_TRY_HIP(hipHostMalloc((void **)&buf, bytes, hipHostMallocDefault));
        cap = bytes;
    }
    void reset() { used = 0; }
    uint8_t *take(size_t bytes) {
        const size_t at = (used + 255) & ~(size_t)255;
        DITCH_CHECK(at + bytes <= cap, DITCH_DEVICE_FAILED, "checkpoint: staging overflow");
        used = at + bytes;
        return buf + at;
    }
};

// ---------------------------------------------------------------------------
// safetensors (safetensors.zig): an 8-byte header length, a JSON header of
// name -> {dtype, shape, data_offsets}, then the data

struct StTensor {
    const Mapped *file = nullptr;
    std::string dtype;
    std::vector<int64_t> shape;
    size_t begin = 0, end = 0;  // absolute offsets in the file
    const uint8_t *data() const { return file->base + begin; }
    size_t bytes() const { return end - begin; }
    int64_t numel() const {  // -1 when a dimension is negative or the product overflows
        int64_t n = 1;
        for (int64_t d : shape)
            if (d < 0 || __builtin_mul_overflow(n, d, &n)) return -1;
        return n;
    }
};

static size_t st_elem_bytes(const std::string &dt) {
    if (dt == "F32" || dt == "I32" || dt == "U32") return 4;
    if (dt == "F16" || dt == "BF16" || dt == "I16" || dt == "U16") return 2;
    if (dt == "F8_E4M3" || dt == "F8_E5M2" || dt == "U8" || dt == "I8" || dt == "BOOL" || dt == "F8_E8M0") return 1;
    if (dt == "I64" || dt == "U64" || dt == "F64") return 8;
    return 0;
}

static void read_safetensors(const Mapped &f, std::map<std::string, StTensor> &out) {
    DITCH_CHECK(f.size >= 8, DITCH_INVALID_ARGUMENT, "safetensors: short file " + f.path);
    uint64_t n;
    memcpy(&n, f.base, 8);
    DITCH_CHECK(n <= f.size - 8, DITCH_INVALID_ARGUMENT, "safetensors: header past the end of " + f.path);
    const JVal hdr = parse_json((const char *)f.base + 8, (size_t)n);
    DITCH_CHECK(hdr.kind == JVal::OBJ, DITCH_INVALID_ARGUMENT, "safetensors: header is not an object");
    const size_t base = 8 + (size_t)n;
    for (const auto &kv : hdr.obj) {
        if (kv.first == "__metadata__") continue;
        const JVal &t = kv.second;
        StTensor st;
        st.file = &f;
        st.dtype = t.str_or("dtype", "");
        const JVal *shape = t.get("shape"), *off = t.get("data_offsets");
        DITCH_CHECK(shape && shape->kind == JVal::ARR && off && off->kind == JVal::ARR && off->arr.size() == 2,
                    DITCH_INVALID_ARGUMENT, "safetensors: bad entry " + kv.first);
        for (const JVal &d : shape->arr) st.shape.push_back((int64_t)d.num);
        st.begin = base + (size_t)off->arr[0].num;
        st.end = base + (size_t)off->arr[1].num;
        const size_t eb = st_elem_bytes(st.dtype);
        DITCH_CHECK(eb && st.numel() >= 0 && st.begin <= st.end && st.end <= f.size &&
                        (uint64_t)st.numel() <= UINT64_MAX / eb && st.bytes() == (size_t)st.numel() * eb,
                    DITCH_INVALID_ARGUMENT, "safetensors: entry " + kv.first + " out of range or of unknown dtype");
        out[kv.first] = st;
    }
}

// ---------------------------------------------------------------------------
// GGUF v3 (gguf.zig): header, metadata, tensor infos, aligned data

struct GgufMeta {
    enum Kind { U, I, F, B, S, A } kind = U;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0;
    std::string s;
    std::vector<GgufMeta> a;
    double as_num() const { return kind == U ? (double)u : kind == I ? (double)i : kind == F ? f : kind == B ? u : 0; }
};

struct GgufTensor {
    std::string type;  // F32, F16, BF16, Q8_0, ...
    int64_t rows = 0, cols = 0;
    const uint8_t *data = nullptr;
    size_t bytes = 0;
};

struct GgufReader {
    const Mapped &f;
    size_t pos = 0;
    explicit GgufReader(const Mapped &m) : f(m) {}
    void need(size_t n) {
        DITCH_CHECK(n <= f.size && pos <= f.size - n, DITCH_INVALID_ARGUMENT, "gguf: truncated " + f.path);
    }
    template <typename T>
    T take() {
        need(sizeof(T));
        T v;
        memcpy(&v, f.base + pos, sizeof(T));
        pos += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = take<uint64_t>();
        need(n);
        std::string s((const char *)f.base + pos, (size_t)n);
        pos += n;
        return s;
    }
    GgufMeta value(uint32_t t, int depth = 0) {
        DITCH_CHECK(depth < 4, DITCH_INVALID_ARGUMENT, "gguf: nested arrays");
        GgufMeta m;
        switch (t) {
        case 0: m.kind = GgufMeta::U; m.u = take<uint8_t>(); break;
        case 1: m.kind = GgufMeta::I; m.i = take<int8_t>(); break;
        case 2: m.kind = GgufMeta::U; m.u = take<uint16_t>(); break;
        case 3: m.kind = GgufMeta::I; m.i = take<int16_t>(); break;
        case 4: m.kind = GgufMeta::U; m.u = take<uint32_t>(); break;
        case 5: m.kind = GgufMeta::I; m.i = take<int32_t>(); break;
        case 6: m.kind = GgufMeta::F; m.f = take<float>(); break;
        case 7: m.kind = GgufMeta::B; m.u = take<uint8_t>(); break;
        case 8: m.kind = GgufMeta::S; m.s = str(); break;
        case 9: {
            m.kind = GgufMeta::A;
            const uint32_t it = take<uint32_t>();
            const uint64_t n = take<uint64_t>();
            DITCH_CHECK(n <= f.size, DITCH_INVALID_ARGUMENT, "gguf: array length");
            if (it == 8 || it == 9) {  // strings (tokenizer tables): skipped, not kept
                for (uint64_t k = 0; k < n; k++) (void)value(it, depth + 1);
            } else {
                m.a.reserve((size_t)n);
                for (uint64_t k = 0; k < n; k++) m.a.push_back(value(it, depth + 1));
            }
            break;
        }
        case 10: m.kind = GgufMeta::U; m.u = take<uint64_t>(); break;
        case 11: m.kind = GgufMeta::I; m.i = take<int64_t>(); break;
        case 12: m.kind = GgufMeta::F; m.f = take<double>(); break;
        default: throw Error{DITCH_INVALID_ARGUMENT, "gguf: value type " + std::to_string(t)};
        }
        return m;
    }
};

static bool gguf_block(uint32_t t, std::string &name, int64_t &bs, int64_t &bb) {
    switch (t) {
    case 0: name = "F32"; bs = 1; bb = 4; return true;
    case 1: name = "F16"; bs = 1; bb = 2; return true;
    case 2: name = "Q4_0"; bs = 32; bb = 18; return true;
    case 3: name = "Q4_1"; bs = 32; bb = 20; return true;
    case 6: name = "Q5_0"; bs = 32; bb = 22; return true;
    case 7: name = "Q5_1"; bs = 32; bb = 24; return true;
    case 8: name = "Q8_0"; bs = 32; bb = 34; return true;
    case 12: name = "Q4_K"; bs = 256; bb = 144; return true;
    case 14: name = "Q6_K"; bs = 256; bb = 210; return true;
    case 15: name = "Q8_K"; bs = 256; bb = 292; return true;
    case 30: name = "BF16"; bs = 1; bb = 2; return true;
    default: return false;
    }
}

static void read_gguf(const Mapped &f, std::map<std::string, GgufMeta> &meta, std::map<std::string, GgufTensor> &out) {
    GgufReader r(f);
    r.need(4);
    DITCH_CHECK(!memcmp(f.base, "GGUF", 4), DITCH_INVALID_ARGUMENT, "gguf: bad magic in " + f.path);
    r.pos = 4;
    const uint32_t version = r.take<uint32_t>();
    DITCH_CHECK(version >= 2 && version <= 3, DITCH_UNSUPPORTED, "gguf: version " + std::to_string(version));
    const uint64_t n_tensors = r.take<uint64_t>(), n_kv = r.take<uint64_t>();
    for (uint64_t k = 0; k < n_kv; k++) {
        std::string key = r.str();
        const uint32_t t = r.take<uint32_t>();
        meta[key] = r.value(t);
    }
    struct Info {
        std::string name, type;
        int64_t rows, cols, bs, bb;
        uint64_t off;
    };
    std::vector<Info> infos;
    for (uint64_t k = 0; k < n_tensors; k++) {
        Info in;
        in.name = r.str();
        const uint32_t nd = r.take<uint32_t>();
        DITCH_CHECK(nd >= 1 && nd <= 4, DITCH_INVALID_ARGUMENT, "gguf: tensor rank");
        std::vector<uint64_t> dims(nd);
        for (uint32_t d = 0; d < nd; d++) dims[d] = r.take<uint64_t>();
        const uint32_t tt = r.take<uint32_t>();
        in.off = r.take<uint64_t>();
        DITCH_CHECK(gguf_block(tt, in.type, in.bs, in.bb), DITCH_UNSUPPORTED,
                    "gguf: tensor type " + std::to_string(tt) + " of " + in.name);
        DITCH_CHECK(dims[0] < (1ull << 40), DITCH_INVALID_ARGUMENT, "gguf: dimensions of " + in.name);
        in.cols = (int64_t)dims[0];
        in.rows = 1;
        for (uint32_t d = 1; d < nd; d++)
            DITCH_CHECK(dims[d] < (1ull << 40) && !__builtin_mul_overflow(in.rows, (int64_t)dims[d], &in.rows),
                        DITCH_INVALID_ARGUMENT, "gguf: dimensions of " + in.name);
        infos.push_back(in);
    }
    uint64_t align = 32;
    auto a = meta.find("general.alignment");
    if (a != meta.end()) align = (uint64_t)a->second.as_num();
    DITCH_CHECK(align >= 1, DITCH_INVALID_ARGUMENT, "gguf: alignment");
    const size_t base = (r.pos + align - 1) / align * align;
    for (const Info &in : infos) {
        DITCH_CHECK(in.cols % in.bs == 0, DITCH_INVALID_ARGUMENT, "gguf: row of " + in.name + " not whole blocks");
        GgufTensor g;
        g.type = in.type;
        g.rows = in.rows;
        g.cols = in.cols;
        int64_t nb = 0;
        DITCH_CHECK(in.rows >= 0 && in.cols >= 0 && !__builtin_mul_overflow(in.rows, in.cols / in.bs, &nb) &&
                        !__builtin_mul_overflow(nb, in.bb, &nb),
                    DITCH_INVALID_ARGUMENT, "gguf: size of tensor " + in.name + " overflows");
        g.bytes = (size_t)nb;
        DITCH_CHECK(in.off <= f.size && base <= f.size - in.off && g.bytes <= f.size - base - in.off, DITCH_INVALID_ARGUMENT,
                    "gguf: tensor " + in.name + " past the end of the file");
        g.data = f.base + base + in.off;
        out[in.name] = g;
    }
}

// ---------------------------------------------------------------------------
// weights: the pieces of a (possibly quantised) matrix copied into pinned
// memory and described as a ditch_weight

static int32_t st_plain_dtype(const std::string &dt) {
    if (dt == "F32") return DITCH_F32;
    if (dt == "F16") return DITCH_F16;
    if (dt == "BF16") return DITCH_BF16;
    return -1;
}

struct HfWeights {
    std::map<std::string, StTensor> t;
    // quantisation (dequant.zig:108-233)
    int fp8_block_rows = 0, fp8_block_cols = 0;
    int int_bits = 0;
    int64_t int_group = 0;
    bool mxfp4_packed = false;

    const StTensor *find(const std::string &n) const {
        auto it = t.find(n);
        return it == t.end() ? nullptr : &it->second;
    }
    const StTensor &at(const std::string &n) const {
        const StTensor *s = find(n);
        DITCH_CHECK(s, DITCH_INVALID_ARGUMENT, "checkpoint: tensor " + n + " missing");
        return *s;
    }
};

static const uint8_t *stage_copy(PinnedStage &ps, const uint8_t *src, size_t n) {
    uint8_t *d = ps.take(n);
    memcpy(d, src, n);
    return d;
}

// The bytes the upload will read from each piece of w (its shape and
// quantisation description) must lie inside what was staged for it, or a
// checkpoint whose tensors disagree with each other would be read past the
// end of the staging buffer.
static ditch_weight staged_checked(const ditch_weight &w, const std::string &prefix, size_t data, size_t scale = 0,
                                   size_t zero = 0, size_t gidx = 0) {
    const RawSizes z = raw_sizes(&w);
    DITCH_CHECK(z.data <= data && z.scale <= scale && z.zero <= zero && z.gidx <= gidx, DITCH_INVALID_ARGUMENT,
                "checkpoint: " + prefix + ": the tensors hold fewer bytes than its shape needs");
    return w;
}

// The matrix at `prefix` (...proj): plain, FP8, pack-quantized INT or
// mxfp4-pack-quantized, its pieces in `ps`.
static ditch_weight hf_weight(const HfWeights &hw, const std::string &prefix, PinnedStage &ps) {
    ditch_weight w{};
    ps.reset();
    if (const StTensor *packed = hw.find(prefix + ".weight_packed")) {
        const StTensor &sc = hw.at(prefix + ".weight_scale");
        if (hw.mxfp4_packed || packed->dtype == "U8") {
            // mxfp4-pack-quantized: codes U8 [rows][cols/2], E8M0 scales U8 [rows][cols/32]
            DITCH_CHECK(packed->shape.size() == 2 && sc.dtype == "U8", DITCH_INVALID_ARGUMENT,
                        "checkpoint: MXFP4 tensor " + prefix);
            ps.reserve(packed->bytes() + sc.bytes() + 1024);
            w.dtype = DITCH_MXFP4;
            w.rows = (uint64_t)packed->shape[0];
            w.cols = (uint64_t)packed->shape[1] * 2;
            w.data = stage_copy(ps, packed->data(), packed->bytes());
            w.scale = stage_copy(ps, sc.data(), sc.bytes());
            w.scale_dtype = DITCH_E8M0;
            return staged_checked(w, prefix, packed->bytes(), sc.bytes());
        }
        const StTensor &shape = hw.at(prefix + ".weight_shape");
        DITCH_CHECK(shape.dtype == "I64" && shape.numel() == 2 && sc.shape.size() == 2, DITCH_INVALID_ARGUMENT,
                    "checkpoint: pack-quantized tensor " + prefix);
        int64_t rc[2];
        memcpy(rc, shape.data(), 16);
        DITCH_CHECK(rc[0] > 0 && rc[1] > 0, DITCH_INVALID_ARGUMENT, "checkpoint: weight_shape of " + prefix);
        const StTensor *zp = hw.find(prefix + ".weight_zero_point"), *gi = hw.find(prefix + ".weight_g_idx");
        ps.reserve(packed->bytes() + sc.bytes() + (zp ? zp->bytes() : 0) + (gi ? gi->bytes() : 0) + 2048);
        w.dtype = DITCH_INT_PACKED;
        w.rows = (uint64_t)rc[0];
        w.cols = (uint64_t)rc[1];
        w.data = stage_copy(ps, packed->data(), packed->bytes());
        w.scale = stage_copy(ps, sc.data(), sc.bytes());
        w.scale_dtype = st_plain_dtype(sc.dtype);
        DITCH_CHECK(w.scale_dtype >= 0, DITCH_UNSUPPORTED, "checkpoint: scale dtype of " + prefix);
        w.scale_rows = (uint64_t)sc.shape[0];
        w.scale_cols = (uint64_t)sc.shape[1];
        w.bits = hw.int_bits ? hw.int_bits : 4;
        w.group = hw.int_group ? (uint64_t)hw.int_group : (w.cols + w.scale_cols - 1) / w.scale_cols;
        if (zp) w.zero = stage_copy(ps, zp->data(), zp->bytes());
        if (gi) {
            DITCH_CHECK(gi->dtype == "I32" && (uint64_t)gi->numel() == w.cols, DITCH_INVALID_ARGUMENT,
                        "checkpoint: g_idx of " + prefix);
            w.g_idx = (const int32_t *)stage_copy(ps, gi->data(), gi->bytes());
        }
        DITCH_CHECK(w.scale_rows >= w.rows, DITCH_INVALID_ARGUMENT, "checkpoint: scale rows of " + prefix);
        return staged_checked(w, prefix, packed->bytes(), sc.bytes(), zp ? zp->bytes() : 0, gi ? gi->bytes() : 0);
    }
    const StTensor &wt = hw.at(prefix + ".weight");
    DITCH_CHECK(wt.shape.size() == 2, DITCH_INVALID_ARGUMENT, "checkpoint: " + prefix + " is not a matrix");
    w.rows = (uint64_t)wt.shape[0];
    w.cols = (uint64_t)wt.shape[1];
    if (wt.dtype == "F8_E4M3" || wt.dtype == "F8_E5M2") {
        const StTensor *sc = hw.find(prefix + ".weight_scale_inv");
        if (!sc) sc = &hw.at(prefix + ".weight_scale");
        DITCH_CHECK(sc->shape.size() == 2, DITCH_INVALID_ARGUMENT, "checkpoint: FP8 scale grid of " + prefix);
        ps.reserve(wt.bytes() + sc->bytes() + 1024);
        w.dtype = DITCH_FP8;
        w.fp8_e5m2 = wt.dtype == "F8_E5M2";
        w.data = stage_copy(ps, wt.data(), wt.bytes());
        w.scale = stage_copy(ps, sc->data(), sc->bytes());
        w.scale_dtype = sc->dtype == "F8_E8M0" || sc->dtype == "U8" ? DITCH_E8M0 : st_plain_dtype(sc->dtype);
        DITCH_CHECK(w.scale_dtype >= 0, DITCH_UNSUPPORTED, "checkpoint: FP8 scale dtype of " + prefix);
        w.scale_rows = (uint64_t)sc->shape[0];
        w.scale_cols = (uint64_t)sc->shape[1];
        w.block_rows = hw.fp8_block_rows ? (uint64_t)hw.fp8_block_rows : (w.rows + w.scale_rows - 1) / w.scale_rows;
        w.block_cols = hw.fp8_block_cols ? (uint64_t)hw.fp8_block_cols : (w.cols + w.scale_cols - 1) / w.scale_cols;
        return staged_checked(w, prefix, wt.bytes(), sc->bytes());
    }
    w.dtype = st_plain_dtype(wt.dtype);
    DITCH_CHECK(w.dtype >= 0, DITCH_UNSUPPORTED, "checkpoint: dtype " + wt.dtype + " of " + prefix);
    ps.reserve(wt.bytes() + 256);
    w.data = stage_copy(ps, wt.data(), wt.bytes());
    return staged_checked(w, prefix, wt.bytes());
}

// A norm or bias vector widened to f32 in pinned memory.
static ditch_weight vec_weight(const uint8_t *data, const std::string &dt, int64_t n, PinnedStage &ps) {
    ps.reset();
    ps.reserve((size_t)n * 4 + 256);
    float *out = (float *)ps.take((size_t)n * 4);
    for (int64_t i = 0; i < n; i++) {
        if (dt == "F32") memcpy(&out[i], data + 4 * i, 4);
        else if (dt == "BF16") {
            uint16_t b;
            memcpy(&b, data + 2 * i, 2);
            const uint32_t u = (uint32_t)b << 16;
            memcpy(&out[i], &u, 4);
        } else if (dt == "F16") {
            uint16_t hb;
            memcpy(&hb, data + 2 * i, 2);
            const uint32_t sign = (uint32_t)(hb & 0x8000u) << 16, e = (hb >> 10) & 0x1fu, m = hb & 0x3ffu;
            if (e == 0) {
                const float v = (float)m * 5.9604644775390625e-08f;
                out[i] = sign ? -v : v;
            } else {
                const uint32_t bits = e == 31 ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
                memcpy(&out[i], &bits, 4);
            }
        } else {
            throw Error{DITCH_UNSUPPORTED, "checkpoint: vector dtype " + dt};
        }
    }
    ditch_weight w{};
    w.data = out;
    w.dtype = DITCH_F32;
    w.rows = 1;
    w.cols = (uint64_t)n;
    return w;
}

static ditch_weight st_vec(const StTensor &t, PinnedStage &ps) { return vec_weight(t.data(), t.dtype, t.numel(), ps); }

// arch.zig:1722-1725: 0.1 * mscale * ln(scale) + 1 in f32
static float yarn_mscale(float scale, float mscale) {
    if (scale <= 1.f) return 1.f;
    return 0.1f * mscale * (float)log((double)scale) + 1.0f;
}

static uint64_t rope_len_for(double max_pos) {
    const double v = max_pos < 512 ? 512 : max_pos > 8192 ? 8192 : max_pos;
    return (uint64_t)v;
}

// ---------------------------------------------------------------------------
// Hugging Face directories

static std::vector<std::string> list_safetensors(const std::string &dir) {
    std::vector<std::string> out;
    DIR *d = opendir(dir.c_str());
    DITCH_CHECK(d, DITCH_INVALID_ARGUMENT, "checkpoint: cannot open directory " + dir);
    while (struct dirent *e = readdir(d)) {
        const std::string n = e->d_name;
        if (n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0) out.push_back(dir + "/" + n);
    }
    closedir(d);
    std::sort(out.begin(), out.end());
    return out;
}

static std::string read_text(const std::string &path) {
    Mapped f(path);
    return std::string((const char *)f.base, f.size);
}

static ditch_hip_model *load_hf(ditch_hip *h, const std::string &dir, uint64_t expert_cache) {
    const std::string cfg_text = read_text(dir + "/config.json");
    const JVal cfg = parse_json(cfg_text.data(), cfg_text.size());
    DITCH_CHECK(cfg.kind == JVal::OBJ, DITCH_INVALID_ARGUMENT, "checkpoint: config.json is not an object");
    const std::string mt = cfg.str_or("model_type", "");
    DITCH_CHECK(mt == "llama" || mt == "mistral" || mt == "qwen2" || mt == "qwen3" || mt == "qwen3_moe" ||
                    mt == "deepseek_v3",
                DITCH_UNSUPPORTED, "checkpoint: model_type '" + mt + "' (llama, qwen2, qwen3, qwen3_moe, deepseek_v3)");
    std::vector<std::unique_ptr<Mapped>> files;
    HfWeights hw;
    for (const std::string &p : list_safetensors(dir)) {
        files.emplace_back(new Mapped(p));
        read_safetensors(*files.back(), hw.t);
    }
    DITCH_CHECK(!hw.t.empty(), DITCH_INVALID_ARGUMENT, "checkpoint: no safetensors in " + dir);
    // quantization_config (dequant.zig:108-233)
    if (const JVal *qc = cfg.get("quantization_config")) {
        const std::string method = qc->str_or("quant_method", ""), format = qc->str_or("format", "");
        if (method == "fp8") {
            if (const JVal *bs = qc->get("weight_block_size"); bs && bs->kind == JVal::ARR && bs->arr.size() == 2) {
                hw.fp8_block_rows = (int)bs->arr[0].num;
                hw.fp8_block_cols = (int)bs->arr[1].num;
            }
        } else if (format == "pack-quantized" || format == "mxfp4-pack-quantized") {
            hw.mxfp4_packed = format == "mxfp4-pack-quantized";
            if (const JVal *groups = qc->get("config_groups"); groups && groups->kind == JVal::OBJ && !groups->obj.empty())
                if (const JVal *wq = groups->obj.front().second.get("weights")) {
                    hw.int_bits = (int)wq->num_or("num_bits", 4);
                    hw.int_group = (int64_t)wq->num_or("group_size", 0);
                }
        }
    }
    ditch_model_config c{};
    const int64_t hidden = (int64_t)cfg.num_or("hidden_size", 0), heads = (int64_t)cfg.num_or("num_attention_heads", 0);
    const int64_t layers = (int64_t)cfg.num_or("num_hidden_layers", 0);
    DITCH_CHECK(hidden > 0 && heads > 0 && layers > 0, DITCH_INVALID_ARGUMENT, "checkpoint: config sizes");
    c.hidden = (uint64_t)hidden;
    c.inter = (uint64_t)cfg.num_or("intermediate_size", 0);
    c.layers = (uint64_t)layers;
    c.heads = (uint64_t)heads;
    c.kv_heads = (uint64_t)cfg.num_or("num_key_value_heads", (double)heads);
    c.head_dim = (uint64_t)(cfg.has("head_dim") ? cfg.num_or("head_dim", 0) : (double)(hidden / heads));
    c.vocab = (uint64_t)cfg.num_or("vocab_size", 0);
    c.rms_eps = (float)cfg.num_or("rms_norm_eps", 1e-6);
    c.rope_theta = (float)cfg.num_or("rope_theta", 10000.0);
    c.rope_len = rope_len_for(cfg.num_or("max_position_embeddings", 2048));
    c.tie_embeddings = cfg.num_or("tie_word_embeddings", 0) != 0;
    c.rope_style = DITCH_ROPE_NEOX;
    c.rope_scaling = DITCH_ROPE_SCALING_NONE;
    c.rope_factor = 1.f;
    c.rope_low_freq_factor = 1.f;
    c.rope_high_freq_factor = 4.f;
    c.rope_original_max_position = 8192.f;
    c.yarn_beta_fast = 32.f;
    c.yarn_beta_slow = 1.f;
    c.yarn_attention_factor = 1.f;
    c.yarn_truncate = 1;
    c.routed_scaling = 1.f;
    c.n_group = 1;
    c.topk_group = 1;
    c.mla_norm_eps = 1e-6f;
    if (mt == "qwen2") c.qkv_bias = cfg.num_or("attention_bias", 1) != 0;
    if (mt == "qwen3" || mt == "qwen3_moe") c.qk_norm = 1;
    const JVal *rs = cfg.get("rope_scaling");
    std::string rt;
    if (rs && rs->kind == JVal::OBJ) rt = rs->str_or("rope_type", rs->str_or("type", ""));
    if (rt == "llama3") {
        c.rope_scaling = DITCH_ROPE_SCALING_LLAMA3;
        c.rope_factor = (float)rs->num_or("factor", 8.0);
        c.rope_low_freq_factor = (float)rs->num_or("low_freq_factor", 1.0);
        c.rope_high_freq_factor = (float)rs->num_or("high_freq_factor", 4.0);
        c.rope_original_max_position = (float)rs->num_or("original_max_position_embeddings", 8192);
    } else if (rt == "yarn") {
        const float factor = (float)rs->num_or("factor", 1.0), ms = (float)rs->num_or("mscale", 1.0),
                    msa = (float)rs->num_or("mscale_all_dim", 0.0);
        float af;
        if (rs->has("attention_factor")) af = (float)rs->num_or("attention_factor", 1.0);
        else if (ms != 0.f && msa != 0.f) af = yarn_mscale(factor, ms) / yarn_mscale(factor, msa);
        else af = yarn_mscale(factor, 1.f);
        c.rope_scaling = DITCH_ROPE_SCALING_YARN;
        c.rope_factor = factor;
        c.rope_original_max_position =
            (float)rs->num_or("original_max_position_embeddings", cfg.num_or("original_max_position_embeddings", 4096));
        c.yarn_beta_fast = (float)rs->num_or("beta_fast", 32);
        c.yarn_beta_slow = (float)rs->num_or("beta_slow", 1);
        c.yarn_attention_factor = af;
        c.yarn_truncate = rs->num_or("truncate", 1) != 0;
    }
    const int64_t n_exp = (int64_t)(cfg.has("num_experts") ? cfg.num_or("num_experts", 0) : cfg.num_or("n_routed_experts", 0));
    std::vector<uint8_t> moe(layers, 0);
    if (n_exp > 0) {
        int64_t step = (int64_t)(cfg.has("decoder_sparse_step") ? cfg.num_or("decoder_sparse_step", 1)
                                                                 : cfg.num_or("moe_layer_freq", 1));
        step = step < 1 ? 1 : step;
        const int64_t first = (int64_t)cfg.num_or("first_k_dense_replace", 0);
        const bool by_freq = cfg.has("moe_layer_freq");
        for (int64_t i = 0; i < layers; i++)
            moe[i] = i >= first && (by_freq ? i % step == 0 : (i + 1) % step == 0);
        if (const JVal *mlo = cfg.get("mlp_only_layers"); mlo && mlo->kind == JVal::ARR)
            for (const JVal &v : mlo->arr)
                if ((int64_t)v.num >= 0 && (int64_t)v.num < layers) moe[(size_t)v.num] = 0;
        c.n_experts = (uint64_t)n_exp;
        c.top_k = (uint64_t)cfg.num_or("num_experts_per_tok", 2);
        c.moe_inter = (uint64_t)cfg.num_or("moe_intermediate_size", 0);
        c.norm_topk_prob = cfg.num_or("norm_topk_prob", 0) != 0;
    }
    if (mt == "deepseek_v3") {
        const int64_t nope = (int64_t)cfg.num_or("qk_nope_head_dim", 0), rd = (int64_t)cfg.num_or("qk_rope_head_dim", 0);
        float scale = 1.0f / sqrtf((float)(nope + rd));
        if (rt == "yarn" && rs->num_or("mscale_all_dim", 0) != 0) {
            const float ms = yarn_mscale((float)rs->num_or("factor", 1.0), (float)rs->num_or("mscale_all_dim", 0));
            scale = scale * ms * ms;
        }
        c.mla = 1;
        c.head_dim = (uint64_t)(nope + rd);
        c.v_head_dim = (uint64_t)cfg.num_or("v_head_dim", 0);
        c.kv_heads = (uint64_t)heads;
        c.q_lora_rank = (uint64_t)cfg.num_or("q_lora_rank", 0);
        c.kv_lora_rank = (uint64_t)cfg.num_or("kv_lora_rank", 0);
        c.qk_nope_dim = (uint64_t)nope;
        c.qk_rope_dim = (uint64_t)rd;
        c.rotary_dim = (uint64_t)rd;
        c.attn_scale = scale;
        c.rope_style = cfg.num_or("rope_interleave", 1) != 0 ? DITCH_ROPE_GPTJ : DITCH_ROPE_NEOX;
        c.scoring = cfg.str_or("scoring_func", "softmax") == "sigmoid" ? DITCH_SCORING_SIGMOID : DITCH_SCORING_SOFTMAX;
        const std::string tm = cfg.str_or("topk_method", "");
        c.group_limited = tm == "noaux_tc" || tm == "group_limited_greedy";
        c.n_group = (uint64_t)std::max(1.0, cfg.num_or("n_group", 1));
        c.topk_group = (uint64_t)std::max(1.0, cfg.num_or("topk_group", 1));
        c.routed_scaling = (float)cfg.num_or("routed_scaling_factor", 1.0);
        c.shared_inter = (uint64_t)(cfg.num_or("moe_intermediate_size", 0) * cfg.num_or("n_shared_experts", 0));
    }
    if (!c.v_head_dim) c.v_head_dim = c.head_dim;
    if (!c.rotary_dim) c.rotary_dim = c.mla ? c.qk_rope_dim : c.head_dim;
    if (c.attn_scale == 0.f) c.attn_scale = 1.0f / sqrtf((float)c.head_dim);
    c.moe_layers = moe.data();

    ditch_hip_model *m = model_create(h, &c);
    std::unique_ptr<ditch_hip_model> guard(m);
    if (expert_cache) m->expert_budget = expert_cache;
    PinnedStage ps;
    auto set_mat = [&](int layer, int slot, int expert, const std::string &prefix) {
        const ditch_weight w = hf_weight(hw, prefix, ps);
        model_set(m, layer, slot, expert, &w);
    };
    auto set_plain = [&](int layer, int slot, const std::string &name) {
        const StTensor &t = hw.at(name);
        ps.reset();
        ps.reserve(t.bytes() + 256);
        ditch_weight w{};
        w.dtype = st_plain_dtype(t.dtype);
        DITCH_CHECK(w.dtype >= 0 && t.shape.size() == 2, DITCH_UNSUPPORTED, "checkpoint: " + name);
        w.rows = (uint64_t)t.shape[0];
        w.cols = (uint64_t)t.shape[1];
        w.data = stage_copy(ps, t.data(), t.bytes());
        model_set(m, layer, slot, -1, &w);
    };
    auto set_vec = [&](int layer, int slot, const std::string &name) {
        const ditch_weight w = st_vec(hw.at(name), ps);
        model_set(m, layer, slot, -1, &w);
    };
    // Routed experts stored as two stacked tensors (Layout.fused /
    // .fused_transposed, moe.zig:83-93, detection and slicing at
    // moe.zig:688-770): `experts.gate_up_proj` [E, 2I, hidden] with
    // `experts.down_proj` [E, hidden, I], each expert a contiguous row-major
    // block whose rows 0..I are the gate and I..2I the up projection; or
    // [E, hidden, 2I] with [E, I, hidden], each block transposed on load
    // (columns 0..I the gate, I..2I the up). Plain dtypes (the stacked
    // tensors are sliced element-wise).
    auto set_fused_experts = [&](int layer, const std::string &mp, const StTensor &gu) {
        const StTensor *dn = hw.find(mp + "experts.down_proj");
        if (!dn) dn = hw.find(mp + "experts.down_proj.weight");
        DITCH_CHECK(dn != nullptr, DITCH_INVALID_ARGUMENT, "checkpoint: " + mp + "experts.down_proj missing");
        const int64_t E = n_exp, I = (int64_t)c.moe_inter, H = (int64_t)hidden;
        const int32_t dt = st_plain_dtype(gu.dtype);
        DITCH_CHECK(dt >= 0 && st_plain_dtype(dn->dtype) == dt, DITCH_UNSUPPORTED,
                    "checkpoint: stacked experts of " + mp + " in dtype " + gu.dtype + " (F32, F16, BF16)");
        DITCH_CHECK(gu.shape.size() == 3 && dn->shape.size() == 3 && gu.shape[0] == E && dn->shape[0] == E,
                    DITCH_INVALID_ARGUMENT, "checkpoint: stacked experts of " + mp + ": expert count");
        bool transposed;
        if (gu.shape[1] == 2 * I && gu.shape[2] == H) {
            transposed = false;
            DITCH_CHECK(dn->shape[1] == H && dn->shape[2] == I, DITCH_INVALID_ARGUMENT,
                        "checkpoint: " + mp + "experts.down_proj shape");
        } else if (gu.shape[1] == H && gu.shape[2] == 2 * I) {
            transposed = true;
            DITCH_CHECK(dn->shape[1] == I && dn->shape[2] == H, DITCH_INVALID_ARGUMENT,
                        "checkpoint: " + mp + "experts.down_proj shape");
        } else {
            throw Error{DITCH_INVALID_ARGUMENT, "checkpoint: unexpected stacked expert shape in " + mp};
        }
        const size_t es = st_elem_bytes(gu.dtype);
        // rows x cols of the matrix [rows][cols] whose element (r, c) lies at
        // src + (r * rs + c * cs) * es
        auto put = [&](int slot, int e, const uint8_t *src, int64_t rows, int64_t cols, int64_t rs, int64_t cs) {
            ps.reset();
            ps.reserve((size_t)(rows * cols) * es + 256);
            uint8_t *d = ps.take((size_t)(rows * cols) * es);
            if (cs == 1)
                for (int64_t r = 0; r < rows; r++) memcpy(d + (size_t)(r * cols) * es, src + (size_t)(r * rs) * es, cols * es);
            else
                for (int64_t r = 0; r < rows; r++)
                    for (int64_t k = 0; k < cols; k++)
                        memcpy(d + (size_t)(r * cols + k) * es, src + (size_t)(r * rs + k * cs) * es, es);
            ditch_weight w{};
            w.dtype = dt;
            w.rows = (uint64_t)rows;
            w.cols = (uint64_t)cols;
            w.data = d;
            model_set(m, layer, slot, e, &w);
        };
        for (int64_t e = 0; e < E; e++) {
            const uint8_t *g = gu.data() + (size_t)(e * 2 * I * H) * es, *dw = dn->data() + (size_t)(e * H * I) * es;
            if (!transposed) {
                put(DITCH_SLOT_EXPERT_GATE, (int)e, g, I, H, H, 1);
                put(DITCH_SLOT_EXPERT_UP, (int)e, g + (size_t)(I * H) * es, I, H, H, 1);
                put(DITCH_SLOT_EXPERT_DOWN, (int)e, dw, H, I, I, 1);
            } else {
                // block [H][2I]: gate (r, k) = block[k][r], up (r, k) = block[k][I + r]
                put(DITCH_SLOT_EXPERT_GATE, (int)e, g, I, H, 1, 2 * I);
                put(DITCH_SLOT_EXPERT_UP, (int)e, g + (size_t)I * es, I, H, 1, 2 * I);
                // block [I][H]: down (r, k) = block[k][r]
                put(DITCH_SLOT_EXPERT_DOWN, (int)e, dw, H, I, 1, H);
            }
        }
    };
    set_plain(-1, DITCH_SLOT_EMBED, "model.embed_tokens.weight");
    set_vec(-1, DITCH_SLOT_FINAL_NORM, "model.norm.weight");
    if (hw.find("lm_head.weight")) set_plain(-1, DITCH_SLOT_LM_HEAD, "lm_head.weight");
    for (int li = 0; li < (int)layers; li++) {
        const std::string p = "model.layers." + std::to_string(li) + ".";
        set_vec(li, DITCH_SLOT_ATTN_NORM, p + "input_layernorm.weight");
        set_vec(li, DITCH_SLOT_FFN_NORM, p + "post_attention_layernorm.weight");
        const std::string a = p + "self_attn.";
        if (c.mla) {
            if (hw.find(a + "q_a_proj.weight") || hw.find(a + "q_a_proj.weight_packed")) {
                set_mat(li, DITCH_SLOT_MLA_Q_A, -1, a + "q_a_proj");
                set_vec(li, DITCH_SLOT_MLA_Q_A_NORM, a + "q_a_layernorm.weight");
                set_mat(li, DITCH_SLOT_MLA_Q_B, -1, a + "q_b_proj");
            } else {
                set_mat(li, DITCH_SLOT_MLA_Q_B, -1, a + "q_proj");
            }
            set_mat(li, DITCH_SLOT_MLA_KV_A, -1, a + "kv_a_proj_with_mqa");
            set_vec(li, DITCH_SLOT_MLA_KV_A_NORM, a + "kv_a_layernorm.weight");
            set_mat(li, DITCH_SLOT_MLA_KV_B, -1, a + "kv_b_proj");
        } else {
            const struct {
                int slot, bias;
                const char *name;
            } qkv[3] = {{DITCH_SLOT_Q, DITCH_SLOT_Q_BIAS, "q_proj"},
                        {DITCH_SLOT_K, DITCH_SLOT_K_BIAS, "k_proj"},
                        {DITCH_SLOT_V, DITCH_SLOT_V_BIAS, "v_proj"}};
            for (const auto &q : qkv) {
                set_mat(li, q.slot, -1, a + q.name);
                if (hw.find(a + q.name + ".bias")) set_vec(li, q.bias, a + q.name + ".bias");
            }
            if (hw.find(a + "q_norm.weight")) {
                set_vec(li, DITCH_SLOT_Q_NORM, a + "q_norm.weight");
                set_vec(li, DITCH_SLOT_K_NORM, a + "k_norm.weight");
            }
        }
        set_mat(li, DITCH_SLOT_O, -1, a + "o_proj");
        const std::string mp = p + "mlp.";
        if (n_exp > 0 && moe[li]) {
            set_plain(li, DITCH_SLOT_ROUTER, mp + "gate.weight");
            if (hw.find(mp + "gate.e_score_correction_bias"))
                set_vec(li, DITCH_SLOT_ROUTER_CORRECTION, mp + "gate.e_score_correction_bias");
            const StTensor *fgu = hw.find(mp + "experts.gate_up_proj");
            if (!fgu) fgu = hw.find(mp + "experts.gate_up_proj.weight");
            if (fgu) set_fused_experts(li, mp, *fgu);
            else
                for (int e = 0; e < (int)n_exp; e++) {
                    const std::string ep = mp + "experts." + std::to_string(e) + ".";
                    set_mat(li, DITCH_SLOT_EXPERT_GATE, e, ep + "gate_proj");
                    set_mat(li, DITCH_SLOT_EXPERT_UP, e, ep + "up_proj");
                    set_mat(li, DITCH_SLOT_EXPERT_DOWN, e, ep + "down_proj");
                }
            if (hw.find(mp + "shared_experts.gate_proj.weight") || hw.find(mp + "shared_experts.gate_proj.weight_packed")) {
                set_mat(li, DITCH_SLOT_SHARED_GATE, -1, mp + "shared_experts.gate_proj");
                set_mat(li, DITCH_SLOT_SHARED_UP, -1, mp + "shared_experts.up_proj");
                set_mat(li, DITCH_SLOT_SHARED_DOWN, -1, mp + "shared_experts.down_proj");
            }
        } else {
            set_mat(li, DITCH_SLOT_GATE, -1, mp + "gate_proj");
            set_mat(li, DITCH_SLOT_UP, -1, mp + "up_proj");
            set_mat(li, DITCH_SLOT_DOWN, -1, mp + "down_proj");
        }
    }
    return guard.release();
}

// ---------------------------------------------------------------------------
// GGUF files (gguf_model.zig)

static ditch_hip_model *load_gguf(ditch_hip *h, const std::string &path, uint64_t expert_cache) {
    Mapped f(path);
    std::map<std::string, GgufMeta> meta;
    std::map<std::string, GgufTensor> t;
    read_gguf(f, meta, t);
    auto ms = [&](const std::string &k) -> const GgufMeta * {
        auto it = meta.find(k);
        return it == meta.end() ? nullptr : &it->second;
    };
    const GgufMeta *archm = ms("general.architecture");
    DITCH_CHECK(archm && archm->kind == GgufMeta::S, DITCH_INVALID_ARGUMENT, "gguf: no general.architecture");
    const std::string arch = archm->s;
    DITCH_CHECK(arch == "llama" || arch == "qwen2", DITCH_UNSUPPORTED, "gguf: architecture '" + arch + "' (llama, qwen2)");
    auto num = [&](const std::string &k, double dflt) {
        const GgufMeta *v = ms(arch + "." + k);
        return v ? v->as_num() : dflt;
    };
    auto tensor = [&](const std::string &n) -> const GgufTensor & {
        auto it = t.find(n);
        DITCH_CHECK(it != t.end(), DITCH_INVALID_ARGUMENT, "gguf: tensor " + n + " missing");
        return it->second;
    };
    ditch_model_config c{};
    c.hidden = (uint64_t)num("embedding_length", 0);
    c.heads = (uint64_t)num("attention.head_count", 0);
    c.kv_heads = (uint64_t)num("attention.head_count_kv", (double)c.heads);
    c.layers = (uint64_t)num("block_count", 0);
    DITCH_CHECK(c.hidden && c.heads && c.layers, DITCH_INVALID_ARGUMENT, "gguf: model sizes");
    c.inter = (uint64_t)num("feed_forward_length", 0);
    c.vocab = (uint64_t)tensor("token_embd.weight").rows;
    c.head_dim = (uint64_t)num("attention.key_length", (double)(c.hidden / c.heads));
    c.v_head_dim = c.head_dim;
    c.rotary_dim = c.head_dim;
    c.rms_eps = (float)num("attention.layer_norm_rms_epsilon", 1e-6);
    c.rope_theta = (float)num("rope.freq_base", 10000.0);
    c.rope_len = rope_len_for(num("context_length", 2048));
    c.rope_style = DITCH_ROPE_NEOX;
    c.rope_factor = 1.f;
    c.rope_low_freq_factor = 1.f;
    c.rope_high_freq_factor = 4.f;
    c.rope_original_max_position = 8192.f;
    c.yarn_beta_fast = 32.f;
    c.yarn_beta_slow = 1.f;
    c.yarn_attention_factor = 1.f;
    c.yarn_truncate = 1;
    c.routed_scaling = 1.f;
    c.n_group = 1;
    c.topk_group = 1;
    c.attn_scale = 1.0f / sqrtf((float)c.head_dim);
    c.qkv_bias = arch == "qwen2";
    c.tie_embeddings = t.find("output.weight") == t.end();
    std::vector<float> factors;
    if (auto it = t.find("rope_freqs.weight"); it != t.end()) {
        // per-frequency divisors (gguf_model.zig:171-180, 320-336)
        DITCH_CHECK(it->second.type == "F32", DITCH_UNSUPPORTED, "gguf: rope_freqs dtype");
        factors.resize((size_t)(it->second.rows * it->second.cols));
        memcpy(factors.data(), it->second.data, factors.size() * 4);
        c.rope_scaling = DITCH_ROPE_SCALING_FACTORS;
        c.rope_factors = factors.data();
    }
    ditch_hip_model *m = model_create(h, &c);
    std::unique_ptr<ditch_hip_model> guard(m);
    if (expert_cache) m->expert_budget = expert_cache;
    PinnedStage ps;
    const bool permute = arch == "llama";
    // llama.cpp writes q/k head rows as (pair, half); the forward reads (half, pair)
    auto set_mat = [&](int layer, int slot, const std::string &name, int64_t n_head) {
        const GgufTensor &g = tensor(name);
        std::string tname;
        int64_t bs = 1, bb = 4;
        static const std::map<std::string, uint32_t> ids = {{"F32", 0}, {"F16", 1}, {"Q4_0", 2}, {"Q4_1", 3},
                                                            {"Q5_0", 6}, {"Q5_1", 7}, {"Q8_0", 8}, {"Q4_K", 12},
                                                            {"Q6_K", 14}, {"Q8_K", 15}, {"BF16", 30}};
        gguf_block(ids.at(g.type), tname, bs, bb);
        const size_t row_bytes = (size_t)(g.cols / bs * bb);
        ps.reset();
        ps.reserve(g.bytes + 256);
        uint8_t *d = ps.take(g.bytes);
        if (n_head > 0) {
            const int64_t hd = g.rows / n_head;
            DITCH_CHECK(hd % 2 == 0 && hd * n_head == g.rows, DITCH_INVALID_ARGUMENT, "gguf: q/k rows per head");
            for (int64_t hh = 0; hh < n_head; hh++)
                for (int64_t half = 0; half < 2; half++)
                    for (int64_t pr = 0; pr < hd / 2; pr++)
                        memcpy(d + (size_t)(hh * hd + half * (hd / 2) + pr) * row_bytes,
                               g.data + (size_t)(hh * hd + pr * 2 + half) * row_bytes, row_bytes);
        } else {
            memcpy(d, g.data, g.bytes);
        }
        ditch_weight w{};
        w.data = d;
        w.rows = (uint64_t)g.rows;
        w.cols = (uint64_t)g.cols;
        static const std::map<std::string, int32_t> dt = {{"F32", DITCH_F32}, {"F16", DITCH_F16}, {"BF16", DITCH_BF16},
                                                          {"Q8_0", DITCH_Q8_0}, {"Q4_0", DITCH_Q4_0}, {"Q4_1", DITCH_Q4_1},
                                                          {"Q5_0", DITCH_Q5_0}, {"Q5_1", DITCH_Q5_1}, {"Q4_K", DITCH_Q4_K},
                                                          {"Q6_K", DITCH_Q6_K}, {"Q8_K", DITCH_Q8_K}};
        w.dtype = dt.at(g.type);
        model_set(m, layer, slot, -1, &w);
    };
    auto set_vec = [&](int layer, int slot, const std::string &name, int64_t n_head) {
        const GgufTensor &g = tensor(name);
        const int64_t n = g.rows * g.cols;
        const size_t eb = g.type == "F32" ? 4 : 2;
        DITCH_CHECK(g.type == "F32" || g.type == "F16" || g.type == "BF16", DITCH_UNSUPPORTED, "gguf: vector dtype");
        std::vector<uint8_t> tmp(g.data, g.data + (size_t)n * eb);
        if (n_head > 0) {  // a q/k bias: the same head permutation as its rows
            const int64_t hd = n / n_head;
            for (int64_t hh = 0; hh < n_head; hh++)
                for (int64_t half = 0; half < 2; half++)
                    for (int64_t pr = 0; pr < hd / 2; pr++)
                        memcpy(tmp.data() + (size_t)(hh * hd + half * (hd / 2) + pr) * eb,
                               g.data + (size_t)(hh * hd + pr * 2 + half) * eb, eb);
        }
        const ditch_weight w = vec_weight(tmp.data(), g.type, n, ps);
        model_set(m, layer, slot, -1, &w);
    };
    set_mat(-1, DITCH_SLOT_EMBED, "token_embd.weight", 0);
    set_vec(-1, DITCH_SLOT_FINAL_NORM, "output_norm.weight", 0);
    if (!c.tie_embeddings) set_mat(-1, DITCH_SLOT_LM_HEAD, "output.weight", 0);
    for (int li = 0; li < (int)c.layers; li++) {
        const std::string b = "blk." + std::to_string(li) + ".";
        set_vec(li, DITCH_SLOT_ATTN_NORM, b + "attn_norm.weight", 0);
        set_vec(li, DITCH_SLOT_FFN_NORM, b + "ffn_norm.weight", 0);
        const struct {
            int slot, bias;
            const char *name;
            int64_t heads;
        } qkv[3] = {{DITCH_SLOT_Q, DITCH_SLOT_Q_BIAS, "attn_q", permute ? (int64_t)c.heads : 0},
                    {DITCH_SLOT_K, DITCH_SLOT_K_BIAS, "attn_k", permute ? (int64_t)c.kv_heads : 0},
                    {DITCH_SLOT_V, DITCH_SLOT_V_BIAS, "attn_v", 0}};
        for (const auto &q : qkv) {
            set_mat(li, q.slot, b + q.name + ".weight", q.heads);
            if (t.count(b + q.name + ".bias")) set_vec(li, q.bias, b + q.name + ".bias", q.heads);
        }
        set_mat(li, DITCH_SLOT_O, b + "attn_output.weight", 0);
        set_mat(li, DITCH_SLOT_GATE, b + "ffn_gate.weight", 0);
        set_mat(li, DITCH_SLOT_UP, b + "ffn_up.weight", 0);
        set_mat(li, DITCH_SLOT_DOWN, b + "ffn_down.weight", 0);
    }
    return guard.release();
}

ditch_hip_model *model_load(ditch_hip *h, const char *path, uint64_t expert_cache) {
    DITCH_CHECK(path && *path, DITCH_INVALID_ARGUMENT, "checkpoint: empty path");
    struct stat st;
    DITCH_CHECK(stat(path, &st) == 0, DITCH_INVALID_ARGUMENT, std::string("checkpoint: cannot stat ") + path);
    const std::string p = path;
    if (S_ISDIR(st.st_mode)) return load_hf(h, p, expert_cache);
    return load_gguf(h, p, expert_cache);
}

}  // namespace ditch
