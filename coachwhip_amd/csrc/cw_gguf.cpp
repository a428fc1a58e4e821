// GGUF reader: header, metadata and tensor directory of a GGUF file (versions 1-3), with the
// tensor data mapped read-only, and the per-expert slicing of a layer's
// blk.{l}.ffn_{gate,up,down}_exps.weight tensors.
//
// Follows candle's gguf_file.rs Content::read (vendor/candle-core/src/quantized/gguf_file.rs:
// 469-567): little-endian fields; 32-bit lengths and dims in version 1, 64-bit after; dims stored
// innermost first and reported outermost first; tensor data at the first multiple of
// general.alignment (any non-negative integer of up to 32 bits, default 32) after the
// directory; the same caps on string and array lengths, array nesting and dims, and the same
// checks that declared counts and lengths fit in the file. Expert slicing follows
// ExpertStore::new (crates/engine/src/experts.rs:697-718): a [E][n][k] tensor holds E matrices
// of n rows, expert e at e times one matrix's bytes. Unlike the reference, IQ3_S (21) and IQ2_S
// (22) are accepted.
#include <fcntl.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/cwmoe.h"

namespace cw {
int set_error(int code, const char *fmt, ...);
}

namespace {

constexpr uint64_t MAX_STRING = 1ull << 30, MAX_ARRAY = 1ull << 30;
constexpr uint32_t MAX_DIMS = 4;
constexpr int MAX_DEPTH = 64;
constexpr uint64_t DEFAULT_ALIGNMENT = 32;

// (block size in weights, bytes per block) of the ggml types, by id; {0, 0} = unknown
struct TypeSize {
    int block, bytes;
};
TypeSize type_size(uint32_t t) {
    switch (t) {
    case 0: return {1, 4};       // F32
    case 1: return {1, 2};       // F16
    case 2: return {32, 18};     // Q4_0
    case 3: return {32, 20};     // Q4_1
    case 6: return {32, 22};     // Q5_0
    case 7: return {32, 24};     // Q5_1
    case 8: return {32, 34};     // Q8_0
    case 9: return {32, 36};     // Q8_1
    case 10: return {256, 84};   // Q2_K
    case 11: return {256, 110};  // Q3_K
    case 12: return {256, 144};  // Q4_K
    case 13: return {256, 176};  // Q5_K
    case 14: return {256, 210};  // Q6_K
    case 15: return {256, 292};  // Q8_K
    case 16: return {256, 66};   // IQ2_XXS
    case 17: return {256, 74};   // IQ2_XS
    case 18: return {256, 98};   // IQ3_XXS
    case 19: return {256, 50};   // IQ1_S
    case 20: return {32, 18};    // IQ4_NL
    case 21: return {256, 110};  // IQ3_S
    case 22: return {256, 82};   // IQ2_S
    case 23: return {256, 136};  // IQ4_XS
    case 24: return {1, 1};      // I8
    case 25: return {1, 2};      // I16
    case 26: return {1, 4};      // I32
    case 27: return {1, 8};      // I64
    case 28: return {1, 8};      // F64
    case 29: return {256, 56};   // IQ1_M
    case 30: return {1, 2};      // BF16
    case 39: return {32, 17};    // MXFP4
    default: return {0, 0};
    }
}

enum VType { U8 = 0, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 };

struct Value {
    int type = -1;
    int64_t i = 0;   // integer types and bool
    double f = 0;    // F32 / F64
    std::string s;   // STRING
    bool integral() const { return type == U8 || type == I8 || type == U16 || type == I16 || type == U32 || type == I32 || type == U64 || type == I64 || type == BOOL; }
};

struct Tensor {
    std::string name;
    uint32_t dtype;
    std::vector<int64_t> dims;  // outermost first
    uint64_t offset;            // from the start of the tensor data
    uint64_t bytes;
};

struct Reader {
    const uint8_t *p, *end;
    int version;
    bool fail = false;
    std::string err;
    bool need(uint64_t n) {
        if (fail) return false;
        if ((uint64_t)(end - p) < n) {
            fail = true;
            err = "truncated file";
            return false;
        }
        return true;
    }
    template <class T>
    T get() {
        T v{};
        if (!need(sizeof(T))) return v;
        memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    uint64_t length() { return version == 1 ? get<uint32_t>() : get<uint64_t>(); }
    uint64_t prefix() const { return version == 1 ? 4 : 8; }
    uint64_t left() const { return (uint64_t)(end - p); }
    bool bad(const std::string &m) {
        if (!fail) {
            fail = true;
            err = m;
        }
        return false;
    }
    bool string(std::string &out) {
        const uint64_t n = length();
        if (fail) return false;
        if (n > MAX_STRING) return bad("string length exceeds the maximum");
        if (n > left()) return bad("string length exceeds the remaining file bytes");
        out.assign((const char *)p, (size_t)n);
        p += n;
        while (!out.empty() && out.back() == 0) out.pop_back();  // some writers add a terminator
        return true;
    }
    uint64_t min_size(int t) const {
        switch (t) {
        case U8: case I8: case BOOL: return 1;
        case U16: case I16: return 2;
        case U32: case I32: case F32: return 4;
        case U64: case I64: case F64: return 8;
        case STRING: return prefix();
        default: return 4 + prefix();  // ARRAY
        }
    }
    bool value(int t, int depth, Value &v) {
        if (depth > MAX_DEPTH) return bad("value nesting exceeds the maximum depth");
        v.type = t;
        switch (t) {
        case U8: v.i = get<uint8_t>(); break;
        case I8: v.i = get<int8_t>(); break;
        case U16: v.i = get<uint16_t>(); break;
        case I16: v.i = get<int16_t>(); break;
        case U32: v.i = get<uint32_t>(); break;
        case I32: v.i = get<int32_t>(); break;
        case U64: v.i = (int64_t)get<uint64_t>(); break;
        case I64: v.i = get<int64_t>(); break;
        case F32: v.f = get<float>(); break;
        case F64: v.f = get<double>(); break;
        case BOOL: {
            const uint8_t b = get<uint8_t>();
            if (b > 1) return bad("bool value other than 0 or 1");
            v.i = b;
            break;
        }
        case STRING: return string(v.s);
        case ARRAY: {
            const uint32_t et = get<uint32_t>();
            if (et > F64) return bad("unknown array element type");
            const uint64_t n = length();
            if (fail) return false;
            if (n > MAX_ARRAY) return bad("array length exceeds the maximum");
            if (n > left() / min_size((int)et)) return bad("array longer than the remaining file bytes");
            Value e;
            for (uint64_t k = 0; k < n; k++)
                if (!value((int)et, depth + 1, e)) return false;
            v.i = (int64_t)n;  // arrays keep only their length
            break;
        }
        default: return bad("unknown value type");
        }
        return !fail;
    }
};

}  // namespace

struct cw_gguf {
    void *map = nullptr;
    size_t size = 0;
    int version = 0;
    uint64_t data_offset = 0;
    std::unordered_map<std::string, Value> meta;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int64_t> index;
};

static cw_gguf *fail_open(cw_gguf *g, int code, const char *path, const std::string &why) {
    cw::set_error(code, "gguf %s: %s", path, why.c_str());
    if (g) {
        if (g->map) munmap(g->map, g->size);
        delete g;
    }
    return nullptr;
}

extern "C" {

cw_gguf *cw_gguf_open(const char *path) {
    if (!path) return fail_open(nullptr, CW_EINVAL, "(null)", "no path");
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail_open(nullptr, CW_EINVAL, path, "cannot open");
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 8) {
        close(fd);
        return fail_open(nullptr, CW_EINVAL, path, "not a GGUF file (too small)");
    }
    cw_gguf *g = new cw_gguf;
    g->size = (size_t)st.st_size;
    g->map = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (g->map == MAP_FAILED) {
        g->map = nullptr;
        return fail_open(g, CW_EINVAL, path, "cannot map");
    }
    Reader r{(const uint8_t *)g->map, (const uint8_t *)g->map + g->size, 0};
    const uint32_t magic = r.get<uint32_t>();
    if (magic != 0x46554747u && magic != 0x47475546u) return fail_open(g, CW_EINVAL, path, "unknown magic");
    const uint32_t version = r.get<uint32_t>();
    if (version < 1 || version > 3) return fail_open(g, CW_ENOTSUP, path, "unsupported version " + std::to_string(version));
    r.version = g->version = (int)version;
    const uint64_t n_tensors = r.length(), n_kv = r.length();
    if (r.fail) return fail_open(g, CW_EINVAL, path, r.err);
    if (n_tensors > MAX_ARRAY || n_kv > MAX_ARRAY) return fail_open(g, CW_EINVAL, path, "tensor or metadata count exceeds the maximum");
    // declared counts must fit at their minimum sizes
    const double need = (double)n_kv * (double)(r.prefix() + 5) + (double)n_tensors * (double)(r.prefix() + 16);
    if (need > (double)r.left()) return fail_open(g, CW_EINVAL, path, "declared counts do not fit in the file");
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key;
        Value v;
        if (!r.string(key)) break;
        const uint32_t t = r.get<uint32_t>();
        if (t > F64) {
            r.bad("unknown value type");
            break;
        }
        if (!r.value((int)t, 0, v)) break;
        g->meta[key] = v;
    }
    if (r.fail) return fail_open(g, CW_EINVAL, path, r.err);
    for (uint64_t i = 0; i < n_tensors; i++) {
        Tensor t;
        if (!r.string(t.name)) break;
        const uint32_t nd = r.get<uint32_t>();
        if (nd > MAX_DIMS) {
            r.bad("tensor '" + t.name + "' has more than 4 dimensions");
            break;
        }
        t.dims.resize(nd);
        for (uint32_t d = 0; d < nd; d++) t.dims[nd - 1 - d] = (int64_t)(version == 1 ? r.get<uint32_t>() : r.get<uint64_t>());
        t.dtype = r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        if (r.fail) break;
        const TypeSize ts = type_size(t.dtype);
        if (!ts.block) return fail_open(g, CW_ENOTSUP, path, "tensor '" + t.name + "' has unknown type " + std::to_string(t.dtype));
        int64_t elems = 1;
        for (int64_t d : t.dims) {
            if (d < 0 || (d && elems > INT64_MAX / d)) return fail_open(g, CW_EINVAL, path, "tensor '" + t.name + "' has bad dims");
            elems *= d;
        }
        if (elems % ts.block) return fail_open(g, CW_EINVAL, path, "tensor '" + t.name + "' is not whole blocks");
        // a tensor bigger than the file is refused before its size is formed, so the product
        // cannot wrap (8-byte types with more than 2^61 elements would)
        if ((uint64_t)(elems / ts.block) > (uint64_t)g->size / (uint64_t)ts.bytes)
            return fail_open(g, CW_EINVAL, path, "tensor '" + t.name + "' is larger than the file");
        t.bytes = (uint64_t)(elems / ts.block) * (uint64_t)ts.bytes;
        g->index[t.name] = (int64_t)g->tensors.size();
        g->tensors.push_back(std::move(t));
    }
    if (r.fail) return fail_open(g, CW_EINVAL, path, r.err);
    uint64_t align = DEFAULT_ALIGNMENT;
    auto it = g->meta.find("general.alignment");
    if (it != g->meta.end()) {
        const Value &v = it->second;
        const bool ok = v.type == U8 || v.type == U16 || v.type == U32 || ((v.type == I8 || v.type == I16 || v.type == I32) && v.i >= 0);
        if (ok) align = (uint64_t)v.i;
    }
    if (align == 0) return fail_open(g, CW_EINVAL, path, "alignment 0");
    const uint64_t pos = (uint64_t)(r.p - (const uint8_t *)g->map);
    g->data_offset = (pos + align - 1) / align * align;
    for (const Tensor &t : g->tensors)
        if (g->data_offset + t.offset > g->size || t.bytes > g->size - g->data_offset - t.offset)
            return fail_open(g, CW_EINVAL, path, "tensor '" + t.name + "' extends past the end of the file");
    return g;
}

void cw_gguf_close(cw_gguf *g) {
    if (!g) return;
    if (g->map) munmap(g->map, g->size);
    delete g;
}

int cw_gguf_version(const cw_gguf *g) { return g ? g->version : 0; }

int64_t cw_gguf_n_tensors(const cw_gguf *g) { return g ? (int64_t)g->tensors.size() : 0; }

int64_t cw_gguf_find(const cw_gguf *g, const char *name) {
    if (!g || !name) return -1;
    auto it = g->index.find(name);
    return it == g->index.end() ? -1 : it->second;
}

int cw_gguf_tensor(const cw_gguf *g, int64_t i, const char **name, int *dtype, int *n_dims, int64_t dims[4],
                   int64_t *file_offset, int64_t *bytes) {
    if (!g || i < 0 || i >= (int64_t)g->tensors.size()) return cw::set_error(CW_EINVAL, "gguf: no tensor %lld", (long long)i);
    const Tensor &t = g->tensors[(size_t)i];
    if (name) *name = t.name.c_str();
    if (dtype) *dtype = (int)t.dtype;
    if (n_dims) *n_dims = (int)t.dims.size();
    if (dims)
        for (int d = 0; d < 4; d++) dims[d] = d < (int)t.dims.size() ? t.dims[(size_t)d] : 0;
    if (file_offset) *file_offset = (int64_t)(g->data_offset + t.offset);
    if (bytes) *bytes = (int64_t)t.bytes;
    return CW_OK;
}

const void *cw_gguf_data(const cw_gguf *g, int64_t i) {
    if (!g || i < 0 || i >= (int64_t)g->tensors.size()) return nullptr;
    return (const uint8_t *)g->map + g->data_offset + g->tensors[(size_t)i].offset;
}

int cw_gguf_meta_int(const cw_gguf *g, const char *key, int64_t *v) {
    if (!g || !key) return cw::set_error(CW_EINVAL, "gguf: null argument");
    auto it = g->meta.find(key);
    if (it == g->meta.end() || !it->second.integral()) return cw::set_error(CW_EINVAL, "gguf: no integer metadata '%s'", key);
    if (v) *v = it->second.i;
    return CW_OK;
}

int cw_gguf_meta_float(const cw_gguf *g, const char *key, double *v) {
    if (!g || !key) return cw::set_error(CW_EINVAL, "gguf: null argument");
    auto it = g->meta.find(key);
    if (it == g->meta.end() || (it->second.type != F32 && it->second.type != F64))
        return cw::set_error(CW_EINVAL, "gguf: no float metadata '%s'", key);
    if (v) *v = it->second.f;
    return CW_OK;
}

const char *cw_gguf_meta_str(const cw_gguf *g, const char *key) {
    if (!g || !key) return nullptr;
    auto it = g->meta.find(key);
    return it == g->meta.end() || it->second.type != STRING ? nullptr : it->second.s.c_str();
}

int cw_gguf_experts(const cw_gguf *g, int layer, int which, int *dtype, int64_t *n_experts, int64_t *n, int64_t *k,
                    int64_t *expert_bytes, const void **data) {
    static const char *parts[3] = {"gate", "up", "down"};
    if (!g || which < 0 || which > 2 || layer < 0) return cw::set_error(CW_EINVAL, "gguf: bad expert query");
    char name[96];
    snprintf(name, sizeof name, "blk.%d.ffn_%s_exps.weight", layer, parts[which]);
    const int64_t i = cw_gguf_find(g, name);
    if (i < 0) return cw::set_error(CW_EINVAL, "gguf: no tensor %s", name);
    const Tensor &t = g->tensors[(size_t)i];
    if (t.dims.size() != 3 || t.dims[0] <= 0) return cw::set_error(CW_EINVAL, "gguf: %s is not [experts][rows][k]", name);
    const TypeSize ts = type_size(t.dtype);
    if ((t.dims[1] * t.dims[2]) % ts.block) return cw::set_error(CW_EINVAL, "gguf: %s expert is not whole blocks", name);
    if (dtype) *dtype = (int)t.dtype;
    if (n_experts) *n_experts = t.dims[0];
    if (n) *n = t.dims[1];
    if (k) *k = t.dims[2];
    if (expert_bytes) *expert_bytes = t.dims[1] * t.dims[2] / ts.block * ts.bytes;
    if (data) *data = cw_gguf_data(g, i);
    return CW_OK;
}

}  // extern "C"
