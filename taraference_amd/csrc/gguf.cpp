// GGUF v2/v3 reader (crates/gguf/src/reader.rs:29-169, value.rs:187-287,
// types.rs:109-180) and the dense-model configuration derived from its
// metadata (crates/core/src/config.rs:107-175).  Host code only: the file is
// memory-mapped read-only and tensor bytes are handed out as pointers into the
// mapping, for the caller to upload (cuda/load.rs:178-271).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "taraference_hip.h"

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" little-endian

// ggml type table: block size (elements) and bytes per block (types.rs:109-180).
struct TypeInfo {
    int block, bytes;
};
TypeInfo type_info(int t) {
    switch (t) {
    case 0: return {1, 4};     // F32
    case 1: return {1, 2};     // F16
    case 2: return {32, 18};   // Q4_0
    case 3: return {32, 20};   // Q4_1
    case 6: return {32, 22};   // Q5_0
    case 7: return {32, 24};   // Q5_1
    case 8: return {32, 34};   // Q8_0
    case 9: return {32, 36};   // Q8_1
    case 10: return {256, 84};   // Q2_K
    case 11: return {256, 110};  // Q3_K
    case 12: return {256, 144};  // Q4_K
    case 13: return {256, 176};  // Q5_K
    case 14: return {256, 210};  // Q6_K
    case 15: return {256, 292};  // Q8_K
    case 16: return {256, 64};   // IQ2_XXS
    case 17: return {256, 64};   // IQ2_XS
    case 18: return {256, 80};   // IQ3_XXS
    case 19: return {256, 50};   // IQ1_S
    case 20: return {256, 52};   // IQ4_NL
    case 21: return {256, 88};   // IQ3_S
    case 22: return {256, 68};   // IQ2_S
    case 23: return {256, 66};   // IQ4_XS
    case 24: return {1, 1};      // I8
    case 25: return {1, 2};      // I16
    case 26: return {1, 4};      // I32
    case 27: return {1, 8};      // I64
    case 28: return {1, 8};      // F64
    case 29: return {256, 56};   // IQ1_M
    case 30: return {1, 2};      // BF16
    default: return {0, 0};
    }
}

uint64_t type_nbytes(int t, uint64_t n) {
    const TypeInfo ti = type_info(t);
    if (ti.block == 0) return 0;
    if (ti.block == 1) return n * (uint64_t)ti.bytes;
    return (n + ti.block - 1) / ti.block * (uint64_t)ti.bytes;
}

// One metadata value (value.rs:54-70); arrays keep their items.
struct Value {
    int type = -1;
    uint64_t u = 0;   // U8/U16/U32/U64/Bool
    int64_t i = 0;    // I8/I16/I32/I64
    double f = 0.0;   // F32/F64
    std::string s;
    int item_type = -1;
    std::vector<Value> items;
};

struct Tensor {
    std::string name;
    int type;
    int n_dims;
    uint64_t dims[4];
    uint64_t offset;
    uint64_t nbytes;
};

struct Cursor {
    const uint8_t* p;
    size_t n, pos = 0;
    bool take(void* dst, size_t k) {
        if (n - pos < k) return false;
        std::memcpy(dst, p + pos, k);
        pos += k;
        return true;
    }
    template <class T>
    bool get(T& v) { return take(&v, sizeof(T)); }
};

bool utf8_ok(const std::string& s) {
    size_t i = 0;
    const size_t n = s.size();
    while (i < n) {
        const uint8_t c = (uint8_t)s[i];
        int k;
        uint32_t cp;
        if (c < 0x80) { i++; continue; }
        if ((c & 0xE0) == 0xC0) { k = 1; cp = c & 0x1F; }
        else if ((c & 0xF0) == 0xE0) { k = 2; cp = c & 0x0F; }
        else if ((c & 0xF8) == 0xF0) { k = 3; cp = c & 0x07; }
        else return false;
        if (n - i <= (size_t)k) return false;
        for (int j = 1; j <= k; j++) {
            const uint8_t cc = (uint8_t)s[i + j];
            if ((cc & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (cc & 0x3F);
        }
        // overlong forms, surrogates and values past U+10FFFF are invalid
        if ((k == 1 && cp < 0x80) || (k == 2 && cp < 0x800) || (k == 3 && cp < 0x10000) ||
            (cp >= 0xD800 && cp <= 0xDFFF) || cp > 0x10FFFF)
            return false;
        i += k + 1;
    }
    return true;
}

int read_string(Cursor& c, std::string& out) {
    uint64_t len;
    if (!c.get(len)) return TF_GGUF_ERR_EOF;
    if (len > 64ull * 1024 * 1024) return TF_GGUF_ERR_MALFORMED;
    if (c.n - c.pos < len) return TF_GGUF_ERR_EOF;
    out.assign(reinterpret_cast<const char*>(c.p + c.pos), (size_t)len);
    c.pos += len;
    if (!utf8_ok(out)) return TF_GGUF_ERR_UTF8;
    return 0;
}

int read_value(Cursor& c, int ty, Value& v) {
    v.type = ty;
    switch (ty) {
    case TF_GGUF_U8: { uint8_t x; if (!c.get(x)) return TF_GGUF_ERR_EOF; v.u = x; return 0; }
    case TF_GGUF_I8: { int8_t x; if (!c.get(x)) return TF_GGUF_ERR_EOF; v.i = x; return 0; }
    case TF_GGUF_U16: { uint16_t x; if (!c.get(x)) return TF_GGUF_ERR_EOF; v.u = x; return 0; }
    case TF_GGUF_I16: { int16_t x; if (!c.get(x)) return TF_GGUF_ERR_EOF; v.i = x; return 0; }
    case TF_GGUF_U32: { uint32_t x; if (!c.get(x)) return TF_GGUF_ERR_EOF; v.u = x; return 0; }
    case TF_GGUF_I32: { int32_t x; if (!c.get(x)) return TF_GGUF_ERR_EOF; v.i = x; return 0; }
    case TF_GGUF_F32: { float x; if (!c.get(x)) return TF_GGUF_ERR_EOF; v.f = x; return 0; }
    case TF_GGUF_BOOL: { uint8_t x; if (!c.get(x)) return TF_GGUF_ERR_EOF; v.u = x != 0; return 0; }
    case TF_GGUF_STRING: return read_string(c, v.s);
    case TF_GGUF_ARRAY: {
        uint32_t it;
        uint64_t n;
        if (!c.get(it)) return TF_GGUF_ERR_EOF;
        if (it > TF_GGUF_F64) return TF_GGUF_ERR_VALUE_TYPE;
        if (!c.get(n)) return TF_GGUF_ERR_EOF;
        if (n > 10000000ull) return TF_GGUF_ERR_MALFORMED;
        v.item_type = (int)it;
        v.items.resize((size_t)n);
        for (uint64_t k = 0; k < n; k++) {
            const int rc = read_value(c, (int)it, v.items[(size_t)k]);
            if (rc) return rc;
        }
        return 0;
    }
    case TF_GGUF_U64: { uint64_t x; if (!c.get(x)) return TF_GGUF_ERR_EOF; v.u = x; return 0; }
    case TF_GGUF_I64: { int64_t x; if (!c.get(x)) return TF_GGUF_ERR_EOF; v.i = x; return 0; }
    case TF_GGUF_F64: { double x; if (!c.get(x)) return TF_GGUF_ERR_EOF; v.f = x; return 0; }
    default: return TF_GGUF_ERR_VALUE_TYPE;
    }
}

// value.rs:72-106 conversions.
bool as_u32(const Value& v, uint32_t& out) {
    switch (v.type) {
    case TF_GGUF_U32: out = (uint32_t)v.u; return true;
    case TF_GGUF_U64: if (v.u > 0xFFFFFFFFull) return false; out = (uint32_t)v.u; return true;
    case TF_GGUF_I32: if (v.i < 0) return false; out = (uint32_t)v.i; return true;
    case TF_GGUF_U8:
    case TF_GGUF_U16: out = (uint32_t)v.u; return true;
    default: return false;
    }
}
bool as_u64(const Value& v, uint64_t& out) {
    switch (v.type) {
    case TF_GGUF_U64:
    case TF_GGUF_U32:
    case TF_GGUF_U8:
    case TF_GGUF_U16: out = v.u; return true;
    case TF_GGUF_I64:
    case TF_GGUF_I32: if (v.i < 0) return false; out = (uint64_t)v.i; return true;
    default: return false;
    }
}
bool as_f32(const Value& v, float& out) {
    if (v.type != TF_GGUF_F32 && v.type != TF_GGUF_F64) return false;
    out = (float)v.f;
    return true;
}

}  // namespace

struct tf_gguf {
    void* map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t data_offset = 0;
    std::unordered_map<std::string, Value> meta;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> index;
    ~tf_gguf() {
        if (map) munmap(map, size);
    }
    const Value* find(const char* key) const {
        if (!key) return nullptr;
        auto it = meta.find(key);
        return it == meta.end() ? nullptr : &it->second;
    }
};

namespace {

int parse(tf_gguf& g) {
    Cursor c{static_cast<const uint8_t*>(g.map), g.size};
    uint32_t magic;
    if (!c.get(magic)) return TF_GGUF_ERR_EOF;
    if (magic != kMagic) return TF_GGUF_ERR_MAGIC;
    if (!c.get(g.version)) return TF_GGUF_ERR_EOF;
    if (g.version != 2 && g.version != 3) return TF_GGUF_ERR_VERSION;
    uint64_t n_tensors, n_kv;
    if (!c.get(n_tensors) || !c.get(n_kv)) return TF_GGUF_ERR_EOF;
    if (n_tensors > 1000000ull || n_kv > 1000000ull) return TF_GGUF_ERR_MALFORMED;
    for (uint64_t k = 0; k < n_kv; k++) {
        std::string key;
        int rc = read_string(c, key);
        if (rc) return rc;
        uint32_t ty;
        if (!c.get(ty)) return TF_GGUF_ERR_EOF;
        if (ty > TF_GGUF_F64) return TF_GGUF_ERR_VALUE_TYPE;
        Value v;
        rc = read_value(c, (int)ty, v);
        if (rc) return rc;
        g.meta[key] = std::move(v);  // a repeated key keeps the last value
    }
    g.tensors.resize((size_t)n_tensors);
    for (uint64_t k = 0; k < n_tensors; k++) {
        Tensor& t = g.tensors[(size_t)k];
        int rc = read_string(c, t.name);
        if (rc) return rc;
        uint32_t nd;
        if (!c.get(nd)) return TF_GGUF_ERR_EOF;
        if (nd > 4) return TF_GGUF_ERR_MALFORMED;
        t.n_dims = (int)nd;
        for (int d = 0; d < 4; d++) t.dims[d] = 1;
        for (uint32_t d = 0; d < nd; d++)
            if (!c.get(t.dims[d])) return TF_GGUF_ERR_EOF;
        uint32_t ty;
        if (!c.get(ty)) return TF_GGUF_ERR_EOF;
        if (type_info((int)ty).block == 0) return TF_GGUF_ERR_TENSOR_TYPE;
        t.type = (int)ty;
        if (!c.get(t.offset)) return TF_GGUF_ERR_EOF;
        uint64_t n = 1;
        for (int d = 0; d < t.n_dims; d++) n *= t.dims[d];
        t.nbytes = type_nbytes(t.type, n);
        g.index[t.name] = (size_t)k;  // a repeated name finds the last tensor
    }
    uint64_t align = 32;
    if (const Value* a = g.find("general.alignment")) {
        uint64_t v;
        if (as_u64(*a, v)) align = v;
    }
    const uint64_t end = c.pos;
    g.data_offset = align == 0 ? end : (end + align - 1) / align * align;
    for (const Tensor& t : g.tensors) {
        const uint64_t start = g.data_offset + t.offset;
        if (start < t.offset || start + t.nbytes < start || start + t.nbytes > g.size)
            return TF_GGUF_ERR_MALFORMED;
    }
    return 0;
}

}  // namespace

extern "C" {

int tf_gguf_open(const char* path, tf_gguf** out) {
    if (!path || !out) return TF_GGUF_ERR_ARG;
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return TF_GGUF_ERR_IO;
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return TF_GGUF_ERR_IO;
    }
    std::unique_ptr<tf_gguf> g(new tf_gguf);
    g->size = (size_t)st.st_size;
    if (g->size > 0) {
        void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            close(fd);
            return TF_GGUF_ERR_IO;
        }
        g->map = m;
    }
    close(fd);
    const int rc = parse(*g);
    if (rc) return rc;
    *out = g.release();
    return 0;
}

void tf_gguf_close(tf_gguf* g) { delete g; }

uint32_t tf_gguf_version(const tf_gguf* g) { return g ? g->version : 0; }

uint64_t tf_gguf_data_offset(const tf_gguf* g) { return g ? g->data_offset : 0; }

uint64_t tf_gguf_file_size(const tf_gguf* g) { return g ? (uint64_t)g->size : 0; }

int64_t tf_gguf_n_tensors(const tf_gguf* g) { return g ? (int64_t)g->tensors.size() : -1; }

static void fill_tensor(const tf_gguf* g, const Tensor& t, tf_gguf_tensor* out) {
    out->name = t.name.c_str();
    out->type = t.type;
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; d++) out->dims[d] = t.dims[d];
    out->offset = t.offset;
    out->nbytes = t.nbytes;
    out->data = static_cast<const uint8_t*>(g->map) + g->data_offset + t.offset;
}

int tf_gguf_tensor_at(const tf_gguf* g, int64_t i, tf_gguf_tensor* out) {
    if (!g || !out || i < 0 || i >= (int64_t)g->tensors.size()) return TF_GGUF_ERR_ARG;
    fill_tensor(g, g->tensors[(size_t)i], out);
    return 0;
}

int tf_gguf_find_tensor(const tf_gguf* g, const char* name, tf_gguf_tensor* out) {
    if (!g || !name || !out) return TF_GGUF_ERR_ARG;
    auto it = g->index.find(name);
    if (it == g->index.end()) return TF_GGUF_ERR_NOT_FOUND;
    fill_tensor(g, g->tensors[it->second], out);
    return 0;
}

int tf_gguf_meta_type(const tf_gguf* g, const char* key) {
    const Value* v = g ? g->find(key) : nullptr;
    return v ? v->type : -1;
}

int tf_gguf_meta_u32(const tf_gguf* g, const char* key, uint32_t* out) {
    if (!g || !out) return TF_GGUF_ERR_ARG;
    const Value* v = g->find(key);
    if (!v) return TF_GGUF_ERR_NOT_FOUND;
    return as_u32(*v, *out) ? 0 : TF_GGUF_ERR_TYPE;
}

int tf_gguf_meta_u64(const tf_gguf* g, const char* key, uint64_t* out) {
    if (!g || !out) return TF_GGUF_ERR_ARG;
    const Value* v = g->find(key);
    if (!v) return TF_GGUF_ERR_NOT_FOUND;
    return as_u64(*v, *out) ? 0 : TF_GGUF_ERR_TYPE;
}

int tf_gguf_meta_i64(const tf_gguf* g, const char* key, int64_t* out) {
    if (!g || !out) return TF_GGUF_ERR_ARG;
    const Value* v = g->find(key);
    if (!v) return TF_GGUF_ERR_NOT_FOUND;
    switch (v->type) {
    case TF_GGUF_I8:
    case TF_GGUF_I16:
    case TF_GGUF_I32:
    case TF_GGUF_I64: *out = v->i; return 0;
    case TF_GGUF_U8:
    case TF_GGUF_U16:
    case TF_GGUF_U32:
    case TF_GGUF_BOOL: *out = (int64_t)v->u; return 0;
    case TF_GGUF_U64:
        if (v->u > 0x7FFFFFFFFFFFFFFFull) return TF_GGUF_ERR_TYPE;
        *out = (int64_t)v->u;
        return 0;
    default: return TF_GGUF_ERR_TYPE;
    }
}

int tf_gguf_meta_f64(const tf_gguf* g, const char* key, double* out) {
    if (!g || !out) return TF_GGUF_ERR_ARG;
    const Value* v = g->find(key);
    if (!v) return TF_GGUF_ERR_NOT_FOUND;
    if (v->type != TF_GGUF_F32 && v->type != TF_GGUF_F64) return TF_GGUF_ERR_TYPE;
    *out = v->f;
    return 0;
}

int tf_gguf_meta_f32(const tf_gguf* g, const char* key, float* out) {
    if (!g || !out) return TF_GGUF_ERR_ARG;
    const Value* v = g->find(key);
    if (!v) return TF_GGUF_ERR_NOT_FOUND;
    return as_f32(*v, *out) ? 0 : TF_GGUF_ERR_TYPE;
}

int tf_gguf_meta_bool(const tf_gguf* g, const char* key, int* out) {
    if (!g || !out) return TF_GGUF_ERR_ARG;
    const Value* v = g->find(key);
    if (!v) return TF_GGUF_ERR_NOT_FOUND;
    if (v->type != TF_GGUF_BOOL) return TF_GGUF_ERR_TYPE;
    *out = (int)v->u;
    return 0;
}

int tf_gguf_meta_str(const tf_gguf* g, const char* key, const char** s, uint64_t* len) {
    if (!g || !s || !len) return TF_GGUF_ERR_ARG;
    const Value* v = g->find(key);
    if (!v) return TF_GGUF_ERR_NOT_FOUND;
    if (v->type != TF_GGUF_STRING) return TF_GGUF_ERR_TYPE;
    *s = v->s.data();
    *len = v->s.size();
    return 0;
}

int tf_gguf_meta_array(const tf_gguf* g, const char* key, int* item_type, uint64_t* n) {
    if (!g || !item_type || !n) return TF_GGUF_ERR_ARG;
    const Value* v = g->find(key);
    if (!v) return TF_GGUF_ERR_NOT_FOUND;
    if (v->type != TF_GGUF_ARRAY) return TF_GGUF_ERR_TYPE;
    *item_type = v->item_type;
    *n = v->items.size();
    return 0;
}

int tf_gguf_meta_array_str(const tf_gguf* g, const char* key, uint64_t i, const char** s,
                           uint64_t* len) {
    if (!g || !s || !len) return TF_GGUF_ERR_ARG;
    const Value* v = g->find(key);
    if (!v) return TF_GGUF_ERR_NOT_FOUND;
    if (v->type != TF_GGUF_ARRAY || v->item_type != TF_GGUF_STRING) return TF_GGUF_ERR_TYPE;
    if (i >= v->items.size()) return TF_GGUF_ERR_ARG;
    *s = v->items[(size_t)i].s.data();
    *len = v->items[(size_t)i].s.size();
    return 0;
}

int tf_gguf_meta_array_f64(const tf_gguf* g, const char* key, uint64_t i, double* out) {
    if (!g || !out) return TF_GGUF_ERR_ARG;
    const Value* v = g->find(key);
    if (!v) return TF_GGUF_ERR_NOT_FOUND;
    if (v->type != TF_GGUF_ARRAY) return TF_GGUF_ERR_TYPE;
    if (i >= v->items.size()) return TF_GGUF_ERR_ARG;
    const Value& it = v->items[(size_t)i];
    switch (it.type) {
    case TF_GGUF_U8:
    case TF_GGUF_U16:
    case TF_GGUF_U32:
    case TF_GGUF_U64:
    case TF_GGUF_BOOL: *out = (double)it.u; return 0;
    case TF_GGUF_I8:
    case TF_GGUF_I16:
    case TF_GGUF_I32:
    case TF_GGUF_I64: *out = (double)it.i; return 0;
    case TF_GGUF_F32:
    case TF_GGUF_F64: *out = it.f; return 0;
    default: return TF_GGUF_ERR_TYPE;
    }
}

int tf_ggml_block_size(int type) { return type_info(type).block; }

int tf_ggml_type_size(int type) { return type_info(type).bytes; }

uint64_t tf_ggml_nbytes(int type, uint64_t n_elements) { return type_nbytes(type, n_elements); }

// config.rs:107-175 for the dense decoder (the fields tf_model_create takes).
int tf_gguf_model_config(const tf_gguf* g, int max_seq, tf_model_config* cfg) {
    if (!g || !cfg) return TF_GGUF_ERR_ARG;
    const char* arch;
    uint64_t alen;
    if (tf_gguf_meta_str(g, "general.architecture", &arch, &alen) != 0)
        return TF_GGUF_ERR_NOT_FOUND;
    std::string key(arch, (size_t)alen);
    if (key == "llama2" || key == "llama3") key = "llama";
    auto p = [&](const char* s) { return key + "." + s; };
    // u32, else u64 narrowed (config.rs:118-122)
    auto u = [&](const std::string& k, uint32_t& out) -> bool {
        if (tf_gguf_meta_u32(g, k.c_str(), &out) == 0) return true;
        uint64_t w;
        if (tf_gguf_meta_u64(g, k.c_str(), &w) == 0) {
            out = (uint32_t)w;
            return true;
        }
        return false;
    };
    uint32_t n_embd, n_layer, n_head, n_kv, hd, vd, n_ff;
    if (!u(p("embedding_length"), n_embd) || !u(p("block_count"), n_layer) ||
        !u(p("attention.head_count"), n_head) || !u(p("feed_forward_length"), n_ff))
        return TF_GGUF_ERR_NOT_FOUND;
    if (n_head == 0) return TF_GGUF_ERR_MALFORMED;
    if (!u(p("attention.head_count_kv"), n_kv)) n_kv = n_head;
    if (!u(p("attention.key_length"), hd)) hd = n_embd / n_head;
    if (!u(p("attention.value_length"), vd)) vd = hd;
    if (vd != hd) return TF_GGUF_ERR_MALFORMED;  // unsupported, as the reference
    uint32_t n_vocab;
    if (!u(p("vocab_size"), n_vocab)) {
        tf_gguf_tensor t;
        if (tf_gguf_find_tensor(g, "token_embd.weight", &t) != 0 || t.n_dims < 2)
            return TF_GGUF_ERR_NOT_FOUND;
        n_vocab = (uint32_t)t.dims[1];
    }
    float theta, eps;
    if (tf_gguf_meta_f32(g, p("rope.freq_base").c_str(), &theta) != 0)
        theta = key == "llama" ? 10000.0f : 1000000.0f;
    if (tf_gguf_meta_f32(g, p("attention.layer_norm_rms_epsilon").c_str(), &eps) != 0)
        eps = 1e-6f;
    cfg->n_layer = (int)n_layer;
    cfg->n_embd = (int)n_embd;
    cfg->n_ff = (int)n_ff;
    cfg->n_head = (int)n_head;
    cfg->n_kv = (int)n_kv;
    cfg->head_dim = (int)hd;
    cfg->n_vocab = (int)n_vocab;
    cfg->max_seq = max_seq;
    cfg->rope_theta = theta;
    cfg->rms_eps = eps;
    return 0;
}

}  // extern "C"
