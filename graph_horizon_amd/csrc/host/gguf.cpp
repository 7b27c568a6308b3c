// GGUF model files: parsing (gguf/loader/mod.rs:34-186, loader/cursor.rs, loader/value.rs,
// tensor_index.rs), the dense mistral3 configuration contract (family/mistral/config.rs:43-160)
// and tensor contract (family/mistral/tensors.rs:40-180), and upload into a gh_model in the
// canonical order of cpu/weights.rs:63-174.
//
// The file is untrusted input: it is mapped read-only, every read goes through a bounds-checked
// little-endian cursor, every tensor span is validated against the file size (and against
// every other span) before any byte is handed out, and no malformed file can crash the
// process — failures are GH_E_* statuses with a message from gh_gguf_last_error().
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../../include/gh_backend.h"

namespace {

thread_local std::string g_error;

int gguf_fail(int code, std::string msg) {
    g_error = std::move(msg);
    return code;
}

constexpr uint64_t kDefaultAlignment = 32;
constexpr uint32_t kMaxDims = 4;

// Metadata value: scalars widened, strings kept, arrays reduced to (element type, count)
// plus, for string arrays, nothing else (the token table is only counted).
struct Value {
    uint32_t type = 0;
    uint64_t u = 0;      // unsigned ints, bool
    int64_t i = 0;       // signed ints
    double f = 0;        // f32 / f64
    std::string s;       // string
    uint32_t elem = 0;   // array element type
    uint64_t count = 0;  // array length
};

enum : uint32_t {
    V_U8 = 0, V_I8 = 1, V_U16 = 2, V_I16 = 3, V_U32 = 4, V_I32 = 5, V_F32 = 6, V_BOOL = 7,
    V_STRING = 8, V_ARRAY = 9, V_U64 = 10, V_I64 = 11, V_F64 = 12
};

// Well-formed UTF-8 (shortest forms, no surrogates, <= U+10FFFF), as Rust's String::from_utf8.
bool valid_utf8(const uint8_t* s, size_t n) {
    size_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) { ++i; continue; }
        size_t k;
        uint32_t cp, min;
        if ((c & 0xE0) == 0xC0) { k = 1; cp = c & 0x1F; min = 0x80; }
        else if ((c & 0xF0) == 0xE0) { k = 2; cp = c & 0x0F; min = 0x800; }
        else if ((c & 0xF8) == 0xF0) { k = 3; cp = c & 0x07; min = 0x10000; }
        else return false;
        if (k > n - i - 1) return false;
        for (size_t j = 1; j <= k; ++j) {
            if ((s[i + j] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (s[i + j] & 0x3F);
        }
        if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
        i += k + 1;
    }
    return true;
}

struct Cursor {
    const uint8_t* p;
    size_t n, pos = 0;
    bool take(size_t k, const uint8_t** out) {
        if (k > n - pos) return false;  // pos <= n always
        *out = p + pos;
        pos += k;
        return true;
    }
    template <class T>
    bool get(T* v) {
        const uint8_t* b;
        if (!take(sizeof(T), &b)) return false;
        std::memcpy(v, b, sizeof(T));  // GGUF is little-endian, as is the host
        return true;
    }
    // GGUF string: u64 length + UTF-8 bytes (loader/cursor.rs:76-81). 0 = ok, 1 = truncated,
    // 2 = invalid UTF-8.
    int str(std::string* s) {
        uint64_t len;
        const uint8_t* b;
        if (!get(&len) || len > n - pos || !take((size_t)len, &b)) return 1;
        if (!valid_utf8(b, (size_t)len)) return 2;
        s->assign((const char*)b, (size_t)len);
        return 0;
    }
};

int str_fail(int r) {
    return gguf_fail(GH_E_INVALID, r == 2 ? "gguf: invalid utf-8 in string" : "gguf: file is truncated");
}

// Reads one value of type `t` (loader/cursor.rs:86-127). Returns a status.
int read_value(Cursor& c, uint32_t t, Value* v, bool keep) {
    v->type = t;
    const char* trunc = "gguf: file is truncated";
    switch (t) {
        case V_U8: { uint8_t x; if (!c.get(&x)) return gguf_fail(GH_E_INVALID, trunc); v->u = x; return GH_OK; }
        case V_I8: { int8_t x; if (!c.get(&x)) return gguf_fail(GH_E_INVALID, trunc); v->i = x; return GH_OK; }
        case V_U16: { uint16_t x; if (!c.get(&x)) return gguf_fail(GH_E_INVALID, trunc); v->u = x; return GH_OK; }
        case V_I16: { int16_t x; if (!c.get(&x)) return gguf_fail(GH_E_INVALID, trunc); v->i = x; return GH_OK; }
        case V_U32: { uint32_t x; if (!c.get(&x)) return gguf_fail(GH_E_INVALID, trunc); v->u = x; return GH_OK; }
        case V_I32: { int32_t x; if (!c.get(&x)) return gguf_fail(GH_E_INVALID, trunc); v->i = x; return GH_OK; }
        case V_F32: { float x; if (!c.get(&x)) return gguf_fail(GH_E_INVALID, trunc); v->f = x; return GH_OK; }
        case V_BOOL: { uint8_t x; if (!c.get(&x)) return gguf_fail(GH_E_INVALID, trunc); v->u = x != 0; return GH_OK; }
        case V_STRING: {
            std::string skip;
            const int r = c.str(keep ? &v->s : &skip);
            return r ? str_fail(r) : GH_OK;
        }
        case V_U64: { uint64_t x; if (!c.get(&x)) return gguf_fail(GH_E_INVALID, trunc); v->u = x; return GH_OK; }
        case V_I64: { int64_t x; if (!c.get(&x)) return gguf_fail(GH_E_INVALID, trunc); v->i = x; return GH_OK; }
        case V_F64: { double x; if (!c.get(&x)) return gguf_fail(GH_E_INVALID, trunc); v->f = x; return GH_OK; }
        case V_ARRAY: {
            uint32_t elem;
            uint64_t count;
            if (!c.get(&elem) || !c.get(&count)) return gguf_fail(GH_E_INVALID, trunc);
            if (elem == V_ARRAY) return gguf_fail(GH_E_INVALID, "gguf: nested arrays are not supported");
            v->elem = elem;
            v->count = count;
            // every element is read (bounds-checked) and dropped: an untrusted count can only
            // run the cursor to the end of the file
            Value item;
            for (uint64_t k = 0; k < count; ++k) {
                const int rc = read_value(c, elem, &item, false);
                if (rc) return rc;
            }
            return GH_OK;
        }
        default:
            return gguf_fail(GH_E_INVALID, "gguf: unknown metadata value type " + std::to_string(t));
    }
}

// Integer value as u64 (signed only when non-negative), GgufValue::as_u64 (loader/value.rs).
bool as_u64(const Value& v, uint64_t* out) {
    switch (v.type) {
        case V_U8: case V_U16: case V_U32: case V_U64: *out = v.u; return true;
        case V_I8: case V_I16: case V_I32: case V_I64:
            if (v.i < 0) return false;
            *out = (uint64_t)v.i;
            return true;
        default: return false;
    }
}

// (elements per block, bytes per block) of a ggml type (tensor_index.rs:87-106).
bool block_size(uint32_t t, uint64_t* block, uint64_t* bytes) {
    switch (t) {
        case 0: *block = 1; *bytes = 4; return true;     // F32
        case 1: *block = 1; *bytes = 2; return true;     // F16
        case 30: *block = 1; *bytes = 2; return true;    // BF16
        case 2: *block = 32; *bytes = 18; return true;   // Q4_0
        case 3: *block = 32; *bytes = 20; return true;   // Q4_1
        case 6: *block = 32; *bytes = 22; return true;   // Q5_0
        case 7: *block = 32; *bytes = 24; return true;   // Q5_1
        case 8: *block = 32; *bytes = 34; return true;   // Q8_0
        case 10: *block = 256; *bytes = 84; return true;  // Q2_K
        case 11: *block = 256; *bytes = 110; return true; // Q3_K
        case 12: *block = 256; *bytes = 144; return true; // Q4_K
        case 13: *block = 256; *bytes = 176; return true; // Q5_K
        case 14: *block = 256; *bytes = 210; return true; // Q6_K
        case 15: *block = 256; *bytes = 292; return true; // Q8_K
        default: return false;
    }
}

const char* type_name(uint32_t t) {
    switch (t) {
        case 0: return "F32"; case 1: return "F16"; case 30: return "BF16"; case 2: return "Q4_0";
        case 3: return "Q4_1"; case 6: return "Q5_0"; case 7: return "Q5_1"; case 8: return "Q8_0";
        case 10: return "Q2_K"; case 11: return "Q3_K"; case 12: return "Q4_K"; case 13: return "Q5_K";
        case 14: return "Q6_K"; case 15: return "Q8_K"; default: return "unknown";
    }
}

struct Tensor {
    std::string name;
    uint32_t n_dims = 0;
    uint64_t dims[kMaxDims] = {0, 0, 0, 0};
    uint32_t type = 0;
    uint64_t offset = 0;  // relative to the data section
    uint64_t start = 0, nbytes = 0;  // absolute file span, set by validation
};

// Byte length from the block layout; false for unknown types, element-count overflow or a
// count that is not a whole number of blocks (TensorInfo::byte_len).
bool byte_len(const Tensor& t, uint64_t* out) {
    uint64_t block, bytes, n = 1;
    if (!block_size(t.type, &block, &bytes)) return false;
    for (uint32_t i = 0; i < t.n_dims; ++i) {
        if (t.dims[i] != 0 && n > UINT64_MAX / t.dims[i]) return false;
        n *= t.dims[i];
    }
    if (n % block) return false;
    const uint64_t blocks = n / block;
    if (blocks != 0 && bytes > UINT64_MAX / blocks) return false;
    *out = blocks * bytes;
    return true;
}

}  // namespace

struct gh_gguf {
    const uint8_t* map = nullptr;
    size_t len = 0;
    uint32_t version = 0;
    uint64_t data_offset = 0;
    uint64_t kv_count = 0;
    std::unordered_map<std::string, Value> md;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> by_name;
};

namespace {

int parse(gh_gguf* g) {
    Cursor c{g->map, g->len};
    const uint8_t* magic;
    if (!c.take(4, &magic) || std::memcmp(magic, "GGUF", 4) != 0)
        return gguf_fail(GH_E_INVALID, "gguf: not a GGUF file (bad magic)");
    if (!c.get(&g->version)) return gguf_fail(GH_E_INVALID, "gguf: file is truncated");
    if (g->version != 2 && g->version != 3)
        return gguf_fail(GH_E_UNSUPPORTED, "gguf: unsupported GGUF version " + std::to_string(g->version));
    uint64_t tensor_count;
    if (!c.get(&tensor_count) || !c.get(&g->kv_count)) return gguf_fail(GH_E_INVALID, "gguf: file is truncated");
    // metadata (duplicate keys: the last one wins)
    for (uint64_t k = 0; k < g->kv_count; ++k) {
        std::string key;
        uint32_t vt;
        const int r = c.str(&key);
        if (r) return str_fail(r);
        if (!c.get(&vt)) return gguf_fail(GH_E_INVALID, "gguf: file is truncated");
        Value v;
        const int rc = read_value(c, vt, &v, true);
        if (rc) return rc;
        g->md[key] = std::move(v);
    }
    // tensor table
    for (uint64_t k = 0; k < tensor_count; ++k) {
        Tensor t;
        const int r = c.str(&t.name);
        if (r) return str_fail(r);
        if (!c.get(&t.n_dims)) return gguf_fail(GH_E_INVALID, "gguf: file is truncated");
        if (t.n_dims > kMaxDims) return gguf_fail(GH_E_INVALID, "gguf: tensor '" + t.name + "' has too many dimensions");
        for (uint32_t d = 0; d < t.n_dims; ++d)
            if (!c.get(&t.dims[d])) return gguf_fail(GH_E_INVALID, "gguf: file is truncated");
        if (!c.get(&t.type) || !c.get(&t.offset)) return gguf_fail(GH_E_INVALID, "gguf: file is truncated");
        g->tensors.push_back(std::move(t));
    }
    // data section: after the table, aligned to general.alignment (default 32)
    uint64_t align = kDefaultAlignment;
    auto it = g->md.find("general.alignment");
    uint64_t a;
    if (it != g->md.end() && as_u64(it->second, &a) && a > 0) align = a;
    const uint64_t pos = c.pos;
    const uint64_t rem = pos % align;
    if (rem && pos > UINT64_MAX - (align - rem)) return gguf_fail(GH_E_INVALID, "gguf: data section beyond end of file");
    g->data_offset = rem ? pos + (align - rem) : pos;
    if (g->data_offset > g->len) return gguf_fail(GH_E_INVALID, "gguf: data section beyond end of file");
    // every tensor span inside the file, none overlapping (GgufFile::validate_tensor_spans)
    std::vector<size_t> order;
    for (size_t i = 0; i < g->tensors.size(); ++i) {
        Tensor& t = g->tensors[i];
        if (!byte_len(t, &t.nbytes)) return gguf_fail(GH_E_INVALID, "gguf: cannot size tensor '" + t.name + "'");
        if (t.offset > UINT64_MAX - g->data_offset) return gguf_fail(GH_E_INVALID, "gguf: tensor offset overflow");
        t.start = g->data_offset + t.offset;
        if (t.nbytes > UINT64_MAX - t.start) return gguf_fail(GH_E_INVALID, "gguf: tensor length overflow");
        if (t.start + t.nbytes > g->len)
            return gguf_fail(GH_E_INVALID, "gguf: tensor '" + t.name + "' extends beyond end of file");
        order.push_back(i);
        g->by_name[t.name] = i;  // duplicate names: the last one wins
    }
    std::sort(order.begin(), order.end(), [&](size_t x, size_t y) { return g->tensors[x].start < g->tensors[y].start; });
    for (size_t k = 1; k < order.size(); ++k) {
        const Tensor& prev = g->tensors[order[k - 1]];
        const Tensor& next = g->tensors[order[k]];
        if (prev.start + prev.nbytes > next.start)
            return gguf_fail(GH_E_INVALID, "gguf: tensor '" + next.name + "' overlaps tensor '" + prev.name + "'");
    }
    return GH_OK;
}

// ---- mistral3 configuration contract (family/mistral/config.rs:43-160) ----

const Value* find(const gh_gguf* g, const std::string& key) {
    auto it = g->md.find(key);
    return it == g->md.end() ? nullptr : &it->second;
}

int e06(const std::string& key) { return gguf_fail(GH_E_INVALID, "E06 missing or invalid GGUF metadata '" + key + "'"); }

// positive unsigned (u8/u16/u32/u64 only, config.rs:128-141 and 156-164)
int pos_u32(const gh_gguf* g, const std::string& key, uint32_t* out) {
    const Value* v = find(g, key);
    if (!v || !(v->type == V_U8 || v->type == V_U16 || v->type == V_U32 || v->type == V_U64) || v->u == 0 ||
        v->u > UINT32_MAX)
        return e06(key);
    *out = (uint32_t)v->u;
    return GH_OK;
}

// positive finite F32 (config.rs:143-154)
int pos_f32(const gh_gguf* g, const std::string& key, float* out) {
    const Value* v = find(g, key);
    if (!v || v->type != V_F32) return e06(key);
    const float f = (float)v->f;
    if (!(f > 0.0f) || f > 3.4e38f) return e06(key);
    *out = f;
    return GH_OK;
}

// ---- tensor contract (family/mistral/tensors.rs:40-180) ----

const Tensor* tensor(const gh_gguf* g, const std::string& name) {
    auto it = g->by_name.find(name);
    return it == g->by_name.end() ? nullptr : &g->tensors[it->second];
}

int e07(const std::string& name) { return gguf_fail(GH_E_INVALID, "E07 missing or invalid tensor '" + name + "'"); }
int e08(uint32_t type) { return gguf_fail(GH_E_UNSUPPORTED, std::string("E08 unsupported tensor type '") + type_name(type) + "'"); }

int check_norm(const Tensor* t, const std::string& name, uint32_t len) {
    if (!t || t->n_dims != 1 || t->dims[0] != len) return e07(name);
    if (t->type != GH_FMT_F32) return e08(t->type);
    return GH_OK;
}

int check_matrix(const Tensor* t, const std::string& name, uint32_t in, uint32_t out) {
    if (!t || t->n_dims != 2 || t->dims[0] != in || t->dims[1] != out) return e07(name);
    if (t->type != GH_FMT_Q4_K && t->type != GH_FMT_Q6_K) return e08(t->type);
    return GH_OK;
}

const char* const kLayerNames[9] = {"attn_norm.weight",   "attn_q.weight",  "attn_k.weight",
                                    "attn_v.weight",      "attn_output.weight", "ffn_norm.weight",
                                    "ffn_gate.weight",    "ffn_up.weight",  "ffn_down.weight"};

// Resolves and checks every tensor of the model; `visit(layer, id, tensor)` is called in the
// canonical load order (token_embd, output_norm, output, then per layer) when non-null.
template <class F>
int walk_model(const gh_gguf* g, const gh_model_config& c, F&& visit) {
    const uint32_t d = c.embedding_length;
    int rc;
    const Tensor* embd = tensor(g, "token_embd.weight");
    if ((rc = check_matrix(embd, "token_embd.weight", d, c.vocab_size))) return rc;
    const Tensor* onorm = tensor(g, "output_norm.weight");
    if ((rc = check_norm(onorm, "output_norm.weight", d))) return rc;
    const Tensor* out = tensor(g, "output.weight");
    if (out && (rc = check_matrix(out, "output.weight", d, c.vocab_size))) return rc;
    const uint32_t qw = c.head_count * c.key_length, kw = c.kv_head_count * c.key_length;
    const uint32_t vw = c.kv_head_count * c.value_length, aw = c.head_count * c.value_length;
    const uint32_t ins[9] = {d, d, d, d, aw, d, d, d, c.feed_forward_length};
    const uint32_t outs[9] = {0, qw, kw, vw, d, 0, c.feed_forward_length, c.feed_forward_length, d};
    std::vector<const Tensor*> layer_t((size_t)c.block_count * 9);
    for (uint32_t i = 0; i < c.block_count; ++i)
        for (uint32_t k = 0; k < 9; ++k) {
            const std::string name = "blk." + std::to_string(i) + "." + kLayerNames[k];
            const Tensor* t = tensor(g, name);
            rc = (k == GH_T_ATTN_NORM || k == GH_T_FFN_NORM) ? check_norm(t, name, d)
                                                             : check_matrix(t, name, ins[k], outs[k]);
            if (rc) return rc;
            layer_t[(size_t)i * 9 + k] = t;
        }
    constexpr uint32_t kNoLayer = UINT32_MAX;
    if ((rc = visit(kNoLayer, (uint32_t)GH_T_TOKEN_EMBD, embd))) return rc;
    if ((rc = visit(kNoLayer, (uint32_t)GH_T_OUTPUT_NORM, onorm))) return rc;
    // tied output (no output.weight): the token table is the output matrix as well
    if ((rc = visit(kNoLayer, (uint32_t)GH_T_OUTPUT, out ? out : embd))) return rc;
    for (uint32_t i = 0; i < c.block_count; ++i)
        for (uint32_t k = 0; k < 9; ++k)
            if ((rc = visit(i, k, layer_t[(size_t)i * 9 + k]))) return rc;
    return GH_OK;
}

}  // namespace

extern "C" {

const char* gh_gguf_last_error(void) { return g_error.c_str(); }

int gh_gguf_open(const char* path, gh_gguf** out) {
    if (!path || !out) return gguf_fail(GH_E_INVALID, "gguf: null argument");
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return gguf_fail(GH_E_INVALID, "gguf: cannot open model file");
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        ::close(fd);
        return gguf_fail(GH_E_INVALID, "gguf: not a GGUF file (bad magic)");
    }
    void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) return gguf_fail(GH_E_INVALID, "gguf: cannot mmap model file");
    gh_gguf* g = new gh_gguf;
    g->map = (const uint8_t*)m;
    g->len = (size_t)st.st_size;
    const int rc = parse(g);
    if (rc) {
        gh_gguf_close(g);
        return rc;
    }
    *out = g;
    return GH_OK;
}

void gh_gguf_close(gh_gguf* g) {
    if (!g) return;
    if (g->map) munmap((void*)g->map, g->len);
    delete g;
}

int gh_gguf_info(const gh_gguf* g, uint32_t* version, uint64_t* tensor_count, uint64_t* kv_count,
                 uint64_t* data_offset) {
    if (!g) return gguf_fail(GH_E_INVALID, "gguf: null handle");
    if (version) *version = g->version;
    if (tensor_count) *tensor_count = g->tensors.size();
    if (kv_count) *kv_count = g->kv_count;
    if (data_offset) *data_offset = g->data_offset;
    return GH_OK;
}

int gh_gguf_tensor(const gh_gguf* g, uint64_t index, gh_gguf_tensor_info* out) {
    if (!g || !out) return gguf_fail(GH_E_INVALID, "gguf: null argument");
    if (index >= g->tensors.size()) return gguf_fail(GH_E_RANGE, "gguf: tensor index out of range");
    const Tensor& t = g->tensors[index];
    out->name = t.name.c_str();
    out->n_dims = t.n_dims;
    for (uint32_t i = 0; i < kMaxDims; ++i) out->dims[i] = t.dims[i];
    out->type = t.type;
    out->offset = t.offset;
    out->nbytes = t.nbytes;
    out->data = g->map + t.start;
    return GH_OK;
}

int gh_gguf_find(const gh_gguf* g, const char* name, uint64_t* index) {
    if (!g || !name || !index) return gguf_fail(GH_E_INVALID, "gguf: null argument");
    auto it = g->by_name.find(name);
    if (it == g->by_name.end()) return gguf_fail(GH_E_RANGE, std::string("gguf: no tensor '") + name + "'");
    *index = it->second;
    return GH_OK;
}

int gh_gguf_meta_u64(const gh_gguf* g, const char* key, uint64_t* out) {
    if (!g || !key || !out) return gguf_fail(GH_E_INVALID, "gguf: null argument");
    const Value* v = find(g, key);
    if (!v || !as_u64(*v, out)) return gguf_fail(GH_E_RANGE, std::string("gguf: no integer metadata '") + key + "'");
    return GH_OK;
}

int gh_gguf_meta_f64(const gh_gguf* g, const char* key, double* out) {
    if (!g || !key || !out) return gguf_fail(GH_E_INVALID, "gguf: null argument");
    const Value* v = find(g, key);
    if (!v || (v->type != V_F32 && v->type != V_F64))
        return gguf_fail(GH_E_RANGE, std::string("gguf: no float metadata '") + key + "'");
    *out = v->f;
    return GH_OK;
}

const char* gh_gguf_meta_str(const gh_gguf* g, const char* key) {
    if (!g || !key) return nullptr;
    const Value* v = find(g, key);
    return v && v->type == V_STRING ? v->s.c_str() : nullptr;
}

int gh_gguf_meta_array_len(const gh_gguf* g, const char* key, uint64_t* out) {
    if (!g || !key || !out) return gguf_fail(GH_E_INVALID, "gguf: null argument");
    const Value* v = find(g, key);
    if (!v || v->type != V_ARRAY) return gguf_fail(GH_E_RANGE, std::string("gguf: no array metadata '") + key + "'");
    *out = v->count;
    return GH_OK;
}

int gh_gguf_model_config(const gh_gguf* g, uint32_t kv_context, uint32_t prefill_rows, gh_model_config* cfg) {
    if (!g || !cfg) return gguf_fail(GH_E_INVALID, "gguf: null argument");
    const Value* scaling = find(g, "mistral3.rope.scaling.type");
    if (!scaling || scaling->type != V_STRING || scaling->s != "yarn") return e06("mistral3.rope.scaling.type");
    gh_model_config c{};
    uint32_t vocab, rope_dim, orig;
    int rc;
    if ((rc = pos_u32(g, "mistral3.block_count", &c.block_count))) return rc;
    if ((rc = pos_u32(g, "mistral3.context_length", &c.context_length))) return rc;
    if ((rc = pos_u32(g, "mistral3.embedding_length", &c.embedding_length))) return rc;
    if ((rc = pos_u32(g, "mistral3.feed_forward_length", &c.feed_forward_length))) return rc;
    if ((rc = pos_u32(g, "mistral3.vocab_size", &vocab))) return rc;
    // the vocabulary is the tokenizer's token table (config.rs:62-65)
    const Value* tokens = find(g, "tokenizer.ggml.tokens");
    if (!tokens || tokens->type != V_ARRAY || tokens->count != vocab) return e06("mistral3.vocab_size");
    c.vocab_size = vocab;
    if ((rc = pos_u32(g, "mistral3.attention.head_count", &c.head_count))) return rc;
    if ((rc = pos_u32(g, "mistral3.attention.head_count_kv", &c.kv_head_count))) return rc;
    if ((rc = pos_u32(g, "mistral3.attention.key_length", &c.key_length))) return rc;
    if ((rc = pos_u32(g, "mistral3.attention.value_length", &c.value_length))) return rc;
    if (c.kv_head_count > c.head_count || c.head_count % c.kv_head_count || c.embedding_length % c.head_count)
        return e06("mistral3.attention.head_count");
    if ((rc = pos_u32(g, "mistral3.rope.dimension_count", &rope_dim))) return rc;
    if (rope_dim > c.key_length || rope_dim % 2) return e06("mistral3.rope.dimension_count");
    // Q/K/V/attention widths must not overflow (config.rs:84-95)
    if ((uint64_t)c.head_count * c.key_length > UINT32_MAX || (uint64_t)c.head_count * c.value_length > UINT32_MAX)
        return e06("mistral3.attention.key_length");
    gh_yarn& y = c.yarn;
    y.rope_dim = rope_dim;
    if ((rc = pos_f32(g, "mistral3.rope.freq_base", &y.freq_base))) return rc;
    if ((rc = pos_f32(g, "mistral3.attention.layer_norm_rms_epsilon", &c.rms_epsilon))) return rc;
    if ((rc = pos_f32(g, "mistral3.rope.scaling.factor", &y.factor))) return rc;
    if ((rc = pos_f32(g, "mistral3.rope.scaling.yarn_beta_fast", &y.beta_fast))) return rc;
    if ((rc = pos_f32(g, "mistral3.rope.scaling.yarn_beta_slow", &y.beta_slow))) return rc;
    if ((rc = pos_f32(g, "mistral3.rope.scaling.yarn_log_multiplier", &y.log_multiplier))) return rc;
    if ((rc = pos_u32(g, "mistral3.rope.scaling.original_context_length", &orig))) return rc;
    y.original_context = orig;
    if ((rc = pos_f32(g, "mistral3.attention.temperature_scale", &y.q_temperature_scale))) return rc;
    if (kv_context == 0 || kv_context > c.context_length)
        return gguf_fail(GH_E_RANGE, "gguf: KV context outside 1..context_length");
    c.kv_context = kv_context;
    c.prefill_rows = prefill_rows;
    *cfg = c;
    return GH_OK;
}

int gh_gguf_check_model(const gh_gguf* g, const gh_model_config* cfg) {
    if (!g || !cfg) return gguf_fail(GH_E_INVALID, "gguf: null argument");
    return walk_model(g, *cfg, [](uint32_t, uint32_t, const Tensor*) { return (int)GH_OK; });
}

int gh_gguf_load_model(const gh_gguf* g, const gh_model_config* cfg, gh_model* m) {
    if (!g || !cfg || !m) return gguf_fail(GH_E_INVALID, "gguf: null argument");
    // everything is checked before the first byte is uploaded
    int rc = gh_gguf_check_model(g, cfg);
    if (rc) return rc;
    return walk_model(g, *cfg, [&](uint32_t layer, uint32_t id, const Tensor* t) {
        const int r = gh_model_load_tensor(m, layer, id, t->type, g->map + t->start, t->nbytes);
        return r ? gguf_fail(r, "gguf: upload of tensor '" + t->name + "' failed") : (int)GH_OK;
    });
}

}  // extern "C"
