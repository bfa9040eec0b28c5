// GGUF reader of kf-hip (host code): the file format the reference's loader reads (crates/kf-gguf/src/lib.rs), so
// real model tensors feed the quantized products with their bytes unchanged. GGUF v2 and v3: magic "GGUF", u32
// version, u64 tensor count, u64 key-value count, the typed key-value header, then per tensor its name, dims
// (innermost first), ggml type and offset into the data section, which starts at the header's end rounded up to
// general.alignment (32 when absent). Split files (name-0000i-of-0000N.gguf) open all their shards. Every shard is
// memory-mapped read-only and tensor data is handed out as pointers into the maps (no copy), as the reference's
// WeightSource borrows from its mmap.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/kf_hip.h"

void kf_set_error(const char* fmt, ...);  // api.cpp: the thread's last error

namespace {

// ggml block layouts the reference's kf_quant knows (crates/kf-quant/src/types/*.rs, TypeInfo statics): id -> (block, bytes)
bool ggml_layout(uint32_t id, int& block, int& bytes) {
    struct L {
        uint32_t id;
        int block, bytes;
    };
    static const L table[] = {{0, 1, 4},      {1, 1, 2},      {2, 32, 18},    {3, 32, 20},    {6, 32, 22},    {7, 32, 24},
                              {8, 32, 34},    {9, 32, 36},    {10, 256, 84},  {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
                              {14, 256, 210}, {15, 256, 292}, {16, 256, 66},  {17, 256, 74},  {18, 256, 98},  {19, 256, 50},
                              {20, 32, 18},   {21, 256, 110}, {22, 256, 82},  {23, 256, 136}, {29, 256, 56},  {30, 1, 2},
                              {34, 256, 54},  {35, 256, 66},  {39, 32, 17},   {40, 64, 36},   {41, 128, 18},  {42, 64, 18}};
    for (const L& l : table)
        if (l.id == id) {
            block = l.block;
            bytes = l.bytes;
            return true;
        }
    return false;
}

// One metadata value (crates/kf-gguf/src/lib.rs:11-26): scalar kinds 0..12, arrays (kind 9) of any kind, nested
struct Value {
    uint32_t kind = 0;
    uint64_t u = 0;  // unsigned integers, bool
    int64_t i = 0;   // signed integers
    double f = 0.0;  // f32 / f64
    std::string s;
    uint32_t elem = 0;  // arrays: element kind
    std::vector<Value> arr;
};

struct Tensor {
    std::string name;
    std::vector<int64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;
    int shard = 0;
    int64_t nbytes = -1;  // -1: a type without a known layout, or dims that do not fit it
};

struct Shard {
    std::string path;
    const uint8_t* map = nullptr;
    size_t size = 0;
    size_t data_start = 0;
};

struct Cursor {
    const uint8_t* buf;
    size_t size, at;
    bool ok = true;
    char err[160] = {0};

    bool take(size_t n, const uint8_t** p) {
        if (!ok) return false;
        if (n > size || at > size - n) {
            ok = false;
            snprintf(err, sizeof err, "truncated header at %zu", at);
            return false;
        }
        *p = buf + at;
        at += n;
        return true;
    }
    template <class T>
    T scalar() {
        const uint8_t* p;
        T v{};
        if (take(sizeof(T), &p)) std::memcpy(&v, p, sizeof(T));  // little-endian host, as GGUF
        return v;
    }
    std::string str() {
        const uint64_t n = scalar<uint64_t>();
        const uint8_t* p;
        if (!take((size_t)n, &p)) return std::string();
        return std::string(reinterpret_cast<const char*>(p), (size_t)n);
    }
    Value value(uint32_t kind, int depth) {
        Value v;
        v.kind = kind;
        switch (kind) {
            case 0: v.u = scalar<uint8_t>(); break;
            case 1: v.i = scalar<int8_t>(); break;
            case 2: v.u = scalar<uint16_t>(); break;
            case 3: v.i = scalar<int16_t>(); break;
            case 4: v.u = scalar<uint32_t>(); break;
            case 5: v.i = scalar<int32_t>(); break;
            case 6: v.f = scalar<float>(); break;
            case 7: v.u = scalar<uint8_t>() != 0; break;
            case 8: v.s = str(); break;
            case 9: {
                if (depth > 8) {
                    ok = false;
                    snprintf(err, sizeof err, "arrays nested deeper than 8 at %zu", at);
                    break;
                }
                v.elem = scalar<uint32_t>();
                const uint64_t n = scalar<uint64_t>();
                if (!ok) break;
                // every element takes at least one byte: a count past the buffer is a truncated header
                if (n > size - at) {
                    ok = false;
                    snprintf(err, sizeof err, "array of %llu elements past the end at %zu", (unsigned long long)n, at);
                    break;
                }
                v.arr.reserve((size_t)n);
                for (uint64_t k = 0; k < n && ok; k++) v.arr.push_back(value(v.elem, depth + 1));
                break;
            }
            case 10: v.u = scalar<uint64_t>(); break;
            case 11: v.i = scalar<int64_t>(); break;
            case 12: v.f = scalar<double>(); break;
            default:
                ok = false;
                snprintf(err, sizeof err, "unknown metadata value type %u", kind);
        }
        return v;
    }
};

// Value::as_u64 / as_i64 / as_f64 (crates/kf-gguf/src/lib.rs:28-62)
bool as_u64(const Value& v, uint64_t& out) {
    switch (v.kind) {
        case 0: case 2: case 4: case 10: case 7: out = v.u; return true;
        case 1: case 3: case 5: case 11:
            if (v.i < 0) return false;
            out = (uint64_t)v.i;
            return true;
        default: return false;
    }
}
bool as_i64(const Value& v, int64_t& out) {
    switch (v.kind) {
        case 1: case 3: case 5: case 11: out = v.i; return true;
        default: {
            uint64_t u;
            if (!as_u64(v, u)) return false;
            out = (int64_t)u;
            return true;
        }
    }
}
bool as_f64(const Value& v, double& out) {
    if (v.kind == 6 || v.kind == 12) {
        out = v.f;
        return true;
    }
    int64_t i;
    if (!as_i64(v, i)) return false;
    out = (double)i;
    return true;
}

// shard_paths (crates/kf-gguf/src/lib.rs:226-239): base-0000i-of-0000N.gguf opens all N, any other name itself
std::vector<std::string> shard_paths(const std::string& path) {
    const size_t slash = path.find_last_of('/');
    const std::string dir = slash == std::string::npos ? std::string() : path.substr(0, slash + 1);
    const std::string name = slash == std::string::npos ? path : path.substr(slash + 1);
    const size_t of = name.rfind("-of-");
    if (of == std::string::npos) return {path};
    const std::string rest = name.substr(of + 4);
    if (rest.size() <= 5 || rest.compare(rest.size() - 5, 5, ".gguf") != 0) return {path};
    const std::string tot = rest.substr(0, rest.size() - 5);
    if (tot.empty() || tot.find_first_not_of("0123456789") != std::string::npos) return {path};
    const size_t total = std::stoul(tot);
    const std::string stem = name.substr(0, of);
    const size_t dash = stem.rfind('-');
    if (dash == std::string::npos) return {path};
    const std::string idx = stem.substr(dash + 1);
    if (idx.size() != 5 || idx.find_first_not_of("0123456789") != std::string::npos) return {path};
    const std::string base = stem.substr(0, dash);
    std::vector<std::string> out;
    for (size_t i = 1; i <= total; i++) {
        char buf[32];
        snprintf(buf, sizeof buf, "-%05zu-of-%05zu.gguf", i, total);
        out.push_back(dir + base + buf);
    }
    return out;
}

}  // namespace

struct kf_gguf {
    std::map<std::string, Value> meta;  // sorted by key, later keys replace earlier ones (a BTreeMap in the reference)
    std::vector<const std::pair<const std::string, Value>*> meta_order;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int64_t> by_name;
    std::vector<Shard> shards;

    ~kf_gguf() {
        for (Shard& s : shards)
            if (s.map) munmap(const_cast<uint8_t*>(s.map), s.size);
    }
};

namespace {

bool parse(kf_gguf* g, Shard& sh, int shard_index, bool keep_meta) {
    Cursor c{sh.map, sh.size, 0};
    const uint8_t* magic;
    if (!c.take(4, &magic) || std::memcmp(magic, "GGUF", 4) != 0) {
        kf_set_error("%s: not a GGUF file", sh.path.c_str());
        return false;
    }
    const uint32_t version = c.scalar<uint32_t>();
    if (c.ok && version != 2 && version != 3) {
        kf_set_error("%s: unsupported GGUF version %u", sh.path.c_str(), version);
        return false;
    }
    const uint64_t n_tensors = c.scalar<uint64_t>();
    const uint64_t n_kv = c.scalar<uint64_t>();
    std::map<std::string, Value> meta;
    for (uint64_t k = 0; k < n_kv && c.ok; k++) {
        std::string key = c.str();
        const uint32_t kind = c.scalar<uint32_t>();
        Value v = c.value(kind, 0);
        if (c.ok) meta[key] = std::move(v);
    }
    std::vector<Tensor> ts;
    for (uint64_t t = 0; t < n_tensors && c.ok; t++) {
        Tensor x;
        x.name = c.str();
        const uint32_t nd = c.scalar<uint32_t>();
        if (c.ok && nd > 16) {
            kf_set_error("%s: tensor with %u dims", sh.path.c_str(), nd);
            return false;
        }
        for (uint32_t d = 0; d < nd && c.ok; d++) x.dims.push_back((int64_t)c.scalar<uint64_t>());
        x.type = c.scalar<uint32_t>();
        x.offset = c.scalar<uint64_t>();
        x.shard = shard_index;
        // nbytes (crates/kf-quant/src/lib.rs:224-232): inner dim a multiple of the block, rows = product of the rest
        int block, bytes;
        if (!x.dims.empty() && ggml_layout(x.type, block, bytes) && x.dims[0] % block == 0) {
            int64_t rows = 1;
            for (size_t d = 1; d < x.dims.size(); d++) rows *= x.dims[d];
            x.nbytes = x.dims[0] / block * bytes * rows;
        }
        ts.push_back(std::move(x));
    }
    if (!c.ok) {
        kf_set_error("%s: %s", sh.path.c_str(), c.err);
        return false;
    }
    size_t alignment = 32;
    const auto al = meta.find("general.alignment");
    uint64_t a;
    if (al != meta.end() && as_u64(al->second, a) && a > 0) alignment = (size_t)a;
    sh.data_start = (c.at + alignment - 1) / alignment * alignment;
    if (keep_meta) g->meta = std::move(meta);
    for (Tensor& x : ts) g->tensors.push_back(std::move(x));
    return true;
}

const Value* kv_value(const kf_gguf* g, int64_t i) {
    if (!g || i < 0 || i >= (int64_t)g->meta_order.size()) {
        kf_set_error("metadata index %lld out of range", (long long)i);
        return nullptr;
    }
    return &g->meta_order[(size_t)i]->second;
}

// element idx of an array value, or the value itself (idx 0) for a scalar
const Value* element(const Value* v, uint64_t idx) {
    if (!v) return nullptr;
    if (v->kind == 9) {
        if (idx >= v->arr.size()) {
            kf_set_error("array index %llu of %zu elements", (unsigned long long)idx, v->arr.size());
            return nullptr;
        }
        return &v->arr[(size_t)idx];
    }
    if (idx != 0) {
        kf_set_error("index %llu into a scalar value", (unsigned long long)idx);
        return nullptr;
    }
    return v;
}

}  // namespace

extern "C" {

kf_gguf* kf_gguf_open(const char* path) {
    if (!path) {
        kf_set_error("null path");
        return nullptr;
    }
    std::unique_ptr<kf_gguf> g(new kf_gguf());
    const std::vector<std::string> paths = shard_paths(path);
    for (size_t i = 0; i < paths.size(); i++) {
        Shard sh;
        sh.path = paths[i];
        const int fd = open(sh.path.c_str(), O_RDONLY);
        if (fd < 0) {
            kf_set_error("open %s: %s", sh.path.c_str(), strerror(errno));
            return nullptr;
        }
        struct stat st;
        if (fstat(fd, &st) != 0 || st.st_size <= 0) {
            close(fd);
            kf_set_error("%s: empty or unreadable", sh.path.c_str());
            return nullptr;
        }
        sh.size = (size_t)st.st_size;
        void* m = mmap(nullptr, sh.size, PROT_READ, MAP_PRIVATE, fd, 0);
        close(fd);
        if (m == MAP_FAILED) {
            kf_set_error("map %s: %s", sh.path.c_str(), strerror(errno));
            return nullptr;
        }
        sh.map = static_cast<const uint8_t*>(m);
        g->shards.push_back(sh);
        if (!parse(g.get(), g->shards.back(), (int)i, i == 0)) return nullptr;
    }
    for (const auto& kv : g->meta) g->meta_order.push_back(&kv);
    for (size_t i = 0; i < g->tensors.size(); i++) g->by_name[g->tensors[i].name] = (int64_t)i;
    return g.release();
}

void kf_gguf_close(kf_gguf* g) { delete g; }

int kf_gguf_n_shards(const kf_gguf* g) { return g ? (int)g->shards.size() : KF_E_INVALID; }

int64_t kf_gguf_n_tensors(const kf_gguf* g) { return g ? (int64_t)g->tensors.size() : KF_E_INVALID; }

int64_t kf_gguf_find_tensor(const kf_gguf* g, const char* name) {
    if (!g || !name) return KF_E_INVALID;
    const auto it = g->by_name.find(name);
    if (it == g->by_name.end()) {
        kf_set_error("no tensor %s", name);
        return KF_E_INVALID;
    }
    return it->second;
}

int kf_gguf_tensor_info(const kf_gguf* g, int64_t i, const char** name, int64_t* dims, int max_dims, uint32_t* ggml_type, int* shard,
                        uint64_t* offset, int64_t* nbytes) {
    if (!g || i < 0 || i >= (int64_t)g->tensors.size()) {
        kf_set_error("tensor index %lld out of range", (long long)i);
        return KF_E_INVALID;
    }
    const Tensor& t = g->tensors[(size_t)i];
    if (name) *name = t.name.c_str();
    for (int d = 0; dims && d < max_dims && d < (int)t.dims.size(); d++) dims[d] = t.dims[(size_t)d];
    if (ggml_type) *ggml_type = t.type;
    if (shard) *shard = t.shard;
    if (offset) *offset = t.offset;
    if (nbytes) *nbytes = t.nbytes;
    return (int)t.dims.size();
}

const void* kf_gguf_tensor_data(const kf_gguf* g, int64_t i) {
    if (!g || i < 0 || i >= (int64_t)g->tensors.size()) {
        kf_set_error("tensor index %lld out of range", (long long)i);
        return nullptr;
    }
    const Tensor& t = g->tensors[(size_t)i];
    if (t.nbytes < 0) {
        kf_set_error("%s: ggml type %u does not fit dims", t.name.c_str(), t.type);
        return nullptr;
    }
    const Shard& sh = g->shards[(size_t)t.shard];
    const uint64_t start = sh.data_start + t.offset;
    if (start > sh.size || (uint64_t)t.nbytes > sh.size - start) {
        kf_set_error("%s: data past end of %s", t.name.c_str(), sh.path.c_str());
        return nullptr;
    }
    return sh.map + start;
}

int64_t kf_gguf_n_kv(const kf_gguf* g) { return g ? (int64_t)g->meta_order.size() : KF_E_INVALID; }

int64_t kf_gguf_find_kv(const kf_gguf* g, const char* key) {
    if (!g || !key) return KF_E_INVALID;
    const auto it = g->meta.find(key);
    if (it == g->meta.end()) {
        kf_set_error("no metadata key %s", key);
        return KF_E_INVALID;
    }
    for (size_t i = 0; i < g->meta_order.size(); i++)
        if (g->meta_order[i] == &*it) return (int64_t)i;
    return KF_E_INVALID;
}

int kf_gguf_kv(const kf_gguf* g, int64_t i, const char** key, uint32_t* kind, uint32_t* elem_kind, uint64_t* count) {
    const Value* v = kv_value(g, i);
    if (!v) return KF_E_INVALID;
    if (key) *key = g->meta_order[(size_t)i]->first.c_str();
    if (kind) *kind = v->kind;
    if (elem_kind) *elem_kind = v->kind == 9 ? v->elem : v->kind;
    if (count) *count = v->kind == 9 ? v->arr.size() : 1;
    return KF_OK;
}

int kf_gguf_kv_u64(const kf_gguf* g, int64_t i, uint64_t idx, uint64_t* out) {
    const Value* v = element(kv_value(g, i), idx);
    if (!v || !out) return KF_E_INVALID;
    if (!as_u64(*v, *out)) {
        kf_set_error("metadata value of type %u is not an unsigned integer", v->kind);
        return KF_E_INVALID;
    }
    return KF_OK;
}

int kf_gguf_kv_i64(const kf_gguf* g, int64_t i, uint64_t idx, int64_t* out) {
    const Value* v = element(kv_value(g, i), idx);
    if (!v || !out) return KF_E_INVALID;
    if (!as_i64(*v, *out)) {
        kf_set_error("metadata value of type %u is not an integer", v->kind);
        return KF_E_INVALID;
    }
    return KF_OK;
}

int kf_gguf_kv_f64(const kf_gguf* g, int64_t i, uint64_t idx, double* out) {
    const Value* v = element(kv_value(g, i), idx);
    if (!v || !out) return KF_E_INVALID;
    if (!as_f64(*v, *out)) {
        kf_set_error("metadata value of type %u is not a number", v->kind);
        return KF_E_INVALID;
    }
    return KF_OK;
}

int kf_gguf_kv_str(const kf_gguf* g, int64_t i, uint64_t idx, const char** out, uint64_t* len) {
    const Value* v = element(kv_value(g, i), idx);
    if (!v || !out) return KF_E_INVALID;
    if (v->kind != 8) {
        kf_set_error("metadata value of type %u is not a string", v->kind);
        return KF_E_INVALID;
    }
    *out = v->s.data();
    if (len) *len = v->s.size();
    return KF_OK;
}

}  // extern "C"
