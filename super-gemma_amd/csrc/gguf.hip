// GGUF v3 reader (host code) and the loader of a GGUF's tensors into a
// decode model.
//
// Format (crates/sg-gguf/src/parse.rs:112-210, the public GGUF v3 layout):
// u32 magic "GGUF", u32 version 3, u64 tensor_count, u64 kv_count; kv_count
// metadata entries (string key = u64 length + bytes, u32 value type, value;
// arrays = u32 element type + u64 count + elements); tensor_count tensor
// infos (name, u32 n_dims <= 4, u64 dims in ggml order — dims[0] is the
// contiguous one —, u32 ggml type, u64 offset); the data section starts at
// the next multiple of general.alignment (default 32) and every offset is a
// multiple of it.  Every read is bounds-checked against the file; malformed
// input is an error, never a crash.  The file is mapped read-only and
// tensor data is handed out as pointers into the mapping.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "sgq_internal.h"

struct sgq_gguf {
    int fd = -1;
    const uint8_t *map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32;
    size_t data_start = 0;
    struct Tensor {
        std::string name;
        uint32_t n_dims, type;
        uint64_t dims[4];
        uint64_t offset, bytes;
    };
    struct Meta {
        uint32_t type;  // GGUF value type
        uint64_t u = 0;
        int64_t i = 0;
        double f = 0;
        std::string s;
    };
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> index;
    std::unordered_map<std::string, Meta> meta;
};

using namespace sgq;

namespace {

// ggml types this library reads: (elements per block, bytes per block).
bool ggml_block(uint32_t type, uint64_t *elems, uint64_t *bytes) {
    switch (type) {
        case 0: *elems = 1, *bytes = 4; return true;     // F32
        case 1: *elems = 1, *bytes = 2; return true;     // F16
        case 2: *elems = 32, *bytes = 18; return true;   // Q4_0
        case 8: *elems = 32, *bytes = 34; return true;   // Q8_0
        case 14: *elems = 256, *bytes = 210; return true; // Q6_K
        default: return false;
    }
}

struct Cursor {
    const uint8_t *p;
    size_t size, pos = 0;
    bool take(size_t n, const uint8_t **out) {
        if (n > size - pos) return false;
        *out = p + pos;
        pos += n;
        return true;
    }
    template <typename T>
    bool get(T *v) {
        const uint8_t *b;
        if (!take(sizeof(T), &b)) return false;
        std::memcpy(v, b, sizeof(T));
        return true;
    }
    bool str(std::string *s) {
        uint64_t n;
        const uint8_t *b;
        if (!get(&n) || n > size - pos || !take((size_t)n, &b)) return false;
        s->assign(reinterpret_cast<const char *>(b), (size_t)n);
        return true;
    }
};

int bad(const char *what, size_t at) {
    return fail(SGQ_ERR_VALIDATION, "gguf: malformed or truncated %s at offset %zu", what, at);
}

// One metadata value of type `ty` (scalars kept; arrays walked and skipped).
int read_value(Cursor &c, uint32_t ty, sgq_gguf::Meta *m, int depth) {
    m->type = ty;
    const size_t at = c.pos;
    switch (ty) {
        case 0: { uint8_t v; if (!c.get(&v)) return bad("u8 value", at); m->u = v; m->i = v; return SGQ_OK; }
        case 1: { int8_t v; if (!c.get(&v)) return bad("i8 value", at); m->i = v; m->u = (uint64_t)v; return SGQ_OK; }
        case 2: { uint16_t v; if (!c.get(&v)) return bad("u16 value", at); m->u = v; m->i = v; return SGQ_OK; }
        case 3: { int16_t v; if (!c.get(&v)) return bad("i16 value", at); m->i = v; m->u = (uint64_t)v; return SGQ_OK; }
        case 4: { uint32_t v; if (!c.get(&v)) return bad("u32 value", at); m->u = v; m->i = v; return SGQ_OK; }
        case 5: { int32_t v; if (!c.get(&v)) return bad("i32 value", at); m->i = v; m->u = (uint64_t)v; return SGQ_OK; }
        case 6: { float v; if (!c.get(&v)) return bad("f32 value", at); m->f = v; return SGQ_OK; }
        case 7: {
            uint8_t v;
            if (!c.get(&v) || v > 1) return bad("bool value", at);
            m->u = v;
            return SGQ_OK;
        }
        case 8: if (!c.str(&m->s)) return bad("string value", at); return SGQ_OK;
        case 9: {
            if (depth >= 8) return fail(SGQ_ERR_VALIDATION, "gguf: arrays nested too deep at %zu", at);
            uint32_t et;
            uint64_t n;
            if (!c.get(&et) || !c.get(&n)) return bad("array header", at);
            m->u = n;  // element count
            for (uint64_t k = 0; k < n; k++) {
                sgq_gguf::Meta e;
                if (int rc = read_value(c, et, &e, depth + 1)) return rc;
            }
            return SGQ_OK;
        }
        case 10: { uint64_t v; if (!c.get(&v)) return bad("u64 value", at); m->u = v; m->i = (int64_t)v; return SGQ_OK; }
        case 11: { int64_t v; if (!c.get(&v)) return bad("i64 value", at); m->i = v; m->u = (uint64_t)v; return SGQ_OK; }
        case 12: { double v; if (!c.get(&v)) return bad("f64 value", at); m->f = v; return SGQ_OK; }
        default: return fail(SGQ_ERR_VALIDATION, "gguf: unknown value type %u at %zu", ty, at);
    }
}

int parse(sgq_gguf *g) {
    Cursor c{g->map, g->size};
    uint32_t magic;
    uint64_t n_tensors, n_kv;
    if (!c.get(&magic)) return bad("magic", 0);
    if (magic != 0x46554747u) return fail(SGQ_ERR_VALIDATION, "gguf: bad magic %#010x", magic);
    if (!c.get(&g->version)) return bad("version", 4);
    if (g->version != 3) return fail(SGQ_ERR_VALIDATION, "gguf: unsupported version %u", g->version);
    if (!c.get(&n_tensors) || !c.get(&n_kv)) return bad("counts", 8);
    for (uint64_t k = 0; k < n_kv; k++) {
        std::string key;
        uint32_t ty;
        const size_t at = c.pos;
        if (!c.str(&key) || !c.get(&ty)) return bad("metadata key", at);
        sgq_gguf::Meta m;
        if (int rc = read_value(c, ty, &m, 0)) return rc;
        if (!g->meta.emplace(key, std::move(m)).second)
            return fail(SGQ_ERR_VALIDATION, "gguf: duplicate metadata key '%s'", key.c_str());
    }
    auto al = g->meta.find("general.alignment");
    if (al != g->meta.end()) {
        const uint64_t a = al->second.u;
        if (al->second.type > 11 || al->second.type == 6 || al->second.type == 7 ||
            al->second.type == 8 || al->second.type == 9 || a == 0 || (a & (a - 1)))
            return fail(SGQ_ERR_VALIDATION, "gguf: bad general.alignment");
        g->alignment = a;
    }
    for (uint64_t k = 0; k < n_tensors; k++) {
        sgq_gguf::Tensor t{};
        const size_t at = c.pos;
        if (!c.str(&t.name) || !c.get(&t.n_dims)) return bad("tensor info", at);
        if (t.n_dims > 4) return fail(SGQ_ERR_VALIDATION, "gguf: tensor '%s' has %u dims", t.name.c_str(), t.n_dims);
        uint64_t elems = 1;
        for (uint32_t d = 0; d < 4; d++) t.dims[d] = 1;
        for (uint32_t d = 0; d < t.n_dims; d++) {
            if (!c.get(&t.dims[d])) return bad("tensor dims", at);
            if (t.dims[d] && elems > UINT64_MAX / t.dims[d])
                return fail(SGQ_ERR_VALIDATION, "gguf: tensor '%s' size overflows", t.name.c_str());
            elems *= t.dims[d];
        }
        if (!c.get(&t.type) || !c.get(&t.offset)) return bad("tensor type/offset", at);
        uint64_t be, bb;
        if (!ggml_block(t.type, &be, &bb))
            return fail(SGQ_ERR_VALIDATION, "gguf: tensor '%s' has unsupported type %u", t.name.c_str(), t.type);
        if (elems % be) return fail(SGQ_ERR_VALIDATION, "gguf: tensor '%s' is not whole blocks", t.name.c_str());
        t.bytes = elems / be * bb;
        if (!g->index.emplace(t.name, g->tensors.size()).second)
            return fail(SGQ_ERR_VALIDATION, "gguf: duplicate tensor '%s'", t.name.c_str());
        g->tensors.push_back(std::move(t));
    }
    const uint64_t a = g->alignment;
    const uint64_t ds = ((uint64_t)c.pos + a - 1) / a * a;
    if (ds > g->size && !g->tensors.empty()) return bad("data section", c.pos);
    g->data_start = (size_t)std::min<uint64_t>(ds, g->size);
    const uint64_t data_len = g->size - g->data_start;
    for (const auto &t : g->tensors) {
        if (t.offset % a)
            return fail(SGQ_ERR_VALIDATION, "gguf: tensor '%s' offset %llu is not aligned to %llu",
                        t.name.c_str(), (unsigned long long)t.offset, (unsigned long long)a);
        if (t.offset > data_len || t.bytes > data_len - t.offset)
            return fail(SGQ_ERR_VALIDATION, "gguf: tensor '%s' lies outside the data section",
                        t.name.c_str());
    }
    return SGQ_OK;
}

void fill(const sgq_gguf *g, const sgq_gguf::Tensor &t, sgq_gguf_tensor *out) {
    out->name = t.name.c_str();
    out->type = t.type;
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; d++) out->dims[d] = t.dims[d];
    out->offset = t.offset;
    out->bytes = t.bytes;
    out->data = g->map + g->data_start + t.offset;
}

}  // namespace

extern "C" {

int sgq_gguf_open(const char *path, sgq_gguf **out) {
    if (!path || !out) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    *out = nullptr;
    auto *g = new sgq_gguf;
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (g->fd < 0) {
        delete g;
        return fail(SGQ_ERR_VALIDATION, "gguf: cannot open '%s'", path);
    }
    struct stat st;
    if (fstat(g->fd, &st) != 0 || st.st_size <= 0) {
        sgq_gguf_close(g);
        return fail(SGQ_ERR_VALIDATION, "gguf: '%s' is empty or unreadable", path);
    }
    g->size = (size_t)st.st_size;
    void *p = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (p == MAP_FAILED) {
        sgq_gguf_close(g);
        return fail(SGQ_ERR_VALIDATION, "gguf: cannot map '%s'", path);
    }
    g->map = static_cast<const uint8_t *>(p);
    if (int rc = parse(g)) {
        sgq_gguf_close(g);
        return rc;
    }
    *out = g;
    return SGQ_OK;
}

int sgq_gguf_close(sgq_gguf *g) {
    if (!g) return SGQ_OK;
    if (g->map) munmap(const_cast<uint8_t *>(g->map), g->size);
    if (g->fd >= 0) close(g->fd);
    delete g;
    return SGQ_OK;
}

uint64_t sgq_gguf_tensor_count(const sgq_gguf *g) { return g ? g->tensors.size() : 0; }

int sgq_gguf_tensor_at(const sgq_gguf *g, uint64_t i, sgq_gguf_tensor *out) {
    if (!g || !out) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    if (i >= g->tensors.size()) return fail(SGQ_ERR_VALIDATION, "gguf: tensor %llu of %zu", (unsigned long long)i, g->tensors.size());
    fill(g, g->tensors[i], out);
    return SGQ_OK;
}

int sgq_gguf_tensor_find(const sgq_gguf *g, const char *name, sgq_gguf_tensor *out) {
    if (!g || !name || !out) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    auto it = g->index.find(name);
    if (it == g->index.end()) return fail(SGQ_ERR_VALIDATION, "gguf: no tensor '%s'", name);
    fill(g, g->tensors[it->second], out);
    return SGQ_OK;
}

int sgq_gguf_meta_int(const sgq_gguf *g, const char *key, int64_t *out) {
    if (!g || !key || !out) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    auto it = g->meta.find(key);
    if (it == g->meta.end()) return fail(SGQ_ERR_VALIDATION, "gguf: no metadata '%s'", key);
    const uint32_t t = it->second.type;
    if (t == 6 || t == 8 || t == 9 || t == 12)
        return fail(SGQ_ERR_VALIDATION, "gguf: metadata '%s' is not an integer", key);
    *out = (t == 0 || t == 2 || t == 4 || t == 7 || t == 10) ? (int64_t)it->second.u : it->second.i;
    return SGQ_OK;
}

int sgq_gguf_meta_float(const sgq_gguf *g, const char *key, double *out) {
    if (!g || !key || !out) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    auto it = g->meta.find(key);
    if (it == g->meta.end()) return fail(SGQ_ERR_VALIDATION, "gguf: no metadata '%s'", key);
    if (it->second.type != 6 && it->second.type != 12)
        return fail(SGQ_ERR_VALIDATION, "gguf: metadata '%s' is not a float", key);
    *out = it->second.f;
    return SGQ_OK;
}

int sgq_gguf_meta_string(const sgq_gguf *g, const char *key, const char **out) {
    if (!g || !key || !out) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    auto it = g->meta.find(key);
    if (it == g->meta.end()) return fail(SGQ_ERR_VALIDATION, "gguf: no metadata '%s'", key);
    if (it->second.type != 8) return fail(SGQ_ERR_VALIDATION, "gguf: metadata '%s' is not a string", key);
    *out = it->second.s.c_str();
    return SGQ_OK;
}

}  // extern "C"
