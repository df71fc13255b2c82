// dq_gguf.cpp - GGUF model files on the host: header, metadata and tensor
// directory parsed from a read-only memory map, tensor bytes handed out as
// pointers into the map, and the upload of a quantized matrix into the
// device layout (cuda_upload_weights).
//
// Follows the engine's GgufReader (src/gguf/gguf_reader.cpp:100-300):
//  * magic "GGUF", u32 version, u64 tensor count, u64 key/value count;
//  * key: u64 length + bytes; value: u32 type + payload (types 0-12 below;
//    8 = string, 9 = array of u32 element type + u64 count + elements);
//  * tensor info: name, u32 n_dims, u64 dims[n_dims], u32 type, u64 offset;
//  * data section: for version >= 2 the offsets are relative to the end of
//    the tensor infos rounded up to `general.alignment` (a power of two,
//    default 32); for version < 2 they are absolute file offsets, as the
//    reader computes it (gguf_reader.cpp:273-283);
//  * a tensor's bytes: row_size(type, ne0) * prod(dims[1..]) (read_tensor_raw,
//    gguf_reader.cpp:288-305), with row_size of quant/quant.cpp:839-910.
// Every read is bounds-checked against the file size: a truncated header or
// directory is DQ_ERR_INVALID_ARG, a tensor whose bytes run past the end has
// no bytes (its read is NOT_SUPPORTED); nothing reads past the map.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/desireeia_hip.h"

namespace {

constexpr uint32_t GGUF_MAGIC = 0x46554747u;  // "GGUF" little-endian
constexpr uint32_t MAX_DIMS = 8;

struct Kv {
    std::string key;
    uint32_t type = 0;
    uint64_t u = 0;          // unsigned/bool scalars, and integer view of signed ones
    int64_t i = 0;           // signed view
    double f = 0.0;          // float scalars
    const char* str = nullptr;  // string payload (in the map)
    uint64_t len = 0;        // string length / array count
    uint32_t elem = 0;       // array element type
    const uint8_t* data = nullptr;  // array payload (in the map)
};

struct Tensor {
    std::string name;
    uint32_t type = 0;
    uint32_t n_dims = 0;
    uint64_t dims[MAX_DIMS] = {1, 1, 1, 1, 1, 1, 1, 1};
    uint64_t offset = 0;  // absolute, in the file
    uint64_t nbytes = 0;
};

// Element size of a scalar metadata type (0 for string/array/unknown).
size_t scalar_size(uint32_t t) {
    switch (t) {
    case 0: case 1: case 7: return 1;   // U8, I8, BOOL
    case 2: case 3: return 2;           // U16, I16
    case 4: case 5: case 6: return 4;   // U32, I32, F32
    case 10: case 11: case 12: return 8;  // U64, I64, F64
    default: return 0;
    }
}

struct Cursor {
    const uint8_t* p;
    const uint8_t* end;
    bool take(void* dst, size_t n) {
        if ((size_t)(end - p) < n) return false;
        std::memcpy(dst, p, n);
        p += n;
        return true;
    }
    bool skip(uint64_t n) {
        if ((uint64_t)(end - p) < n) return false;
        p += n;
        return true;
    }
    template <typename T>
    bool get(T& v) { return take(&v, sizeof(T)); }
    bool str(const char** s, uint64_t* len) {
        if (!get(*len)) return false;
        *s = reinterpret_cast<const char*>(p);
        return skip(*len);
    }
};

// Skips one value of type t (arrays recursively).
bool skip_value(Cursor& c, uint32_t t, int depth = 0) {
    const size_t sz = scalar_size(t);
    if (sz) return c.skip(sz);
    if (t == 8) {
        uint64_t len = 0;
        return c.get(len) && c.skip(len);
    }
    if (t == 9 && depth < 4) {
        uint32_t elem = 0;
        uint64_t n = 0;
        if (!c.get(elem) || !c.get(n)) return false;
        const size_t es = scalar_size(elem);
        if (es) {
            if (n > (uint64_t)(c.end - c.p) / es) return false;
            return c.skip(n * es);
        }
        for (uint64_t a = 0; a < n; ++a)
            if (!skip_value(c, elem, depth + 1)) return false;
        return true;
    }
    return false;
}

}  // namespace

struct dq_gguf {
    int fd = -1;
    const uint8_t* map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t data_start = 0;
    uint64_t alignment = 32;
    std::vector<Kv> kv;
    std::unordered_map<std::string, size_t> kv_index;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> tensor_index;

    ~dq_gguf() {
        if (map) munmap(const_cast<uint8_t*>(map), size);
        if (fd >= 0) close(fd);
    }

    bool parse() {
        Cursor c{map, map + size};
        uint32_t magic = 0;
        uint64_t n_tensors = 0, n_kv = 0;
        if (!c.get(magic) || magic != GGUF_MAGIC) return false;
        if (!c.get(version) || !c.get(n_tensors) || !c.get(n_kv)) return false;
        // every entry needs at least a few bytes: counts beyond the file are malformed
        if (n_kv > size / 12 || n_tensors > size / 24) return false;
        kv.reserve((size_t)n_kv);
        for (uint64_t k = 0; k < n_kv; ++k) {
            Kv e;
            const char* key = nullptr;
            uint64_t klen = 0;
            if (!c.str(&key, &klen) || !c.get(e.type)) return false;
            e.key.assign(key, (size_t)klen);
            switch (e.type) {
            case 0: { uint8_t v; if (!c.get(v)) return false; e.u = v; e.i = v; e.f = v; break; }
            case 1: { int8_t v; if (!c.get(v)) return false; e.i = v; e.u = (uint64_t)(int64_t)v; e.f = v; break; }
            case 2: { uint16_t v; if (!c.get(v)) return false; e.u = v; e.i = v; e.f = v; break; }
            case 3: { int16_t v; if (!c.get(v)) return false; e.i = v; e.u = (uint64_t)(int64_t)v; e.f = v; break; }
            case 4: { uint32_t v; if (!c.get(v)) return false; e.u = v; e.i = v; e.f = v; break; }
            case 5: { int32_t v; if (!c.get(v)) return false; e.i = v; e.u = (uint64_t)(int64_t)v; e.f = v; break; }
            case 6: { float v; if (!c.get(v)) return false; e.f = v; e.i = (int64_t)v; e.u = (uint64_t)e.i; break; }
            case 7: { uint8_t v; if (!c.get(v)) return false; e.u = v; e.i = v; e.f = v; break; }
            case 10: { uint64_t v; if (!c.get(v)) return false; e.u = v; e.i = (int64_t)v; e.f = (double)v; break; }
            case 11: { int64_t v; if (!c.get(v)) return false; e.i = v; e.u = (uint64_t)v; e.f = (double)v; break; }
            case 12: { double v; if (!c.get(v)) return false; e.f = v; e.i = (int64_t)v; e.u = (uint64_t)e.i; break; }
            case 8:
                if (!c.str(&e.str, &e.len)) return false;
                break;
            case 9: {
                if (!c.get(e.elem) || !c.get(e.len)) return false;
                e.data = c.p;
                const size_t es = scalar_size(e.elem);
                if (es) {
                    if (e.len > (uint64_t)(c.end - c.p) / es || !c.skip(e.len * es)) return false;
                } else {
                    for (uint64_t a = 0; a < e.len; ++a)
                        if (!skip_value(c, e.elem, 1)) return false;
                }
                break;
            }
            default:
                return false;  // unknown value type: the rest cannot be parsed
            }
            kv_index[e.key] = kv.size();
            kv.push_back(std::move(e));
        }
        tensors.reserve((size_t)n_tensors);
        for (uint64_t t = 0; t < n_tensors; ++t) {
            Tensor e;
            const char* name = nullptr;
            uint64_t nlen = 0;
            if (!c.str(&name, &nlen) || !c.get(e.n_dims)) return false;
            // no dims: the tensor is listed but has no bytes (its read fails, as
            // gguf_reader.cpp:292 does)
            if (e.n_dims > MAX_DIMS) return false;
            e.name.assign(name, (size_t)nlen);
            for (uint32_t d = 0; d < e.n_dims; ++d)
                if (!c.get(e.dims[d])) return false;
            if (!c.get(e.type) || !c.get(e.offset)) return false;
            tensors.push_back(std::move(e));
        }
        auto al = kv_index.find("general.alignment");
        if (al != kv_index.end()) {
            const uint64_t a = kv[al->second].u;
            const uint32_t ty = kv[al->second].type;
            // the integer kinds the engine keeps (gguf_reader.cpp:224-250, 276-281)
            if ((ty == 4 || ty == 5 || ty == 7 || ty == 10 || ty == 11) && a > 0 && (a & (a - 1)) == 0) alignment = a;
        }
        const uint64_t pos = (uint64_t)(c.p - map);
        data_start = version >= 2 ? (pos + alignment - 1) / alignment * alignment : 0;
        for (size_t t = 0; t < tensors.size(); ++t) {
            Tensor& e = tensors[t];
            uint64_t rows = 1;
            for (uint32_t d = 1; d < e.n_dims; ++d) {
                if (e.dims[d] && rows > UINT64_MAX / e.dims[d]) return false;
                rows *= e.dims[d];
            }
            const size_t rb = e.n_dims ? dq_row_size((int)e.type, (int64_t)e.dims[0]) : 0;
            e.offset += data_start;
            // unknown types have no size: their bytes cannot be handed out
            e.nbytes = rb && rows <= UINT64_MAX / rb ? (uint64_t)rb * rows : 0;
            // bytes past the end of the file: the tensor is listed but cannot be
            // read (the engine's open succeeds and that read fails)
            if (e.nbytes && (e.offset > size || e.nbytes > size - e.offset)) e.nbytes = 0;
            tensor_index[e.name] = t;
        }
        return true;
    }
};

namespace {
const Kv* find_kv(const dq_gguf* g, const char* key) {
    if (!g || !key) return nullptr;
    auto it = g->kv_index.find(key);
    return it == g->kv_index.end() ? nullptr : &g->kv[it->second];
}
bool is_int_type(uint32_t t) { return t <= 5 || t == 7 || t == 10 || t == 11; }

// Block size and block bytes of a GGUF tensor type (quant/quant.h:24-265,
// quant.cpp:839-903). 0 bytes: unknown.
void type_traits(int type, int* blck, size_t* bytes) {
    *blck = 1;
    *bytes = 0;
    switch (type) {
    case 0: *bytes = 4; return;                  // F32
    case 1: case 30: case 25: *bytes = 2; return;  // F16, BF16, I16
    case 24: *bytes = 1; return;                 // I8
    case 26: *bytes = 4; return;                 // I32
    case 27: case 28: *bytes = 8; return;        // I64, F64
    case 2: *blck = 32; *bytes = 18; return;     // Q4_0
    case 3: *blck = 32; *bytes = 20; return;     // Q4_1
    case 6: *blck = 32; *bytes = 22; return;     // Q5_0
    case 7: *blck = 32; *bytes = 24; return;     // Q5_1
    case 8: *blck = 32; *bytes = 34; return;     // Q8_0
    case 9: *blck = 32; *bytes = 36; return;     // Q8_1
    case 20: *blck = 32; *bytes = 18; return;    // IQ4_NL
    case 39: *blck = 32; *bytes = 17; return;    // MXFP4
    case 40: *blck = 64; *bytes = 36; return;    // NVFP4
    case 41: *blck = 128; *bytes = 18; return;   // Q1_0
    case 42: *blck = 64; *bytes = 18; return;    // Q2_0
    case 10: *blck = 256; *bytes = 84; return;   // Q2_K
    case 11: *blck = 256; *bytes = 110; return;  // Q3_K
    case 12: *blck = 256; *bytes = 144; return;  // Q4_K
    case 13: *blck = 256; *bytes = 176; return;  // Q5_K
    case 14: *blck = 256; *bytes = 210; return;  // Q6_K
    case 15: *blck = 256; *bytes = 292; return;  // Q8_K
    case 16: *blck = 256; *bytes = 66; return;   // IQ2_XXS
    case 17: *blck = 256; *bytes = 74; return;   // IQ2_XS
    case 18: *blck = 256; *bytes = 98; return;   // IQ3_XXS
    case 19: *blck = 256; *bytes = 50; return;   // IQ1_S
    case 21: *blck = 256; *bytes = 110; return;  // IQ3_S
    case 22: *blck = 256; *bytes = 82; return;   // IQ2_S
    case 23: *blck = 256; *bytes = 136; return;  // IQ4_XS
    case 29: *blck = 256; *bytes = 56; return;   // IQ1_M
    case 34: *blck = 256; *bytes = 54; return;   // TQ1_0
    case 35: *blck = 256; *bytes = 66; return;   // TQ2_0
    default: return;
    }
}
}  // namespace

extern "C" size_t dq_row_size(int type, int64_t ne0) {
    int blck = 1;
    size_t bytes = 0;
    type_traits(type, &blck, &bytes);
    if (!bytes || ne0 < 0) return 0;
    const int64_t nb = ne0 / blck + (ne0 % blck ? 1 : 0);
    return (size_t)nb * bytes;
}

extern "C" int dq_gguf_open(const char* path, dq_gguf** out) {
    if (!path || !out) return DQ_ERR_INVALID_ARG;
    *out = nullptr;
    auto* g = new dq_gguf();
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    struct stat st;
    if (g->fd < 0 || fstat(g->fd, &st) != 0 || st.st_size <= 0) {
        delete g;
        return DQ_ERR_IO;
    }
    g->size = (size_t)st.st_size;
    void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        g->map = nullptr;
        delete g;
        return DQ_ERR_IO;
    }
    g->map = static_cast<const uint8_t*>(m);
    if (!g->parse()) {
        delete g;
        return DQ_ERR_INVALID_ARG;
    }
    *out = g;
    return DQ_OK;
}

extern "C" void dq_gguf_close(dq_gguf* g) { delete g; }

extern "C" int dq_gguf_version(const dq_gguf* g) { return g ? (int)g->version : -1; }

extern "C" uint64_t dq_gguf_data_offset(const dq_gguf* g) { return g ? g->data_start : 0; }

extern "C" int64_t dq_gguf_kv_count(const dq_gguf* g) { return g ? (int64_t)g->kv.size() : -1; }

extern "C" const char* dq_gguf_kv_key(const dq_gguf* g, int64_t i) {
    return g && i >= 0 && (size_t)i < g->kv.size() ? g->kv[(size_t)i].key.c_str() : nullptr;
}

extern "C" int dq_gguf_kv_type(const dq_gguf* g, const char* key) {
    const Kv* e = find_kv(g, key);
    return e ? (int)e->type : -1;
}

extern "C" int dq_gguf_get_int(const dq_gguf* g, const char* key, int64_t* v) {
    const Kv* e = find_kv(g, key);
    if (!e || !v) return e ? DQ_ERR_INVALID_ARG : DQ_ERR_NOT_SUPPORTED;
    if (!is_int_type(e->type)) return DQ_ERR_NOT_SUPPORTED;
    *v = e->i;
    return DQ_OK;
}

extern "C" int dq_gguf_get_float(const dq_gguf* g, const char* key, double* v) {
    const Kv* e = find_kv(g, key);
    if (!e || !v) return e ? DQ_ERR_INVALID_ARG : DQ_ERR_NOT_SUPPORTED;
    if (e->type == 8 || e->type == 9) return DQ_ERR_NOT_SUPPORTED;
    *v = e->f;
    return DQ_OK;
}

extern "C" int dq_gguf_get_str(const dq_gguf* g, const char* key, const char** s, uint64_t* len) {
    const Kv* e = find_kv(g, key);
    if (!e || !s || !len) return e ? DQ_ERR_INVALID_ARG : DQ_ERR_NOT_SUPPORTED;
    if (e->type != 8) return DQ_ERR_NOT_SUPPORTED;
    *s = e->str;
    *len = e->len;
    return DQ_OK;
}

extern "C" int dq_gguf_get_array(const dq_gguf* g, const char* key, int* elem_type, uint64_t* n,
                                 const void** data) {
    const Kv* e = find_kv(g, key);
    if (!e || !elem_type || !n || !data) return e ? DQ_ERR_INVALID_ARG : DQ_ERR_NOT_SUPPORTED;
    if (e->type != 9) return DQ_ERR_NOT_SUPPORTED;
    *elem_type = (int)e->elem;
    *n = e->len;
    *data = e->data;
    return DQ_OK;
}

extern "C" int64_t dq_gguf_n_tensors(const dq_gguf* g) { return g ? (int64_t)g->tensors.size() : -1; }

extern "C" int64_t dq_gguf_find_tensor(const dq_gguf* g, const char* name) {
    if (!g || !name) return -1;
    auto it = g->tensor_index.find(name);
    return it == g->tensor_index.end() ? -1 : (int64_t)it->second;
}

extern "C" int dq_gguf_tensor_info(const dq_gguf* g, int64_t i, dq_gguf_tensor_t* out) {
    if (!g || !out || i < 0 || (size_t)i >= g->tensors.size()) return DQ_ERR_INVALID_ARG;
    const Tensor& t = g->tensors[(size_t)i];
    out->name = t.name.c_str();
    out->type = (int)t.type;
    out->n_dims = (int)t.n_dims;
    for (uint32_t d = 0; d < 4; ++d) out->dims[d] = d < t.n_dims ? t.dims[d] : 1;
    out->offset = t.offset;
    out->nbytes = t.nbytes;
    out->data = t.nbytes ? g->map + t.offset : nullptr;
    return DQ_OK;
}

extern "C" int dq_gguf_read_tensor_raw(const dq_gguf* g, const char* name, void* dst, size_t cap, int* type,
                                       uint64_t* ne0, uint64_t* rows) {
    const int64_t i = dq_gguf_find_tensor(g, name);
    if (i < 0) return DQ_ERR_NOT_SUPPORTED;
    const Tensor& t = g->tensors[(size_t)i];
    if (!t.nbytes) return DQ_ERR_NOT_SUPPORTED;  // a type without a known row size
    if (type) *type = (int)t.type;
    if (ne0) *ne0 = t.dims[0];
    if (rows) *rows = t.nbytes / dq_row_size((int)t.type, (int64_t)t.dims[0]);
    if (!dst) return DQ_OK;  // sizes only
    if (cap < t.nbytes) return DQ_ERR_INVALID_ARG;
    std::memcpy(dst, g->map + t.offset, t.nbytes);
    return DQ_OK;
}

// GGUF type id -> the backend's format id (core/engine.h:521-527), -1 if the
// device path has no kernels for it.
extern "C" int dq_fmt_of_gguf_type(int type) {
    switch (type) {
    case 8: return DQ_FMT_Q8_0;
    case 2: return DQ_FMT_Q4_0;
    case 12: return DQ_FMT_Q4_K;
    case 14: return DQ_FMT_Q6_K;
    default: return -1;
    }
}

extern "C" int dq_gguf_upload(const dq_gguf* g, const char* name, int* fmt, uint64_t* rows, uint64_t* cols,
                              void** d_qs, void** d_scale) {
    if (!fmt || !rows || !cols || !d_qs || !d_scale) return DQ_ERR_INVALID_ARG;
    *d_qs = *d_scale = nullptr;
    const int64_t i = dq_gguf_find_tensor(g, name);
    if (i < 0) return DQ_ERR_NOT_SUPPORTED;
    const Tensor& t = g->tensors[(size_t)i];
    const int f = dq_fmt_of_gguf_type((int)t.type);
    if (f < 0 || !t.nbytes) return DQ_ERR_NOT_SUPPORTED;
    const uint64_t r = t.nbytes / dq_row_size((int)t.type, (int64_t)t.dims[0]);
    if (!cuda_upload_weights(f, g->map + t.offset, (size_t)r, (size_t)t.dims[0], d_qs, d_scale))
        return DQ_ERR_NOT_SUPPORTED;
    *fmt = f;
    *rows = r;
    *cols = t.dims[0];
    return DQ_OK;
}
