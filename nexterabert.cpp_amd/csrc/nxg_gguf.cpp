// nxg_gguf.cpp -- GGUF model files: reader of the published container format (versions 2
// and 3) and the int8 load of one tensor. Host code only.
//
// File layout read here (little-endian):
//   "GGUF" | u32 version | u64 n_tensors | u64 n_kv
//   n_kv x { string key | u32 value type | value }
//        string = u64 length + bytes; array = u32 element type + u64 count + elements
//   n_tensors x { string name | u32 n_dims | u64 ne[n_dims] | u32 ggml type | u64 offset }
//   padding to `general.alignment` (u32 metadata, default 32), then the tensor data;
//   a tensor's bytes start at data_offset + offset.

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "nxg_gguf.h"
#include "nxg_internal.h"

namespace {

struct value {
    int32_t type = -1;
    int64_t i = 0;             // integer and bool scalars
    double f = 0.0;            // float scalars
    std::string s;             // strings
    int32_t arr_type = -1;     // arrays: element type, count, elements by kind
    uint64_t arr_n = 0;
    std::vector<int64_t> ai;
    std::vector<double> af;
    std::vector<std::string> as;
};

struct tensor {
    std::string name;
    int32_t type = 0;
    int32_t n_dims = 0;
    int64_t ne[4] = { 1, 1, 1, 1 };
    uint64_t offset = 0;
    uint64_t nbytes = 0;
};

int fail(int code, const char * fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char * fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    nxg_set_error(buf);
    return code;
}

bool is_int_type(int32_t t) {
    return t == NXG_GGUF_UINT8 || t == NXG_GGUF_INT8 || t == NXG_GGUF_UINT16 || t == NXG_GGUF_INT16
        || t == NXG_GGUF_UINT32 || t == NXG_GGUF_INT32 || t == NXG_GGUF_UINT64 || t == NXG_GGUF_INT64
        || t == NXG_GGUF_BOOL;
}

bool is_float_type(int32_t t) { return t == NXG_GGUF_FLOAT32 || t == NXG_GGUF_FLOAT64; }

// Bounds-checked little-endian reads over the mapped file.
struct cursor {
    const uint8_t * p;
    uint64_t size, pos = 0;
    bool ok = true;

    bool take(void * dst, uint64_t n) {
        if (!ok || n > size - pos) {
            ok = false;
            return false;
        }
        std::memcpy(dst, p + pos, n);
        pos += n;
        return true;
    }
    template <typename T> T get() {
        T v{};
        take(&v, sizeof(T));
        return v;
    }
    bool string(std::string & s) {
        const uint64_t n = get<uint64_t>();
        if (!ok || n > size - pos) {
            ok = false;
            return false;
        }
        s.assign(reinterpret_cast<const char *>(p + pos), n);
        pos += n;
        return true;
    }
};

// One scalar of type t into v (as integer or float).
bool read_scalar(cursor & c, int32_t t, int64_t & i, double & f) {
    switch (t) {
        case NXG_GGUF_UINT8:   i = c.get<uint8_t>();  break;
        case NXG_GGUF_INT8:    i = c.get<int8_t>();   break;
        case NXG_GGUF_UINT16:  i = c.get<uint16_t>(); break;
        case NXG_GGUF_INT16:   i = c.get<int16_t>();  break;
        case NXG_GGUF_UINT32:  i = c.get<uint32_t>(); break;
        case NXG_GGUF_INT32:   i = c.get<int32_t>();  break;
        case NXG_GGUF_UINT64:  i = (int64_t) c.get<uint64_t>(); break;
        case NXG_GGUF_INT64:   i = c.get<int64_t>();  break;
        case NXG_GGUF_BOOL:    i = c.get<uint8_t>() != 0; break;
        case NXG_GGUF_FLOAT32: f = c.get<float>();    break;
        case NXG_GGUF_FLOAT64: f = c.get<double>();   break;
        default: return false;
    }
    if (is_int_type(t)) f = (double) i;
    else i = (int64_t) f;
    return c.ok;
}

} // namespace

struct nxg_gguf {
    void * map = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint32_t alignment = 32;
    uint64_t data_offset = 0;
    std::vector<std::string> keys;
    std::vector<value> values;
    std::unordered_map<std::string, int64_t> key_index;
    std::vector<tensor> tensors;
    std::unordered_map<std::string, int64_t> tensor_index;

    ~nxg_gguf() {
        if (map && map != MAP_FAILED) munmap(map, size);
    }
};

namespace {

int parse(nxg_gguf & g, const char * path) {
    cursor c{ static_cast<const uint8_t *>(g.map), g.size };
    char magic[4];
    if (!c.take(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0) return fail(NXG_EINVAL, "gguf: '%s' is not a GGUF file", path);
    g.version = c.get<uint32_t>();
    if (!c.ok || (g.version != 2 && g.version != 3)) {
        return fail(NXG_EINVAL, "gguf: '%s': unsupported GGUF version %u (2 and 3 are read)", path, g.version);
    }
    const uint64_t n_tensors = c.get<uint64_t>();
    const uint64_t n_kv = c.get<uint64_t>();
    if (!c.ok) return fail(NXG_EINVAL, "gguf: '%s': truncated header", path);
    // every key/value takes at least 12 bytes and every tensor record at least 24
    if (n_kv > g.size / 12 || n_tensors > g.size / 24) return fail(NXG_EINVAL, "gguf: '%s': implausible counts", path);

    g.keys.reserve(n_kv);
    g.values.reserve(n_kv);
    for (uint64_t k = 0; k < n_kv; ++k) {
        std::string key;
        value v;
        if (!c.string(key)) return fail(NXG_EINVAL, "gguf: '%s': truncated metadata (key %llu)", path, (unsigned long long) k);
        v.type = (int32_t) c.get<uint32_t>();
        if (!c.ok) return fail(NXG_EINVAL, "gguf: '%s': truncated metadata at '%s'", path, key.c_str());
        if (v.type == NXG_GGUF_STRING) {
            c.string(v.s);
        } else if (v.type == NXG_GGUF_ARRAY) {
            v.arr_type = (int32_t) c.get<uint32_t>();
            v.arr_n = c.get<uint64_t>();
            if (!c.ok) return fail(NXG_EINVAL, "gguf: '%s': truncated array '%s'", path, key.c_str());
            if (v.arr_n > c.size - c.pos) return fail(NXG_EINVAL, "gguf: '%s': array '%s' runs past the end", path, key.c_str());
            if (v.arr_type == NXG_GGUF_STRING) {
                v.as.resize(v.arr_n);
                for (uint64_t j = 0; j < v.arr_n && c.ok; ++j) c.string(v.as[j]);
            } else if (is_int_type(v.arr_type) || is_float_type(v.arr_type)) {
                v.ai.resize(v.arr_n);
                v.af.resize(v.arr_n);
                for (uint64_t j = 0; j < v.arr_n && c.ok; ++j) read_scalar(c, v.arr_type, v.ai[j], v.af[j]);
            } else {
                return fail(NXG_EINVAL, "gguf: '%s': array '%s' of element type %d is not supported", path, key.c_str(), v.arr_type);
            }
        } else if (!read_scalar(c, v.type, v.i, v.f)) {
            if (c.ok) return fail(NXG_EINVAL, "gguf: '%s': key '%s' has unknown value type %d", path, key.c_str(), v.type);
        }
        if (!c.ok) return fail(NXG_EINVAL, "gguf: '%s': truncated value of '%s'", path, key.c_str());
        if (!g.key_index.emplace(key, (int64_t) g.keys.size()).second) {
            return fail(NXG_EINVAL, "gguf: '%s': duplicate key '%s'", path, key.c_str());
        }
        g.keys.push_back(std::move(key));
        g.values.push_back(std::move(v));
    }

    auto al = g.key_index.find("general.alignment");
    if (al != g.key_index.end()) {
        const value & v = g.values[al->second];
        if (v.type != NXG_GGUF_UINT32 || v.i <= 0 || (v.i & (v.i - 1)) != 0) {
            return fail(NXG_EINVAL, "gguf: '%s': general.alignment must be a power-of-two u32", path);
        }
        g.alignment = (uint32_t) v.i;
    }

    g.tensors.resize(n_tensors);
    for (uint64_t t = 0; t < n_tensors; ++t) {
        tensor & T = g.tensors[t];
        if (!c.string(T.name)) return fail(NXG_EINVAL, "gguf: '%s': truncated tensor table (tensor %llu)", path, (unsigned long long) t);
        const uint32_t nd = c.get<uint32_t>();
        if (!c.ok || nd < 1 || nd > 4) return fail(NXG_EINVAL, "gguf: '%s': tensor '%s' has %u dimensions", path, T.name.c_str(), nd);
        T.n_dims = (int32_t) nd;
        for (uint32_t d = 0; d < nd; ++d) {
            const uint64_t n = c.get<uint64_t>();
            if (!c.ok) return fail(NXG_EINVAL, "gguf: '%s': truncated tensor table at '%s'", path, T.name.c_str());
            if (n == 0 || n > (uint64_t) INT64_MAX / 2) return fail(NXG_EINVAL, "gguf: '%s': tensor '%s' has a bad dimension", path, T.name.c_str());
            T.ne[d] = (int64_t) n;
        }
        T.type = (int32_t) c.get<uint32_t>();
        T.offset = c.get<uint64_t>();
        if (!c.ok) return fail(NXG_EINVAL, "gguf: '%s': truncated tensor table at '%s'", path, T.name.c_str());
        const size_t row = nxg_row_bytes(T.type, T.ne[0]);
        if (row == 0) {
            return fail(NXG_EINVAL, "gguf: '%s': tensor '%s' has unsupported type %d or a row length %lld its blocks do not divide",
                        path, T.name.c_str(), T.type, (long long) T.ne[0]);
        }
        const long double rows = (long double) T.ne[1] * T.ne[2] * T.ne[3];
        if (rows * row > (long double) g.size) return fail(NXG_EINVAL, "gguf: '%s': tensor '%s' is larger than the file", path, T.name.c_str());
        T.nbytes = (uint64_t) row * (uint64_t) (T.ne[1] * T.ne[2] * T.ne[3]);
        if (T.offset % g.alignment != 0) {
            return fail(NXG_EINVAL, "gguf: '%s': tensor '%s' offset %llu is not a multiple of the alignment %u",
                        path, T.name.c_str(), (unsigned long long) T.offset, g.alignment);
        }
        if (!g.tensor_index.emplace(T.name, (int64_t) t).second) {
            return fail(NXG_EINVAL, "gguf: '%s': duplicate tensor '%s'", path, T.name.c_str());
        }
    }
    g.data_offset = (c.pos + g.alignment - 1) / g.alignment * g.alignment;
    for (const tensor & T : g.tensors) {
        if (T.offset > g.size || g.data_offset > g.size - T.offset || T.nbytes > g.size - g.data_offset - T.offset) {
            return fail(NXG_EINVAL, "gguf: '%s': tensor '%s' (%llu bytes at %llu) runs past the end of the file",
                        path, T.name.c_str(), (unsigned long long) T.nbytes, (unsigned long long) (g.data_offset + T.offset));
        }
    }
    return NXG_OK;
}

const value * kv_at(const nxg_gguf * g, int64_t i) {
    if (!g || i < 0 || i >= (int64_t) g->values.size()) {
        fail(NXG_EINVAL, "gguf: metadata index %lld out of range", (long long) i);
        return nullptr;
    }
    return &g->values[i];
}

const tensor * tensor_at(const nxg_gguf * g, int64_t i) {
    if (!g || i < 0 || i >= (int64_t) g->tensors.size()) {
        fail(NXG_EINVAL, "gguf: tensor index %lld out of range", (long long) i);
        return nullptr;
    }
    return &g->tensors[i];
}

} // namespace

extern "C" {

int32_t nxg_gguf_open(const char * path, nxg_gguf ** out) {
    if (!out) return fail(NXG_EINVAL, "gguf_open: null out");
    *out = nullptr;
    if (!path) return fail(NXG_EINVAL, "gguf_open: null path");
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(NXG_EINVAL, "gguf: cannot open '%s': %s", path, std::strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        return fail(NXG_EINVAL, "gguf: '%s' is not a GGUF file (too short)", path);
    }
    nxg_gguf * g = new (std::nothrow) nxg_gguf();
    if (!g) {
        close(fd);
        return fail(NXG_ENOMEM, "gguf_open: out of memory");
    }
    g->size = (uint64_t) st.st_size;
    g->map = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (g->map == MAP_FAILED) {
        g->map = nullptr;
        delete g;
        return fail(NXG_ENOMEM, "gguf: cannot map '%s': %s", path, std::strerror(errno));
    }
    int rc;
    try {
        rc = parse(*g, path);
    } catch (const std::bad_alloc &) {
        rc = fail(NXG_ENOMEM, "gguf: '%s': out of memory while reading the metadata", path);
    }
    if (rc != NXG_OK) {
        delete g;
        return rc;
    }
    *out = g;
    return NXG_OK;
}

void nxg_gguf_close(nxg_gguf * g) { delete g; }

uint32_t nxg_gguf_version(const nxg_gguf * g) { return g ? g->version : 0; }
uint64_t nxg_gguf_data_offset(const nxg_gguf * g) { return g ? g->data_offset : 0; }
uint32_t nxg_gguf_alignment(const nxg_gguf * g) { return g ? g->alignment : 0; }

int64_t nxg_gguf_n_kv(const nxg_gguf * g) { return g ? (int64_t) g->keys.size() : 0; }

int64_t nxg_gguf_find_key(const nxg_gguf * g, const char * key) {
    if (!g || !key) return -1;
    auto it = g->key_index.find(key);
    return it == g->key_index.end() ? -1 : it->second;
}

const char * nxg_gguf_key(const nxg_gguf * g, int64_t i) {
    return kv_at(g, i) ? g->keys[i].c_str() : nullptr;
}

int32_t nxg_gguf_kv_type(const nxg_gguf * g, int64_t i) {
    const value * v = kv_at(g, i);
    return v ? v->type : -1;
}

int32_t nxg_gguf_get_i64(const nxg_gguf * g, int64_t i, int64_t * out) {
    const value * v = kv_at(g, i);
    if (!v) return NXG_EINVAL;
    if (!out || !(is_int_type(v->type) || is_float_type(v->type))) {
        return fail(NXG_EINVAL, "gguf: '%s' is not a number", g->keys[i].c_str());
    }
    *out = v->i;
    return NXG_OK;
}

int32_t nxg_gguf_get_f64(const nxg_gguf * g, int64_t i, double * out) {
    const value * v = kv_at(g, i);
    if (!v) return NXG_EINVAL;
    if (!out || !(is_int_type(v->type) || is_float_type(v->type))) {
        return fail(NXG_EINVAL, "gguf: '%s' is not a number", g->keys[i].c_str());
    }
    *out = v->f;
    return NXG_OK;
}

int32_t nxg_gguf_get_str(const nxg_gguf * g, int64_t i, const char ** s, uint64_t * len) {
    const value * v = kv_at(g, i);
    if (!v) return NXG_EINVAL;
    if (!s || v->type != NXG_GGUF_STRING) return fail(NXG_EINVAL, "gguf: '%s' is not a string", g->keys[i].c_str());
    *s = v->s.c_str();
    if (len) *len = v->s.size();
    return NXG_OK;
}

int32_t nxg_gguf_arr_info(const nxg_gguf * g, int64_t i, int32_t * elem_type, uint64_t * n) {
    const value * v = kv_at(g, i);
    if (!v) return NXG_EINVAL;
    if (v->type != NXG_GGUF_ARRAY) return fail(NXG_EINVAL, "gguf: '%s' is not an array", g->keys[i].c_str());
    if (elem_type) *elem_type = v->arr_type;
    if (n) *n = v->arr_n;
    return NXG_OK;
}

static const value * arr_elem(const nxg_gguf * g, int64_t i, uint64_t j, bool want_str) {
    const value * v = kv_at(g, i);
    if (!v) return nullptr;
    if (v->type != NXG_GGUF_ARRAY || (want_str != (v->arr_type == NXG_GGUF_STRING))) {
        fail(NXG_EINVAL, "gguf: '%s' is not an array of %s", g->keys[i].c_str(), want_str ? "strings" : "numbers");
        return nullptr;
    }
    if (j >= v->arr_n) {
        fail(NXG_EINVAL, "gguf: '%s' has %llu elements, asked for %llu", g->keys[i].c_str(),
             (unsigned long long) v->arr_n, (unsigned long long) j);
        return nullptr;
    }
    return v;
}

int32_t nxg_gguf_arr_i64(const nxg_gguf * g, int64_t i, uint64_t j, int64_t * out) {
    const value * v = arr_elem(g, i, j, false);
    if (!v || !out) return NXG_EINVAL;
    *out = v->ai[j];
    return NXG_OK;
}

int32_t nxg_gguf_arr_f64(const nxg_gguf * g, int64_t i, uint64_t j, double * out) {
    const value * v = arr_elem(g, i, j, false);
    if (!v || !out) return NXG_EINVAL;
    *out = v->af[j];
    return NXG_OK;
}

int32_t nxg_gguf_arr_str(const nxg_gguf * g, int64_t i, uint64_t j, const char ** s, uint64_t * len) {
    const value * v = arr_elem(g, i, j, true);
    if (!v || !s) return NXG_EINVAL;
    *s = v->as[j].c_str();
    if (len) *len = v->as[j].size();
    return NXG_OK;
}

int64_t nxg_gguf_n_tensors(const nxg_gguf * g) { return g ? (int64_t) g->tensors.size() : 0; }

int64_t nxg_gguf_find_tensor(const nxg_gguf * g, const char * name) {
    if (!g || !name) return -1;
    auto it = g->tensor_index.find(name);
    return it == g->tensor_index.end() ? -1 : it->second;
}

const char * nxg_gguf_tensor_name(const nxg_gguf * g, int64_t i) {
    const tensor * t = tensor_at(g, i);
    return t ? t->name.c_str() : nullptr;
}

int32_t nxg_gguf_tensor_info(const nxg_gguf * g, int64_t i, int32_t * type, int32_t * n_dims,
                             int64_t * ne, uint64_t * offset, uint64_t * nbytes) {
    const tensor * t = tensor_at(g, i);
    if (!t) return NXG_EINVAL;
    if (type) *type = t->type;
    if (n_dims) *n_dims = t->n_dims;
    if (ne) for (int d = 0; d < 4; ++d) ne[d] = t->ne[d];
    if (offset) *offset = t->offset;
    if (nbytes) *nbytes = t->nbytes;
    return NXG_OK;
}

const void * nxg_gguf_tensor_data(const nxg_gguf * g, int64_t i) {
    const tensor * t = tensor_at(g, i);
    return t ? static_cast<const uint8_t *>(g->map) + g->data_offset + t->offset : nullptr;
}

int32_t nxg_gguf_weight_create(const nxg_gguf * g, int64_t i, int32_t n_threads, nxg_weight ** out) {
    if (!out) return fail(NXG_EINVAL, "gguf_weight_create: null out");
    *out = nullptr;
    const tensor * t = tensor_at(g, i);
    if (!t) return NXG_EINVAL;
    if (!nxg_weight_is_int8(t->name.c_str(), t->n_dims, t->type, t->ne[0], t->ne[1], 1)) {
        return fail(NXG_EINVAL, "gguf_weight_create: '%s' is not an int8 linear weight (type %d, %d dims, %lld x %lld)",
                    t->name.c_str(), t->type, t->n_dims, (long long) t->ne[0], (long long) t->ne[1]);
    }
    if (t->ne[0] > INT32_MAX || t->ne[1] > INT32_MAX) return fail(NXG_EINVAL, "gguf_weight_create: '%s' too large", t->name.c_str());
    const int n_in = (int) t->ne[0], n_out = (int) t->ne[1];
    const int n_blk = (n_in + NXG_BLOCK - 1) / NXG_BLOCK;
    std::vector<int8_t> w;
    std::vector<float> scale;
    try {
        w.resize((size_t) n_in * n_out);
        scale.resize((size_t) n_blk * n_out);
    } catch (const std::bad_alloc &) {
        return fail(NXG_ENOMEM, "gguf_weight_create: '%s': out of host memory", t->name.c_str());
    }
    int32_t rc = nxg_expand_weight(t->type, nxg_gguf_tensor_data(g, i), n_in, n_out, 128, n_threads,
                                   w.data(), scale.data(), nullptr);
    if (rc != NXG_OK) return rc;
    return nxg_weight_create(w.data(), scale.data(), n_in, n_out, out);
}

} // extern "C"
