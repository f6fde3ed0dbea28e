// gguf.hip -- GGUF v3 files (src/gguf/gguf.zig): the reader of the header,
// the metadata key/values and the tensor table, with the tensor data mapped
// read-only (gguf.zig:251-332 parse; the file layout of gguf.zig:8-12), and a
// writer that lays a file out the same way (gguf.zig:643-912, the fixture
// writers): header, key/values, tensor infos with offsets aligned to
// general.alignment, padding, then each tensor's bytes at its aligned offset.
// Host code only.  Malformed input fails with the reference's error names,
// bounded as it bounds them: at most 2^20 tensors and key/values, strings
// of at most 16 MB, arrays of at most 2^24 elements nested at most 4 deep,
// 1..8 nonzero dims whose product does not overflow, a power-of-two
// alignment, a data section inside the file.
#include "runtime.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <vector>

namespace lh {

constexpr uint32_t GGUF_MAGIC = 0x46554747; // "GGUF", little-endian
constexpr uint64_t GGUF_MAX_COUNT = 1ull << 20;
constexpr uint64_t GGUF_MAX_STR = 1ull << 24;
constexpr uint64_t GGUF_MAX_ARRAY = 1ull << 24;
constexpr uint32_t GGUF_MAX_DEPTH = 4;
constexpr size_t GGUF_HEAD_CAP = 64ull << 20; // the header region read (gguf.zig:254-256)

enum : uint32_t { V_U8, V_I8, V_U16, V_I16, V_U32, V_I32, V_F32, V_BOOL, V_STR, V_ARRAY, V_U64, V_I64, V_F64 };

struct Kv {
    std::string key;
    uint32_t type = 0;
    int kind = 0;
    int64_t i = 0;
    uint64_t u = 0;
    double f = 0;
    std::string s;
    uint32_t elem_type = 0;
    uint64_t count = 0;
    std::vector<std::string> strs;
    std::vector<const char *> str_ptrs;
    std::vector<float> f32s;
    std::vector<int32_t> i32s;
    uint64_t span_start = 0, span_end = 0;
};

struct Tensor {
    std::string name;
    uint32_t n_dims = 0;
    uint64_t dims[8] = {};
    uint32_t type = 0;
    uint64_t offset = 0;
};

// GGML bytes of a tensor: dims[0] values per row, the other dims' product
// rows; 0 for a type without a known block geometry, a row length that is
// not a whole number of blocks, or a size that overflows 64 bits (every
// product checked, as ggml.zig:143-153 tensorBytesChecked checks them: a
// wrapped size would pass the in-file test and let a reader walk past the
// mapping).
static uint64_t tensor_bytes(const Tensor &t) {
    const int T = (int)t.type;
    if (T != LH_F32 && T != LH_F16 && T != LH_Q4_0 && T != LH_Q8_0 && T != LH_Q4_K && T != LH_Q6_K)
        return 0;
    const uint64_t be = (uint64_t)block_elems(T), bb = (uint64_t)block_bytes(T);
    if (t.n_dims == 0 || t.dims[0] % be)
        return 0;
    uint64_t n = 0;
    if (__builtin_mul_overflow(t.dims[0] / be, bb, &n))
        return 0;
    for (uint32_t d = 1; d < t.n_dims; d++)
        if (__builtin_mul_overflow(n, t.dims[d], &n))
            return 0;
    return n;
}

struct Cursor {
    const uint8_t *buf;
    size_t len, pos = 0;
    const char *err = nullptr;
    const uint8_t *need(size_t n) {
        if (err || n > len - pos) {
            if (!err)
                err = "TruncatedGguf";
            return nullptr;
        }
        const uint8_t *p = buf + pos;
        pos += n;
        return p;
    }
    template <class T> T get() {
        T v{};
        if (const uint8_t *p = need(sizeof(T)))
            memcpy(&v, p, sizeof(T));
        return v;
    }
    bool str(std::string &out) {
        const uint64_t n = get<uint64_t>();
        if (err)
            return false;
        if (n > GGUF_MAX_STR) {
            err = "TruncatedGguf";
            return false;
        }
        const uint8_t *p = need((size_t)n);
        if (!p)
            return false;
        out.assign((const char *)p, (size_t)n);
        return true;
    }
};

// One value of type vt (gguf.zig:189-247 readValueDepth): scalars widen to
// i64 / u64 / f64; string, f32 and i32 arrays are kept; arrays of any other
// element type are walked and skipped.
static bool read_value(Cursor &c, uint32_t vt, Kv &kv, uint32_t depth) {
    if (depth > GGUF_MAX_DEPTH) {
        c.err = "ArrayNestingTooDeep";
        return false;
    }
    switch (vt) {
    case V_U8: kv.kind = 1; kv.u = c.get<uint8_t>(); break;
    case V_I8: kv.kind = 0; kv.i = c.get<int8_t>(); break;
    case V_U16: kv.kind = 1; kv.u = c.get<uint16_t>(); break;
    case V_I16: kv.kind = 0; kv.i = c.get<int16_t>(); break;
    case V_U32: kv.kind = 1; kv.u = c.get<uint32_t>(); break;
    case V_I32: kv.kind = 0; kv.i = c.get<int32_t>(); break;
    case V_F32: kv.kind = 2; kv.f = c.get<float>(); break;
    case V_BOOL: kv.kind = 3; kv.u = c.get<uint8_t>() != 0; break;
    case V_STR: kv.kind = 4; c.str(kv.s); break;
    case V_U64: kv.kind = 1; kv.u = c.get<uint64_t>(); break;
    case V_I64: kv.kind = 0; kv.i = c.get<int64_t>(); break;
    case V_F64: kv.kind = 2; kv.f = c.get<double>(); break;
    case V_ARRAY: {
        const uint32_t et = c.get<uint32_t>();
        const uint64_t n = c.get<uint64_t>();
        if (c.err)
            return false;
        if (n > GGUF_MAX_ARRAY) {
            c.err = "TruncatedGguf";
            return false;
        }
        kv.elem_type = et;
        kv.count = n;
        if (et == V_STR) {
            kv.kind = 5;
            kv.strs.resize((size_t)n);
            for (auto &s : kv.strs)
                if (!c.str(s))
                    return false;
        } else if (et == V_F32) {
            kv.kind = 6;
            kv.f32s.resize((size_t)n);
            for (auto &v : kv.f32s)
                v = c.get<float>();
        } else if (et == V_I32) {
            kv.kind = 7;
            kv.i32s.resize((size_t)n);
            for (auto &v : kv.i32s)
                v = c.get<int32_t>();
        } else {
            kv.kind = 8;
            Kv skip;
            for (uint64_t k = 0; k < n && !c.err; k++)
                read_value(c, et, skip, depth + 1);
        }
        break;
    }
    default: c.err = "UnknownValueType"; return false;
    }
    return !c.err;
}

} // namespace lh

using namespace lh;

struct loomhip_gguf {
    uint32_t version = 0;
    uint64_t alignment = 32, data_offset = 0, file_size = 0;
    std::vector<Kv> kvs;
    std::vector<Tensor> tensors;
    const uint8_t *map = nullptr;
    size_t map_len = 0;
};

struct loomhip_gguf_writer {
    uint64_t alignment = 32;
    std::vector<uint8_t> kv;
    uint64_t n_kv = 0;
    struct T {
        std::string name;
        std::vector<uint64_t> dims;
        uint32_t type;
        std::vector<uint8_t> data;
    };
    std::vector<T> tensors;
};

namespace {

const Kv *find_kv(const loomhip_gguf *g, const char *key) {
    if (!g || !key)
        return nullptr;
    for (const Kv &kv : g->kvs)
        if (kv.key == key)
            return &kv;
    return nullptr;
}

template <class T> void put(std::vector<uint8_t> &b, T v) {
    const uint8_t *p = (const uint8_t *)&v;
    b.insert(b.end(), p, p + sizeof(T));
}
void put_str(std::vector<uint8_t> &b, const char *s, size_t n) {
    put<uint64_t>(b, n);
    b.insert(b.end(), (const uint8_t *)s, (const uint8_t *)s + n);
}

} // namespace

extern "C" {

int loomhip_gguf_open(const char *path, loomhip_gguf **out) {
    if (!path || !out)
        return fail(LOOMHIP_ERR_ARG, "gguf_open: null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0)
        return fail(LOOMHIP_ERR_ARG, "gguf_open: cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        close(fd);
        return fail(LOOMHIP_ERR_ARG, "TruncatedGguf: %s is empty", path);
    }
    const size_t size = (size_t)st.st_size;
    void *m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED)
        return fail(LOOMHIP_ERR_ARG, "gguf_open: cannot map %s", path);
    auto *g = new loomhip_gguf;
    g->map = (const uint8_t *)m;
    g->map_len = size;
    g->file_size = size;
    Cursor c{g->map, std::min(size, GGUF_HEAD_CAP)};
    auto bad = [&](const char *what) {
        loomhip_gguf_close(g);
        return fail(LOOMHIP_ERR_ARG, "%s: %s", what, path);
    };
    if (c.get<uint32_t>() != GGUF_MAGIC)
        return bad(c.err ? c.err : "NotGguf");
    g->version = c.get<uint32_t>();
    if (c.err)
        return bad(c.err);
    if (g->version < 2 || g->version > 3)
        return bad("UnsupportedGgufVersion");
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    if (c.err || n_tensors > GGUF_MAX_COUNT || n_kv > GGUF_MAX_COUNT)
        return bad("TruncatedGguf");
    g->kvs.resize((size_t)n_kv);
    for (Kv &kv : g->kvs) {
        kv.span_start = c.pos;
        if (!c.str(kv.key))
            return bad(c.err);
        kv.type = c.get<uint32_t>();
        if (c.err || !read_value(c, kv.type, kv, 0))
            return bad(c.err);
        kv.span_end = c.pos;
        for (const std::string &s : kv.strs)
            kv.str_ptrs.push_back(s.c_str());
    }
    g->tensors.resize((size_t)n_tensors);
    for (Tensor &t : g->tensors) {
        if (!c.str(t.name))
            return bad(c.err);
        t.n_dims = c.get<uint32_t>();
        if (c.err)
            return bad(c.err);
        if (t.n_dims == 0 || t.n_dims > 8)
            return bad("BadTensorDims");
        uint64_t elems = 1;
        for (uint32_t d = 0; d < t.n_dims; d++) {
            t.dims[d] = c.get<uint64_t>();
            if (c.err)
                return bad(c.err);
            if (t.dims[d] == 0 || elems > UINT64_MAX / t.dims[d])
                return bad("BadTensorDims");
            elems *= t.dims[d];
        }
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        if (c.err)
            return bad(c.err);
    }
    for (const Kv &kv : g->kvs) // general.alignment, unsigned or a positive signed value
        if (kv.key == "general.alignment") {
            if (kv.kind == 1)
                g->alignment = kv.u;
            else if (kv.kind == 0 && kv.i > 0)
                g->alignment = (uint64_t)kv.i;
        }
    if (g->alignment == 0 || (g->alignment & (g->alignment - 1)))
        return bad("BadAlignment");
    g->data_offset = (c.pos + g->alignment - 1) / g->alignment * g->alignment;
    if (g->data_offset > g->file_size)
        return bad("TruncatedGguf");
    *out = g;
    return LOOMHIP_OK;
}

void loomhip_gguf_close(loomhip_gguf *g) {
    if (!g)
        return;
    if (g->map)
        munmap((void *)g->map, g->map_len);
    delete g;
}

int loomhip_gguf_get_info(const loomhip_gguf *g, loomhip_gguf_info *info) {
    if (!g || !info)
        return fail(LOOMHIP_ERR_ARG, "gguf_get_info: null argument");
    info->version = g->version;
    info->alignment = g->alignment;
    info->n_tensors = g->tensors.size();
    info->n_kv = g->kvs.size();
    info->data_offset = g->data_offset;
    info->file_size = g->file_size;
    info->base = g->map;
    return LOOMHIP_OK;
}

int loomhip_gguf_get_tensor(const loomhip_gguf *g, size_t i, loomhip_gguf_tensor *t) {
    if (!g || !t || i >= g->tensors.size())
        return fail(LOOMHIP_ERR_ARG, "gguf_get_tensor: bad argument");
    const Tensor &s = g->tensors[i];
    t->name = s.name.c_str();
    t->n_dims = s.n_dims;
    for (int d = 0; d < 8; d++)
        t->dims[d] = d < (int)s.n_dims ? s.dims[d] : 1;
    t->ggml_type = s.type;
    t->offset = s.offset;
    t->nbytes = tensor_bytes(s);
    // the data pointer only when the bytes lie inside the file (the offset sum
    // checked for overflow, llama.zig:262-266 resolve)
    uint64_t at = 0;
    const bool sum_ok = !__builtin_add_overflow(g->data_offset, s.offset, &at);
    t->data = (t->nbytes && sum_ok && at <= g->file_size && t->nbytes <= g->file_size - at) ? g->map + at : nullptr;
    return LOOMHIP_OK;
}

int loomhip_gguf_find_tensor(const loomhip_gguf *g, const char *name, size_t *index) {
    if (!g || !name || !index)
        return fail(LOOMHIP_ERR_ARG, "gguf_find_tensor: null argument");
    for (size_t i = 0; i < g->tensors.size(); i++)
        if (g->tensors[i].name == name) {
            *index = i;
            return LOOMHIP_OK;
        }
    return fail(LOOMHIP_DECLINED, "gguf_find_tensor: no tensor %s", name);
}

int loomhip_gguf_get_kv(const loomhip_gguf *g, size_t i, loomhip_gguf_kv *out) {
    if (!g || !out || i >= g->kvs.size())
        return fail(LOOMHIP_ERR_ARG, "gguf_get_kv: bad argument");
    const Kv &kv = g->kvs[i];
    memset(out, 0, sizeof(*out));
    out->key = kv.key.c_str();
    out->type = kv.type;
    out->kind = kv.kind;
    out->i = kv.i;
    out->u = kv.u;
    out->f = kv.f;
    out->s = kv.s.c_str();
    out->s_len = kv.s.size();
    out->elem_type = kv.elem_type;
    out->count = kv.count;
    out->strs = kv.str_ptrs.empty() ? nullptr : kv.str_ptrs.data();
    out->f32s = kv.f32s.empty() ? nullptr : kv.f32s.data();
    out->i32s = kv.i32s.empty() ? nullptr : kv.i32s.data();
    out->span_start = kv.span_start;
    out->span_end = kv.span_end;
    return LOOMHIP_OK;
}

// Parsed.getUint / getFloat / getString / getBool (gguf.zig:97-137): the
// same coercions; DECLINED when the key is absent or of another kind.
int loomhip_gguf_get_uint(const loomhip_gguf *g, const char *key, uint64_t *v) {
    const Kv *kv = find_kv(g, key);
    if (!v || !kv || (kv->kind != 1 && !(kv->kind == 0 && kv->i >= 0)))
        return fail(LOOMHIP_DECLINED, "gguf_get_uint: %s", key ? key : "(null)");
    *v = kv->kind == 1 ? kv->u : (uint64_t)kv->i;
    return LOOMHIP_OK;
}

int loomhip_gguf_get_float(const loomhip_gguf *g, const char *key, double *v) {
    const Kv *kv = find_kv(g, key);
    if (!v || !kv || kv->kind > 2)
        return fail(LOOMHIP_DECLINED, "gguf_get_float: %s", key ? key : "(null)");
    *v = kv->kind == 2 ? kv->f : kv->kind == 1 ? (double)kv->u : (double)kv->i;
    return LOOMHIP_OK;
}

int loomhip_gguf_get_string(const loomhip_gguf *g, const char *key, const char **s, size_t *len) {
    const Kv *kv = find_kv(g, key);
    if (!s || !len || !kv || kv->kind != 4)
        return fail(LOOMHIP_DECLINED, "gguf_get_string: %s", key ? key : "(null)");
    *s = kv->s.c_str();
    *len = kv->s.size();
    return LOOMHIP_OK;
}

int loomhip_gguf_get_bool(const loomhip_gguf *g, const char *key, int *v) {
    const Kv *kv = find_kv(g, key);
    if (!v || !kv || (kv->kind != 3 && kv->kind != 1 && kv->kind != 0))
        return fail(LOOMHIP_DECLINED, "gguf_get_bool: %s", key ? key : "(null)");
    *v = kv->kind == 0 ? kv->i != 0 : kv->u != 0;
    return LOOMHIP_OK;
}

// ---- writer ------------------------------------------------------------------

int loomhip_gguf_writer_begin(uint64_t alignment, loomhip_gguf_writer **out) {
    if (!out || alignment == 0 || (alignment & (alignment - 1)))
        return fail(LOOMHIP_ERR_ARG, "gguf_writer_begin: alignment %llu", (unsigned long long)alignment);
    *out = new loomhip_gguf_writer;
    (*out)->alignment = alignment;
    return LOOMHIP_OK;
}

// One key/value: type is a GGUF value type; scalars read their bytes from
// value, a string is value[0..len), an array of elem_type holds len elements
// at value (strings: len const char * pointers, each NUL-terminated).
int loomhip_gguf_writer_kv(loomhip_gguf_writer *w, const char *key, uint32_t type, const void *value, uint64_t len,
                           uint32_t elem_type) {
    if (!w || !key || (!value && (type != V_STR && type != V_ARRAY ? true : len != 0)))
        return fail(LOOMHIP_ERR_ARG, "gguf_writer_kv: null argument");
    static const uint8_t scalar_bytes[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    std::vector<uint8_t> &b = w->kv;
    const size_t mark = b.size();
    put_str(b, key, strlen(key));
    put<uint32_t>(b, type);
    if (type == V_STR) {
        put_str(b, (const char *)value, (size_t)len);
    } else if (type == V_ARRAY) {
        if (elem_type == V_ARRAY || elem_type > V_F64) {
            b.resize(mark);
            return fail(LOOMHIP_ERR_ARG, "gguf_writer_kv: array of type %u", elem_type);
        }
        put<uint32_t>(b, elem_type);
        put<uint64_t>(b, len);
        if (elem_type == V_STR) {
            const char *const *ss = (const char *const *)value;
            for (uint64_t k = 0; k < len; k++)
                put_str(b, ss[k], strlen(ss[k]));
        } else {
            const uint8_t *p = (const uint8_t *)value;
            b.insert(b.end(), p, p + len * scalar_bytes[elem_type]);
        }
    } else if (type <= V_F64) {
        const uint8_t *p = (const uint8_t *)value;
        b.insert(b.end(), p, p + scalar_bytes[type]);
    } else {
        b.resize(mark);
        return fail(LOOMHIP_ERR_ARG, "gguf_writer_kv: value type %u", type);
    }
    w->n_kv++;
    return LOOMHIP_OK;
}

int loomhip_gguf_writer_tensor(loomhip_gguf_writer *w, const char *name, uint32_t n_dims, const uint64_t *dims,
                               uint32_t ggml_type, const void *data, uint64_t nbytes) {
    if (!w || !name || !dims || n_dims == 0 || n_dims > 8 || (nbytes && !data))
        return fail(LOOMHIP_ERR_ARG, "gguf_writer_tensor: bad argument");
    loomhip_gguf_writer::T t{name, std::vector<uint64_t>(dims, dims + n_dims), ggml_type, {}};
    Tensor probe;
    probe.n_dims = n_dims;
    for (uint32_t d = 0; d < n_dims; d++) {
        if (dims[d] == 0)
            return fail(LOOMHIP_ERR_ARG, "gguf_writer_tensor: %s has a zero dim", name);
        probe.dims[d] = dims[d];
    }
    probe.type = ggml_type;
    const uint64_t want = tensor_bytes(probe);
    if (want && want != nbytes)
        return fail(LOOMHIP_ERR_ARG, "gguf_writer_tensor: %s holds %llu bytes, its shape %llu", name,
                    (unsigned long long)nbytes, (unsigned long long)want);
    t.data.assign((const uint8_t *)data, (const uint8_t *)data + nbytes);
    w->tensors.push_back(std::move(t));
    return LOOMHIP_OK;
}

int loomhip_gguf_writer_finish(loomhip_gguf_writer *w, const char *path) {
    if (!w)
        return fail(LOOMHIP_ERR_ARG, "gguf_writer_finish: null writer");
    int rc = LOOMHIP_OK;
    std::vector<uint8_t> head;
    put<uint32_t>(head, GGUF_MAGIC);
    put<uint32_t>(head, 3);
    put<uint64_t>(head, w->tensors.size());
    put<uint64_t>(head, w->n_kv);
    head.insert(head.end(), w->kv.begin(), w->kv.end());
    uint64_t off = 0;
    std::vector<uint64_t> offs;
    for (const auto &t : w->tensors) {
        put_str(head, t.name.c_str(), t.name.size());
        put<uint32_t>(head, (uint32_t)t.dims.size());
        for (uint64_t d : t.dims)
            put<uint64_t>(head, d);
        put<uint32_t>(head, t.type);
        off = (off + w->alignment - 1) / w->alignment * w->alignment;
        put<uint64_t>(head, off);
        offs.push_back(off);
        off += t.data.size();
    }
    while (head.size() % w->alignment)
        head.push_back(0);
    FILE *f = path ? fopen(path, "wb") : nullptr;
    if (!f) {
        rc = fail(LOOMHIP_ERR_ARG, "gguf_writer_finish: cannot create %s", path ? path : "(null)");
    } else {
        bool ok = fwrite(head.data(), 1, head.size(), f) == head.size();
        uint64_t at = 0;
        static const uint8_t zeros[256] = {};
        for (size_t i = 0; ok && i < w->tensors.size(); i++) {
            while (ok && at < offs[i]) {
                const size_t n = (size_t)std::min<uint64_t>(sizeof(zeros), offs[i] - at);
                ok = fwrite(zeros, 1, n, f) == n;
                at += n;
            }
            const auto &d = w->tensors[i].data;
            ok = ok && fwrite(d.data(), 1, d.size(), f) == d.size();
            at += d.size();
        }
        ok = (fclose(f) == 0) && ok;
        if (!ok)
            rc = fail(LOOMHIP_ERR_ARG, "gguf_writer_finish: writing %s failed", path);
    }
    delete w;
    return rc;
}

void loomhip_gguf_writer_abort(loomhip_gguf_writer *w) { delete w; }

} // extern "C"
