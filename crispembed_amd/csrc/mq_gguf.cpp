// mq_gguf.cpp -- GGUF v3 reader (mq_gguf.h): a memory-mapped file, parsed with a cursor that
// checks every read against the file size.
//
// Layout (GGUF v2/v3, little-endian):
//   u32 magic "GGUF", u32 version, u64 n_tensors, u64 n_kv
//   n_kv x { string key, u32 type, value }          string = u64 length + bytes (no NUL)
//            value: scalar | string | array { u32 elem type, u64 n, n values }
//   n_tensors x { string name, u32 n_dims, u64 ne[n_dims], u32 ggml type, u64 offset }
//   padding to general.alignment (default 32); tensor data, each tensor at its offset (a
//   multiple of the alignment) from the start of the data section.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/mq.h"
#include "../../include/mq_gguf.h"

namespace mq {
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));  // mq_api.cpp
}
using mq::set_error;

namespace {

// ggml type -> (values per block, bytes per block); 0 for ids this reader does not size
struct TypeSize {
    int blck, bytes;
};
TypeSize ggml_type_size(int t) {
    switch (t) {
        case 0: return {1, 4};      // F32
        case 1: return {1, 2};      // F16
        case 2: return {32, 18};    // Q4_0
        case 3: return {32, 20};    // Q4_1
        case 6: return {32, 22};    // Q5_0
        case 7: return {32, 24};    // Q5_1
        case 8: return {32, 34};    // Q8_0
        case 9: return {32, 36};    // Q8_1
        case 10: return {256, 84};  // Q2_K
        case 11: return {256, 110}; // Q3_K
        case 12: return {256, 144}; // Q4_K
        case 13: return {256, 176}; // Q5_K
        case 14: return {256, 210}; // Q6_K
        case 15: return {256, 292}; // Q8_K
        case 16: return {256, 66};  // IQ2_XXS
        case 17: return {256, 74};  // IQ2_XS
        case 18: return {256, 98};  // IQ3_XXS
        case 19: return {256, 50};  // IQ1_S
        case 20: return {32, 18};   // IQ4_NL
        case 21: return {256, 110}; // IQ3_S
        case 22: return {256, 82};  // IQ2_S
        case 23: return {256, 136}; // IQ4_XS
        case 24: return {1, 1};     // I8
        case 25: return {1, 2};     // I16
        case 26: return {1, 4};     // I32
        case 27: return {1, 8};     // I64
        case 28: return {1, 8};     // F64
        case 29: return {256, 56};  // IQ1_M
        case 30: return {1, 2};     // BF16
        case 34: return {256, 54};  // TQ1_0
        case 35: return {256, 66};  // TQ2_0
        case 39: return {32, 17};   // MXFP4
        default: return {0, 0};
    }
}

size_t scalar_size(uint32_t t) {
    switch (t) {
        case MQ_GGUF_UINT8:
        case MQ_GGUF_INT8:
        case MQ_GGUF_BOOL: return 1;
        case MQ_GGUF_UINT16:
        case MQ_GGUF_INT16: return 2;
        case MQ_GGUF_UINT32:
        case MQ_GGUF_INT32:
        case MQ_GGUF_FLOAT32: return 4;
        case MQ_GGUF_UINT64:
        case MQ_GGUF_INT64:
        case MQ_GGUF_FLOAT64: return 8;
        default: return 0;
    }
}

struct Cursor {
    const uint8_t *base;
    size_t size, pos = 0;
    bool ok = true;
    const char *what = "";
    bool need(size_t n, const char *w) {
        if (!ok) return false;
        if (n > size - pos) {
            ok = false;
            what = w;
        }
        return ok;
    }
    template <class T>
    T get(const char *w) {
        T v{};
        if (need(sizeof(T), w)) {
            std::memcpy(&v, base + pos, sizeof(T));
            pos += sizeof(T);
        }
        return v;
    }
    // a string: returns its bytes and length (pointing into the mapping)
    bool str(const char *&p, uint64_t &n, const char *w) {
        n = get<uint64_t>(w);
        if (!need(n, w)) return false;
        p = (const char *)base + pos;
        pos += n;
        return true;
    }
    void skip(size_t n, const char *w) {
        if (need(n, w)) pos += n;
    }
};

struct KV {
    std::string key;
    uint32_t type = 0;
    size_t at = 0;  // file offset of the value (scalar) or of the first array element
    uint32_t arr_type = 0;
    uint64_t arr_n = 0;
    std::string sval;                // STRING value
    std::vector<std::string> strs;   // ARRAY of STRING
};

struct Tensor {
    std::string name;
    int type = 0, n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    size_t offset = 0, nbytes = 0;
};

}  // namespace

struct mq_gguf {
    void *map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    size_t alignment = 32, data_off = 0;
    std::vector<KV> kvs;
    std::unordered_map<std::string, int64_t> kv_index;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int64_t> t_index;
    ~mq_gguf() {
        if (map) munmap(map, size);
    }
    const uint8_t *bytes() const { return (const uint8_t *)map; }
};

namespace {

mq_gguf *fail_open(mq_gguf *g, const char *path, const char *why) {
    set_error(MQ_EINVAL, "GGUF '%s': %s", path, why);
    delete g;
    return nullptr;
}

// reads an array value's elements into kv (strings copied, numbers left in the mapping)
bool read_array(Cursor &c, KV &kv) {
    kv.arr_type = c.get<uint32_t>("array type");
    kv.arr_n = c.get<uint64_t>("array length");
    if (!c.ok) return false;
    if (kv.arr_type == MQ_GGUF_STRING) {
        if (kv.arr_n > c.size / 8) {  // every element takes at least its 8-byte length
            c.ok = false;
            c.what = "string array length";
            return false;
        }
        kv.strs.reserve(kv.arr_n);
        for (uint64_t i = 0; i < kv.arr_n && c.ok; i++) {
            const char *p;
            uint64_t n;
            if (c.str(p, n, "string array element")) kv.strs.emplace_back(p, n);
        }
        return c.ok;
    }
    const size_t es = scalar_size(kv.arr_type);
    if (es == 0) {  // nested arrays are not part of the format
        c.ok = false;
        c.what = "array element type";
        return false;
    }
    if (kv.arr_n > (c.size - c.pos) / es) {
        c.ok = false;
        c.what = "array data";
        return false;
    }
    kv.at = c.pos;
    c.skip(kv.arr_n * es, "array data");
    return c.ok;
}

template <class T>
T scalar_at(const mq_gguf *g, const KV &kv) {
    T v;
    std::memcpy(&v, g->bytes() + kv.at, sizeof(T));
    return v;
}

const KV *find(const mq_gguf *g, const char *key) {
    if (!g || !key) return nullptr;
    auto it = g->kv_index.find(key);
    return it == g->kv_index.end() ? nullptr : &g->kvs[it->second];
}

}  // namespace

extern "C" mq_gguf *mq_gguf_open(const char *path) {
    if (!path) {
        set_error(MQ_EINVAL, "NULL path");
        return nullptr;
    }
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        set_error(MQ_EINVAL, "GGUF '%s': cannot open", path);
        return nullptr;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        set_error(MQ_EINVAL, "GGUF '%s': not a GGUF file (too short)", path);
        return nullptr;
    }
    mq_gguf *g = new mq_gguf();
    g->size = (size_t)st.st_size;
    g->map = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (g->map == MAP_FAILED) {
        g->map = nullptr;
        return fail_open(g, path, "mmap failed");
    }
    Cursor c{g->bytes(), g->size};
    if (std::memcmp(g->bytes(), "GGUF", 4) != 0) return fail_open(g, path, "bad magic (not a GGUF file)");
    c.pos = 4;
    g->version = c.get<uint32_t>("version");
    if (g->version != 2 && g->version != 3) return fail_open(g, path, "unsupported GGUF version (2 and 3 are read)");
    const uint64_t n_tensors = c.get<uint64_t>("tensor count"), n_kv = c.get<uint64_t>("kv count");
    // every kv takes >= 12 bytes and every tensor info >= 28: bounds the counts by the file size
    if (n_kv > g->size / 12 || n_tensors > g->size / 28) return fail_open(g, path, "kv or tensor count exceeds the file");
    g->kvs.reserve(n_kv);
    for (uint64_t i = 0; i < n_kv && c.ok; i++) {
        KV kv;
        const char *kp;
        uint64_t kn;
        if (!c.str(kp, kn, "kv key")) break;
        kv.key.assign(kp, kn);
        kv.type = c.get<uint32_t>("kv type");
        if (!c.ok) break;
        if (kv.type == MQ_GGUF_STRING) {
            const char *p;
            uint64_t n;
            if (c.str(p, n, "string value")) kv.sval.assign(p, n);
        } else if (kv.type == MQ_GGUF_ARRAY) {
            read_array(c, kv);
        } else {
            const size_t es = scalar_size(kv.type);
            if (es == 0) return fail_open(g, path, ("unknown value type of key '" + kv.key + "'").c_str());
            kv.at = c.pos;
            c.skip(es, "scalar value");
        }
        if (!c.ok) break;
        if (g->kv_index.count(kv.key)) return fail_open(g, path, ("duplicate key '" + kv.key + "'").c_str());
        g->kv_index.emplace(kv.key, (int64_t)g->kvs.size());
        g->kvs.push_back(std::move(kv));
    }
    if (!c.ok) return fail_open(g, path, (std::string("truncated or malformed metadata (") + c.what + ")").c_str());
    if (const KV *a = find(g, "general.alignment")) {
        if (a->type != MQ_GGUF_UINT32) return fail_open(g, path, "general.alignment is not UINT32");
        const uint32_t al = scalar_at<uint32_t>(g, *a);
        if (al == 0 || (al & (al - 1)) != 0) return fail_open(g, path, "general.alignment is not a power of two");
        g->alignment = al;
    }
    g->tensors.reserve(n_tensors);
    for (uint64_t i = 0; i < n_tensors && c.ok; i++) {
        Tensor t;
        const char *np;
        uint64_t nn;
        if (!c.str(np, nn, "tensor name")) break;
        t.name.assign(np, nn);
        const uint32_t nd = c.get<uint32_t>("tensor dims");
        if (!c.ok) break;
        if (nd < 1 || nd > 4) return fail_open(g, path, ("tensor '" + t.name + "': n_dims not in 1..4").c_str());
        t.n_dims = (int)nd;
        uint64_t nel = 1;
        for (uint32_t d = 0; d < nd; d++) {
            const uint64_t e = c.get<uint64_t>("tensor shape");
            if (!c.ok) break;
            if (e == 0 || e > ((uint64_t)1 << 40) || nel > ((uint64_t)1 << 50) / e)
                return fail_open(g, path, ("tensor '" + t.name + "': bad shape").c_str());
            t.ne[d] = (int64_t)e;
            nel *= e;
        }
        t.type = (int)c.get<uint32_t>("tensor type");
        t.offset = (size_t)c.get<uint64_t>("tensor offset");
        if (!c.ok) break;
        const TypeSize ts = ggml_type_size(t.type);
        if (ts.blck == 0) return fail_open(g, path, ("tensor '" + t.name + "': unknown ggml type").c_str());
        if (t.ne[0] % ts.blck != 0)
            return fail_open(g, path, ("tensor '" + t.name + "': row length not a multiple of the block size").c_str());
        t.nbytes = (size_t)(nel / ts.blck) * ts.bytes;
        if (g->t_index.count(t.name)) return fail_open(g, path, ("duplicate tensor '" + t.name + "'").c_str());
        g->t_index.emplace(t.name, (int64_t)g->tensors.size());
        g->tensors.push_back(std::move(t));
    }
    if (!c.ok) return fail_open(g, path, (std::string("truncated or malformed tensor infos (") + c.what + ")").c_str());
    g->data_off = (c.pos + g->alignment - 1) / g->alignment * g->alignment;
    for (const Tensor &t : g->tensors) {
        if (t.offset % g->alignment != 0)
            return fail_open(g, path, ("tensor '" + t.name + "': data offset not aligned").c_str());
        if (g->data_off > g->size || t.offset > g->size - g->data_off || t.nbytes > g->size - g->data_off - t.offset)
            return fail_open(g, path, ("tensor '" + t.name + "': data past the end of the file").c_str());
    }
    return g;
}

extern "C" void mq_gguf_close(mq_gguf *g) { delete g; }

extern "C" uint32_t mq_gguf_version(const mq_gguf *g) { return g ? g->version : 0; }
extern "C" size_t mq_gguf_alignment(const mq_gguf *g) { return g ? g->alignment : 0; }
extern "C" size_t mq_gguf_data_offset(const mq_gguf *g) { return g ? g->data_off : 0; }
extern "C" int64_t mq_gguf_n_kv(const mq_gguf *g) { return g ? (int64_t)g->kvs.size() : 0; }

extern "C" int64_t mq_gguf_find_key(const mq_gguf *g, const char *key) {
    if (!g || !key) return -1;
    auto it = g->kv_index.find(key);
    return it == g->kv_index.end() ? -1 : it->second;
}

static const KV *kv_at(const mq_gguf *g, int64_t i) {
    return (g && i >= 0 && i < (int64_t)g->kvs.size()) ? &g->kvs[i] : nullptr;
}

extern "C" const char *mq_gguf_kv_key(const mq_gguf *g, int64_t i) {
    const KV *kv = kv_at(g, i);
    return kv ? kv->key.c_str() : nullptr;
}
extern "C" int mq_gguf_kv_type(const mq_gguf *g, int64_t i) {
    const KV *kv = kv_at(g, i);
    return kv ? (int)kv->type : -1;
}
extern "C" int mq_gguf_arr_type(const mq_gguf *g, int64_t i) {
    const KV *kv = kv_at(g, i);
    return (kv && kv->type == MQ_GGUF_ARRAY) ? (int)kv->arr_type : -1;
}
extern "C" int64_t mq_gguf_arr_n(const mq_gguf *g, int64_t i) {
    const KV *kv = kv_at(g, i);
    return (kv && kv->type == MQ_GGUF_ARRAY) ? (int64_t)kv->arr_n : -1;
}
extern "C" const void *mq_gguf_arr_data(const mq_gguf *g, int64_t i) {
    const KV *kv = kv_at(g, i);
    if (!kv || kv->type != MQ_GGUF_ARRAY || kv->arr_type == MQ_GGUF_STRING) return nullptr;
    return g->bytes() + kv->at;
}
extern "C" const void *mq_gguf_kv_data(const mq_gguf *g, int64_t i) {
    const KV *kv = kv_at(g, i);
    if (!kv || scalar_size(kv->type) == 0) return nullptr;
    return g->bytes() + kv->at;
}
extern "C" const char *mq_gguf_arr_str(const mq_gguf *g, int64_t i, int64_t j) {
    const KV *kv = kv_at(g, i);
    if (!kv || kv->type != MQ_GGUF_ARRAY || kv->arr_type != MQ_GGUF_STRING || j < 0 || j >= (int64_t)kv->strs.size())
        return nullptr;
    return kv->strs[j].c_str();
}

extern "C" uint32_t mq_gguf_get_u32(const mq_gguf *g, const char *key, uint32_t def) {
    const KV *kv = find(g, key);
    if (!kv) return def;
    switch (kv->type) {
        case MQ_GGUF_UINT32: return scalar_at<uint32_t>(g, *kv);
        case MQ_GGUF_INT32: return (uint32_t)scalar_at<int32_t>(g, *kv);
        case MQ_GGUF_UINT64: return (uint32_t)scalar_at<uint64_t>(g, *kv);
        case MQ_GGUF_INT64: return (uint32_t)scalar_at<int64_t>(g, *kv);
        case MQ_GGUF_UINT16: return scalar_at<uint16_t>(g, *kv);
        case MQ_GGUF_INT16: return (uint32_t)scalar_at<int16_t>(g, *kv);
        case MQ_GGUF_UINT8: return scalar_at<uint8_t>(g, *kv);
        case MQ_GGUF_INT8: return (uint32_t)scalar_at<int8_t>(g, *kv);
        default: return def;
    }
}
extern "C" int32_t mq_gguf_get_i32(const mq_gguf *g, const char *key, int32_t def) {
    const KV *kv = find(g, key);
    if (!kv) return def;
    switch (kv->type) {
        case MQ_GGUF_INT32: return scalar_at<int32_t>(g, *kv);
        case MQ_GGUF_UINT32: return (int32_t)scalar_at<uint32_t>(g, *kv);
        case MQ_GGUF_INT64: return (int32_t)scalar_at<int64_t>(g, *kv);
        case MQ_GGUF_UINT64: return (int32_t)scalar_at<uint64_t>(g, *kv);
        default: return def;
    }
}
extern "C" float mq_gguf_get_f32(const mq_gguf *g, const char *key, float def) {
    const KV *kv = find(g, key);
    if (!kv) return def;
    if (kv->type == MQ_GGUF_FLOAT32) return scalar_at<float>(g, *kv);
    if (kv->type == MQ_GGUF_FLOAT64) return (float)scalar_at<double>(g, *kv);
    return def;
}
extern "C" int mq_gguf_get_bool(const mq_gguf *g, const char *key, int def) {
    const KV *kv = find(g, key);
    if (!kv || kv->type != MQ_GGUF_BOOL) return def;
    return scalar_at<uint8_t>(g, *kv) != 0;
}
extern "C" const char *mq_gguf_get_str(const mq_gguf *g, const char *key, const char *def) {
    const KV *kv = find(g, key);
    if (!kv || kv->type != MQ_GGUF_STRING) return def;
    return kv->sval.c_str();
}

extern "C" int64_t mq_gguf_n_tensors(const mq_gguf *g) { return g ? (int64_t)g->tensors.size() : 0; }
extern "C" int64_t mq_gguf_find_tensor(const mq_gguf *g, const char *name) {
    if (!g || !name) return -1;
    auto it = g->t_index.find(name);
    return it == g->t_index.end() ? -1 : it->second;
}
extern "C" const char *mq_gguf_tensor_name(const mq_gguf *g, int64_t i) {
    return (g && i >= 0 && i < (int64_t)g->tensors.size()) ? g->tensors[i].name.c_str() : nullptr;
}
extern "C" int mq_gguf_tensor_info(const mq_gguf *g, int64_t i, int *type, int *n_dims, int64_t ne[4], size_t *offset,
                                   size_t *nbytes) {
    if (!g || i < 0 || i >= (int64_t)g->tensors.size()) return set_error(MQ_EINVAL, "bad tensor index %lld", (long long)i);
    const Tensor &t = g->tensors[i];
    if (type) *type = t.type;
    if (n_dims) *n_dims = t.n_dims;
    if (ne)
        for (int d = 0; d < 4; d++) ne[d] = t.ne[d];
    if (offset) *offset = t.offset;
    if (nbytes) *nbytes = t.nbytes;
    return MQ_OK;
}
extern "C" const void *mq_gguf_tensor_data(const mq_gguf *g, int64_t i) {
    if (!g || i < 0 || i >= (int64_t)g->tensors.size()) return nullptr;
    return g->bytes() + g->data_off + g->tensors[i].offset;
}
