// qlin_gguf.cpp -- GGUF container reader and device weight pool behind include/qlin_gguf.h.
//
// Follows the reference's GgufFile (AI/codes/local-llm/src/format/gguf/GgufFile.cpp:152-247) for
// what is accepted and where each tensor's bytes are, and CudaWeightPool::cached_weight
// (src/backend/cuda/mem/CudaWeightPool.cpp:119-175) for residency: one device copy per tensor,
// expert slices as views of it.  Host code only; the kernels never see this file's types.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "qlin_gguf.h"

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" read as a little-endian u32
constexpr uint32_t kDefaultAlignment = 32;

// (elements, bytes) per block of each ggml type the reference knows (GgufFile.cpp:35-55); the on-disk
// format fixes these numbers.
bool block_trait(int type, int64_t &elems, int64_t &bytes) {
    switch (type) {
        case 0: elems = 1; bytes = 4; return true;      // F32
        case 1: elems = 1; bytes = 2; return true;      // F16
        case 30: elems = 1; bytes = 2; return true;     // BF16
        case 2: elems = 32; bytes = 18; return true;    // Q4_0
        case 3: elems = 32; bytes = 20; return true;    // Q4_1
        case 6: elems = 32; bytes = 22; return true;    // Q5_0
        case 7: elems = 32; bytes = 24; return true;    // Q5_1
        case 8: elems = 32; bytes = 34; return true;    // Q8_0
        case 9: elems = 32; bytes = 36; return true;    // Q8_1
        case 10: elems = 256; bytes = 84; return true;  // Q2_K
        case 11: elems = 256; bytes = 110; return true; // Q3_K
        case 12: elems = 256; bytes = 144; return true; // Q4_K
        case 13: elems = 256; bytes = 176; return true; // Q5_K
        case 14: elems = 256; bytes = 210; return true; // Q6_K
        case 15: elems = 256; bytes = 292; return true; // Q8_K
        default: return false;
    }
}

struct FormatError {};

// Bounds-checked little-endian reads from the mapped file.
class Cursor {
public:
    Cursor(const uint8_t *base, size_t size) : base_(base), size_(size) {}
    size_t pos() const { return pos_; }
    size_t left() const { return size_ - pos_; }
    const uint8_t *take(size_t n) {
        if (n > left()) throw FormatError{};
        const uint8_t *p = base_ + pos_;
        pos_ += n;
        return p;
    }
    uint64_t uint(size_t n) {
        const uint8_t *p = take(n);
        uint64_t v = 0;
        for (size_t i = 0; i < n; ++i) v |= static_cast<uint64_t>(p[i]) << (8 * i);
        return v;
    }
    std::string str() {
        const uint64_t len = uint(8);
        if (len > left()) throw FormatError{};
        const uint8_t *p = take(static_cast<size_t>(len));
        return std::string(reinterpret_cast<const char *>(p), static_cast<size_t>(len));
    }

private:
    const uint8_t *base_;
    size_t size_;
    size_t pos_ = 0;
};

struct Value {
    int type = -1;
    int64_t i = 0;   // integers of every width, bool
    double f = 0.0;  // f32, f64
    std::string s;
    int elem = -1;   // arrays
    int64_t count = 0;
    std::vector<int64_t> ai;
    std::vector<double> af;
    std::vector<std::string> as;
};

bool is_int_type(int t) {
    return t == QLIN_GGUF_U8 || t == QLIN_GGUF_I8 || t == QLIN_GGUF_U16 || t == QLIN_GGUF_I16 || t == QLIN_GGUF_U32 ||
           t == QLIN_GGUF_I32 || t == QLIN_GGUF_U64 || t == QLIN_GGUF_I64 || t == QLIN_GGUF_BOOL;
}
bool is_float_type(int t) { return t == QLIN_GGUF_F32 || t == QLIN_GGUF_F64; }

// Smallest encoding of one value of type t (for count sanity checks before reserving memory).
size_t min_size(int t) {
    switch (t) {
        case QLIN_GGUF_U8: case QLIN_GGUF_I8: case QLIN_GGUF_BOOL: return 1;
        case QLIN_GGUF_U16: case QLIN_GGUF_I16: return 2;
        case QLIN_GGUF_U32: case QLIN_GGUF_I32: case QLIN_GGUF_F32: return 4;
        case QLIN_GGUF_STRING: return 8;
        case QLIN_GGUF_ARRAY: return 12;
        default: return 8;
    }
}

Value read_value(Cursor &c, int type, int depth) {
    Value v;
    v.type = type;
    switch (type) {
        case QLIN_GGUF_U8: v.i = static_cast<int64_t>(c.uint(1)); break;
        case QLIN_GGUF_I8: v.i = static_cast<int8_t>(c.uint(1)); break;
        case QLIN_GGUF_U16: v.i = static_cast<int64_t>(c.uint(2)); break;
        case QLIN_GGUF_I16: v.i = static_cast<int16_t>(c.uint(2)); break;
        case QLIN_GGUF_U32: v.i = static_cast<int64_t>(c.uint(4)); break;
        case QLIN_GGUF_I32: v.i = static_cast<int32_t>(c.uint(4)); break;
        case QLIN_GGUF_U64: case QLIN_GGUF_I64: v.i = static_cast<int64_t>(c.uint(8)); break;
        case QLIN_GGUF_BOOL: v.i = c.uint(1) != 0; break;
        case QLIN_GGUF_F32: {
            const uint32_t b = static_cast<uint32_t>(c.uint(4));
            float f;
            std::memcpy(&f, &b, 4);
            v.f = f;
            break;
        }
        case QLIN_GGUF_F64: {
            const uint64_t b = c.uint(8);
            std::memcpy(&v.f, &b, 8);
            break;
        }
        case QLIN_GGUF_STRING: v.s = c.str(); break;
        case QLIN_GGUF_ARRAY: {
            if (depth > 4) throw FormatError{};
            v.elem = static_cast<int>(c.uint(4));
            const uint64_t n = c.uint(8);
            if (v.elem < 0 || v.elem > QLIN_GGUF_F64) throw FormatError{};
            if (n > c.left() / min_size(v.elem)) throw FormatError{};
            v.count = static_cast<int64_t>(n);
            for (uint64_t k = 0; k < n; ++k) {
                Value e = read_value(c, v.elem, depth + 1);
                if (v.elem == QLIN_GGUF_STRING) v.as.push_back(std::move(e.s));
                else if (is_float_type(v.elem)) v.af.push_back(e.f);
                else if (is_int_type(v.elem)) v.ai.push_back(e.i);
                // nested arrays are parsed past but their elements are not kept
            }
            break;
        }
        default: throw FormatError{};
    }
    return v;
}

struct Tensor {
    std::string name;
    int type = 0;
    int n_dims = 0;
    int64_t shape[QLIN_GGUF_MAX_DIMS] = {1, 1, 1, 1};
    uint64_t nbytes = 0, offset = 0;
    const uint8_t *data = nullptr;
};

}  // namespace

struct qlin_gguf {
    int fd = -1;
    const uint8_t *map = nullptr;
    size_t size = 0;
    uint32_t version = 0, alignment = kDefaultAlignment;
    std::vector<std::pair<std::string, Value>> meta;
    std::unordered_map<std::string, size_t> meta_index;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> tensor_index;

    ~qlin_gguf() {
        if (map) munmap(const_cast<uint8_t *>(map), size);
        if (fd >= 0) ::close(fd);
    }
    const Value *find(const char *key) const {
        if (!key) return nullptr;
        const auto it = meta_index.find(key);
        return it == meta_index.end() ? nullptr : &meta[it->second].second;
    }

    // GgufFile.cpp:171-231: header, metadata, tensor table, then the aligned data section.
    void parse() {
        Cursor c(map, size);
        if (c.uint(4) != kMagic) throw FormatError{};
        version = static_cast<uint32_t>(c.uint(4));
        if (version != 2 && version != 3) throw FormatError{};
        const uint64_t n_tensors = c.uint(8), n_kv = c.uint(8);
        if (n_kv > c.left() / 12 || n_tensors > c.left() / 24) throw FormatError{};
        meta.reserve(static_cast<size_t>(n_kv));
        for (uint64_t k = 0; k < n_kv; ++k) {
            std::string key = c.str();
            const int type = static_cast<int>(c.uint(4));
            Value v = read_value(c, type, 0);
            meta_index[key] = meta.size();  // a repeated key: the last value wins, as a std::map assignment
            meta.emplace_back(std::move(key), std::move(v));
        }
        if (const Value *a = find("general.alignment")) {
            if (!is_int_type(a->type) || a->i < 0 || a->i > (int64_t{1} << 30)) throw FormatError{};
            alignment = a->i == 0 ? kDefaultAlignment : static_cast<uint32_t>(a->i);
        }
        tensors.resize(static_cast<size_t>(n_tensors));
        for (Tensor &t : tensors) {
            t.name = c.str();
            const uint32_t nd = static_cast<uint32_t>(c.uint(4));
            if (nd > QLIN_GGUF_MAX_DIMS) throw FormatError{};
            t.n_dims = static_cast<int>(nd);
            uint64_t dims[QLIN_GGUF_MAX_DIMS] = {1, 1, 1, 1};
            uint64_t elems = 1;
            for (uint32_t d = 0; d < nd; ++d) {
                dims[d] = c.uint(8);
                if (dims[d] > (uint64_t{1} << 40) || (dims[d] && elems > (uint64_t{1} << 62) / dims[d]))
                    throw FormatError{};
                elems *= dims[d];
            }
            for (uint32_t d = 0; d < nd; ++d) t.shape[d] = static_cast<int64_t>(dims[nd - 1 - d]);
            t.type = static_cast<int>(c.uint(4));
            t.offset = c.uint(8);
            int64_t be, bb;
            // whole blocks per row (ne[0], the innermost dimension), and a byte count that fits in 64 bits
            if (!block_trait(t.type, be, bb) || elems % static_cast<uint64_t>(be) ||
                (nd > 0 && dims[0] % static_cast<uint64_t>(be)))
                throw FormatError{};
            const uint64_t nblocks = elems / static_cast<uint64_t>(be);
            if (nblocks > UINT64_MAX / static_cast<uint64_t>(bb)) throw FormatError{};
            t.nbytes = nblocks * static_cast<uint64_t>(bb);
        }
        size_t start = c.pos();
        if (start % alignment) start += alignment - start % alignment;
        if (start > size) throw FormatError{};
        for (size_t k = 0; k < tensors.size(); ++k) {
            Tensor &t = tensors[k];
            if (t.offset > size - start || t.nbytes > size - start - t.offset) throw FormatError{};
            t.data = map + start + t.offset;
            tensor_index.emplace(t.name, k);  // the first tensor of a name, as the reference's search
        }
    }
};

namespace {

// Host-to-device copy of file-mapped bytes through a pinned staging buffer of at most 32 MB: the copy
// runs from pinned memory without ever registering (pinning) the mapped file pages themselves.
bool upload(void *dev, const uint8_t *src, uint64_t n) {
    constexpr uint64_t kChunk = uint64_t{32} << 20;
    if (n == 0) return true;
    void *stage = nullptr;
    const uint64_t sz = n < kChunk ? n : kChunk;
    if (hipHostMalloc(&stage, sz, hipHostMallocDefault) != hipSuccess) return false;
    bool ok = true;
    for (uint64_t off = 0; ok && off < n; off += sz) {
        const uint64_t len = n - off < sz ? n - off : sz;
        std::memcpy(stage, src + off, len);
        ok = hipMemcpy(static_cast<uint8_t *>(dev) + off, stage, len, hipMemcpyHostToDevice) == hipSuccess;
    }
    (void)hipHostFree(stage);
    return ok;
}

}  // namespace

struct qlin_pool {
    struct Entry {
        void *dev = nullptr;
        uint64_t bytes = 0;
    };
    std::unordered_map<std::string, Entry> items;
    uint64_t resident = 0;
    ~qlin_pool() {
        for (auto &kv : items) (void)hipFree(kv.second.dev);
    }
};

extern "C" {

int qlin_gguf_open(const char *path, qlin_gguf **out) {
    if (!path || !out) return QLIN_ERR_NULL;
    *out = nullptr;
    std::unique_ptr<qlin_gguf> g(new (std::nothrow) qlin_gguf);
    if (!g) return QLIN_ERR_ALLOC;
    g->fd = ::open(path, O_RDONLY);
    if (g->fd < 0) return QLIN_ERR_IO;
    struct stat st {};
    if (fstat(g->fd, &st) != 0) return QLIN_ERR_IO;
    g->size = static_cast<size_t>(st.st_size);
    if (g->size < 24) return QLIN_ERR_FORMAT;  // magic, version and the two counts
    void *p = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (p == MAP_FAILED) return QLIN_ERR_IO;
    g->map = static_cast<const uint8_t *>(p);
    try {
        g->parse();
    } catch (const FormatError &) {
        return QLIN_ERR_FORMAT;
    } catch (const std::bad_alloc &) {
        return QLIN_ERR_FORMAT;
    }
    *out = g.release();
    return QLIN_OK;
}

void qlin_gguf_close(qlin_gguf *g) { delete g; }
uint32_t qlin_gguf_version(const qlin_gguf *g) { return g ? g->version : 0; }
uint32_t qlin_gguf_alignment(const qlin_gguf *g) { return g ? g->alignment : 0; }
int64_t qlin_gguf_tensor_count(const qlin_gguf *g) { return g ? static_cast<int64_t>(g->tensors.size()) : 0; }

int64_t qlin_gguf_find_tensor(const qlin_gguf *g, const char *name) {
    if (!g || !name) return -1;
    const auto it = g->tensor_index.find(name);
    return it == g->tensor_index.end() ? -1 : static_cast<int64_t>(it->second);
}

int qlin_gguf_tensor_info(const qlin_gguf *g, int64_t index, qlin_gguf_tensor *out) {
    if (!g || !out) return QLIN_ERR_NULL;
    if (index < 0 || index >= static_cast<int64_t>(g->tensors.size())) return QLIN_ERR_NOT_FOUND;
    const Tensor &t = g->tensors[static_cast<size_t>(index)];
    out->name = t.name.c_str();
    out->type = t.type;
    out->n_dims = t.n_dims;
    for (int d = 0; d < QLIN_GGUF_MAX_DIMS; ++d) out->shape[d] = t.shape[d];
    out->nbytes = t.nbytes;
    out->offset = t.offset;
    out->data = t.data;
    return QLIN_OK;
}

int64_t qlin_gguf_metadata_count(const qlin_gguf *g) { return g ? static_cast<int64_t>(g->meta.size()) : 0; }

const char *qlin_gguf_metadata_key(const qlin_gguf *g, int64_t index) {
    if (!g || index < 0 || index >= static_cast<int64_t>(g->meta.size())) return nullptr;
    return g->meta[static_cast<size_t>(index)].first.c_str();
}

int qlin_gguf_metadata_type(const qlin_gguf *g, const char *key) {
    const Value *v = g ? g->find(key) : nullptr;
    return v ? v->type : -1;
}

int qlin_gguf_get_i64(const qlin_gguf *g, const char *key, int64_t *out) {
    if (!g || !key || !out) return QLIN_ERR_NULL;
    const Value *v = g->find(key);
    if (!v || !is_int_type(v->type)) return QLIN_ERR_NOT_FOUND;
    *out = v->i;
    return QLIN_OK;
}

int qlin_gguf_get_f64(const qlin_gguf *g, const char *key, double *out) {
    if (!g || !key || !out) return QLIN_ERR_NULL;
    const Value *v = g->find(key);
    if (!v || !is_float_type(v->type)) return QLIN_ERR_NOT_FOUND;
    *out = v->f;
    return QLIN_OK;
}

int qlin_gguf_get_str(const qlin_gguf *g, const char *key, const char **out, size_t *len) {
    if (!g || !key || !out || !len) return QLIN_ERR_NULL;
    const Value *v = g->find(key);
    if (!v || v->type != QLIN_GGUF_STRING) return QLIN_ERR_NOT_FOUND;
    *out = v->s.c_str();
    *len = v->s.size();
    return QLIN_OK;
}

int qlin_gguf_get_array_info(const qlin_gguf *g, const char *key, int *elem_type, int64_t *count) {
    if (!g || !key || !elem_type || !count) return QLIN_ERR_NULL;
    const Value *v = g->find(key);
    if (!v || v->type != QLIN_GGUF_ARRAY) return QLIN_ERR_NOT_FOUND;
    *elem_type = v->elem;
    *count = v->count;
    return QLIN_OK;
}

int qlin_gguf_get_array_i64(const qlin_gguf *g, const char *key, int64_t index, int64_t *out) {
    if (!g || !key || !out) return QLIN_ERR_NULL;
    const Value *v = g->find(key);
    if (!v || v->type != QLIN_GGUF_ARRAY || index < 0 || index >= static_cast<int64_t>(v->ai.size()))
        return QLIN_ERR_NOT_FOUND;
    *out = v->ai[static_cast<size_t>(index)];
    return QLIN_OK;
}

int qlin_gguf_get_array_f64(const qlin_gguf *g, const char *key, int64_t index, double *out) {
    if (!g || !key || !out) return QLIN_ERR_NULL;
    const Value *v = g->find(key);
    if (!v || v->type != QLIN_GGUF_ARRAY || index < 0 || index >= static_cast<int64_t>(v->af.size()))
        return QLIN_ERR_NOT_FOUND;
    *out = v->af[static_cast<size_t>(index)];
    return QLIN_OK;
}

int qlin_gguf_get_array_str(const qlin_gguf *g, const char *key, int64_t index, const char **out, size_t *len) {
    if (!g || !key || !out || !len) return QLIN_ERR_NULL;
    const Value *v = g->find(key);
    if (!v || v->type != QLIN_GGUF_ARRAY || index < 0 || index >= static_cast<int64_t>(v->as.size()))
        return QLIN_ERR_NOT_FOUND;
    *out = v->as[static_cast<size_t>(index)].c_str();
    *len = v->as[static_cast<size_t>(index)].size();
    return QLIN_OK;
}

int qlin_pool_create(qlin_pool **out) {
    if (!out) return QLIN_ERR_NULL;
    *out = new (std::nothrow) qlin_pool;
    return *out ? QLIN_OK : QLIN_ERR_ALLOC;
}

void qlin_pool_destroy(qlin_pool *p) { delete p; }

uint64_t qlin_pool_resident_bytes(const qlin_pool *p) { return p ? p->resident : 0; }

int qlin_pool_weight(qlin_pool *p, const qlin_gguf *g, const char *name, void **dev, uint64_t *nbytes) {
    if (!p || !g || !name || !dev || !nbytes) return QLIN_ERR_NULL;
    const int64_t idx = qlin_gguf_find_tensor(g, name);
    if (idx < 0) return QLIN_ERR_NOT_FOUND;
    const Tensor &t = g->tensors[static_cast<size_t>(idx)];
    auto it = p->items.find(t.name);
    if (it == p->items.end()) {
        qlin_pool::Entry e;
        e.bytes = t.nbytes;
        if (hipMalloc(&e.dev, t.nbytes ? t.nbytes : 1) != hipSuccess) return QLIN_ERR_ALLOC;
        if (!upload(e.dev, t.data, t.nbytes)) {
            (void)hipFree(e.dev);
            return QLIN_ERR_ALLOC;
        }
        p->resident += t.nbytes;
        it = p->items.emplace(t.name, e).first;
    }
    *dev = it->second.dev;
    *nbytes = it->second.bytes;
    return QLIN_OK;
}

int qlin_pool_expert_view(qlin_pool *p, const qlin_gguf *g, const char *name, int expert, void **dev,
                          uint64_t *expert_bytes, int64_t *rows, int64_t *cols) {
    if (!p || !g || !name || !dev || !expert_bytes || !rows || !cols) return QLIN_ERR_NULL;
    const int64_t idx = qlin_gguf_find_tensor(g, name);
    if (idx < 0) return QLIN_ERR_NOT_FOUND;
    const Tensor &t = g->tensors[static_cast<size_t>(idx)];
    // packed experts [E, rows, cols] (the file's dims [cols, rows, E])
    if (t.n_dims != 3 || t.shape[0] <= 0 || t.nbytes % static_cast<uint64_t>(t.shape[0])) return QLIN_ERR_SHAPE;
    if (expert < 0 || expert >= t.shape[0]) return QLIN_ERR_NOT_FOUND;
    void *base;
    uint64_t total;
    const int rc = qlin_pool_weight(p, g, name, &base, &total);
    if (rc != QLIN_OK) return rc;
    const uint64_t eb = total / static_cast<uint64_t>(t.shape[0]);
    *dev = static_cast<uint8_t *>(base) + static_cast<uint64_t>(expert) * eb;
    *expert_bytes = eb;
    *rows = t.shape[1];
    *cols = t.shape[2];
    return QLIN_OK;
}

}  // extern "C"
