// GGUF v3 reader: the file is memory-mapped read-only; the header, the
// key/value metadata and the tensor table are parsed, and tensor data is
// handed out as pointers into the mapping (never copied or repacked: the
// GEMV kernels read GGUF blocks as they lie).  Replaces the reference's
// k0/gguf.h:30-246 (File::open / parse / find / find_kv) with K-quant types
// (Q4_K, Q6_K, Q8_K), Q8_0, BF16 and the integer types added to its
// type-size table.  Every malformed input -- bad magic or version, a
// truncated header, a tensor of unknown type, a row not a whole number of
// blocks, misaligned or out-of-file data -- is rejected with
// SINTER_ERR_ARG and a message; nothing is read past the end of the file.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "internal.h"

using namespace sinter;

namespace {

// ggml type id -> (elements per block, bytes per block); 0 = unknown
struct TypeSize { uint32_t elems, bytes; };
TypeSize type_size(uint32_t t) {
    switch (t) {
    case 0: return {1, 4};       // F32
    case 1: return {1, 2};       // F16
    case 2: return {32, 18};     // Q4_0
    case 3: return {32, 20};     // Q4_1
    case 6: return {32, 22};     // Q5_0
    case 7: return {32, 24};     // Q5_1
    case 8: return {32, 34};     // Q8_0
    case 10: return {256, 84};   // Q2_K
    case 11: return {256, 110};  // Q3_K
    case 12: return {256, 144};  // Q4_K
    case 13: return {256, 176};  // Q5_K
    case 14: return {256, 210};  // Q6_K
    case 15: return {256, 292};  // Q8_K
    case 24: return {1, 1};      // I8
    case 25: return {1, 2};      // I16
    case 26: return {1, 4};      // I32
    case 27: return {1, 8};      // I64
    case 28: return {1, 8};      // F64
    case 30: return {1, 2};      // BF16
    default: return {0, 0};
    }
}

// metadata value kinds (GGUF v3)
enum : uint32_t { K_U8 = 0, K_I8, K_U16, K_I16, K_U32, K_I32, K_F32, K_BOOL, K_STRING, K_ARRAY, K_U64, K_I64, K_F64 };

struct KV {
    uint32_t kind = 0, arr_kind = 0;
    int64_t i = 0;
    double f = 0.0;
    std::string s;
    std::vector<int64_t> ai;
    std::vector<double> af;
    std::vector<std::string> as;
};

}  // namespace

struct sinter_gguf {
    int fd = -1;
    const uint8_t *map = nullptr;
    uint64_t size = 0, cur = 0;
    uint32_t version = 0;
    uint64_t alignment = 32;
    const uint8_t *data = nullptr;
    std::map<std::string, KV> kv;
    std::vector<std::string> names;
    std::vector<sinter_gguf_tensor> tensors;
    std::map<std::string, size_t> by_name;
    std::string err;

    ~sinter_gguf() {
        if (map) munmap((void *)map, size);
        if (fd >= 0) close(fd);
    }
    bool need(uint64_t n) {
        if (n > size || cur > size - n) {
            err = "truncated file (need " + std::to_string(n) + " bytes at offset " + std::to_string(cur) + ")";
            return false;
        }
        return true;
    }
    template <class T>
    bool rd(T &v) {
        if (!need(sizeof(T))) return false;
        std::memcpy(&v, map + cur, sizeof(T));
        cur += sizeof(T);
        return true;
    }
    bool rd_str(std::string &s) {
        uint64_t n = 0;
        if (!rd(n) || !need(n)) return false;
        s.assign((const char *)map + cur, n);
        cur += n;
        return true;
    }
    bool rd_scalar(uint32_t k, KV &v) {
        switch (k) {
        case K_U8: { uint8_t x; if (!rd(x)) return false; v.i = x; return true; }
        case K_I8: { int8_t x; if (!rd(x)) return false; v.i = x; return true; }
        case K_U16: { uint16_t x; if (!rd(x)) return false; v.i = x; return true; }
        case K_I16: { int16_t x; if (!rd(x)) return false; v.i = x; return true; }
        case K_U32: { uint32_t x; if (!rd(x)) return false; v.i = x; return true; }
        case K_I32: { int32_t x; if (!rd(x)) return false; v.i = x; return true; }
        case K_U64: { uint64_t x; if (!rd(x)) return false; v.i = (int64_t)x; return true; }
        case K_I64: { int64_t x; if (!rd(x)) return false; v.i = x; return true; }
        case K_F32: { float x; if (!rd(x)) return false; v.f = x; return true; }
        case K_F64: { double x; if (!rd(x)) return false; v.f = x; return true; }
        case K_BOOL: { uint8_t x; if (!rd(x)) return false; v.i = x != 0; return true; }
        case K_STRING: return rd_str(v.s);
        default: err = "unknown metadata value kind " + std::to_string(k); return false;
        }
    }
    bool parse() {
        uint32_t magic = 0;
        uint64_t n_tensors = 0, n_kv = 0;
        if (!rd(magic)) return false;
        if (magic != 0x46554747u) { err = "bad magic (not a GGUF file)"; return false; }
        if (!rd(version)) return false;
        if (version != 3) { err = "GGUF version " + std::to_string(version) + " (only v3 is read)"; return false; }
        if (!rd(n_tensors) || !rd(n_kv)) return false;
        // every table entry takes at least 8 bytes: reject absurd counts
        // before reserving anything
        if (n_tensors > size / 8 || n_kv > size / 8) { err = "tensor/kv count larger than the file"; return false; }
        for (uint64_t k = 0; k < n_kv; k++) {
            std::string key;
            KV v;
            if (!rd_str(key) || !rd(v.kind)) return false;
            if (v.kind == K_ARRAY) {
                uint64_t n = 0;
                if (!rd(v.arr_kind) || !rd(n)) return false;
                if (v.arr_kind == K_ARRAY) { err = "nested metadata arrays"; return false; }
                if (n > size) { err = "metadata array longer than the file"; return false; }
                for (uint64_t j = 0; j < n; j++) {
                    KV e;
                    if (!rd_scalar(v.arr_kind, e)) return false;
                    if (v.arr_kind == K_STRING) v.as.push_back(e.s);
                    else if (v.arr_kind == K_F32 || v.arr_kind == K_F64) v.af.push_back(e.f);
                    else v.ai.push_back(e.i);
                }
            } else if (!rd_scalar(v.kind, v)) {
                return false;
            }
            kv[key] = std::move(v);
        }
        auto a = kv.find("general.alignment");
        if (a != kv.end()) {
            if (a->second.kind == K_F32 || a->second.kind == K_F64 || a->second.kind == K_STRING ||
                a->second.i <= 0 || (a->second.i & (a->second.i - 1)) != 0) {
                err = "general.alignment is not a power of two";
                return false;
            }
            alignment = (uint64_t)a->second.i;
        }
        names.resize(n_tensors);
        tensors.resize(n_tensors);
        for (uint64_t t = 0; t < n_tensors; t++) {
            sinter_gguf_tensor &ti = tensors[t];
            std::memset(&ti, 0, sizeof ti);
            if (!rd_str(names[t]) || !rd(ti.n_dims)) return false;
            if (ti.n_dims < 1 || ti.n_dims > 4) { err = "tensor " + names[t] + ": n_dims out of range"; return false; }
            for (int d = 0; d < 4; d++) ti.ne[d] = 1;
            for (uint32_t d = 0; d < ti.n_dims; d++)
                if (!rd(ti.ne[d])) return false;
            // as ggml's reader: every dimension at least 1 and at most INT64_MAX
            for (int d = 0; d < 4; d++)
                if (ti.ne[d] == 0 || ti.ne[d] > (uint64_t)INT64_MAX) {
                    err = "tensor " + names[t] + ": dimension " + std::to_string(d) + " is 0 or exceeds INT64_MAX";
                    return false;
                }
            if (!rd(ti.type) || !rd(ti.offset)) return false;
            const TypeSize ts = type_size(ti.type);
            if (!ts.elems) { err = "tensor " + names[t] + ": unknown type id " + std::to_string(ti.type); return false; }
            if (ti.ne[0] % ts.elems) { err = "tensor " + names[t] + ": row not a whole number of blocks"; return false; }
            // nbytes = ne0/elems*bytes * ne1*ne2*ne3, refused as soon as a
            // partial product exceeds the file (each factor is below 2^63, so
            // a partial product of at most the file size times one factor
            // fits the 128-bit accumulator and cannot wrap)
            unsigned __int128 nb = (unsigned __int128)(ti.ne[0] / ts.elems) * ts.bytes;
            bool fits = nb <= size;
            for (int d = 1; d < 4 && fits; d++) {
                nb *= ti.ne[d];
                fits = nb <= size;
            }
            if (!fits) { err = "tensor " + names[t] + ": larger than the file"; return false; }
            ti.nbytes = (uint64_t)nb;
            if (by_name.count(names[t])) { err = "duplicate tensor name " + names[t]; return false; }
            by_name[names[t]] = t;
        }
        const uint64_t start = (cur + alignment - 1) & ~(alignment - 1);
        if (start > size) { err = "data section starts past the end of the file"; return false; }
        data = map + start;
        const uint64_t dsize = size - start;
        for (uint64_t t = 0; t < n_tensors; t++) {
            sinter_gguf_tensor &ti = tensors[t];
            if (ti.offset % alignment) { err = "tensor " + names[t] + ": data offset not aligned"; return false; }
            if (ti.offset > dsize || ti.nbytes > dsize - ti.offset) {
                err = "tensor " + names[t] + ": data past the end of the file";
                return false;
            }
            ti.data = data + ti.offset;
            ti.name = names[t].c_str();
        }
        return true;
    }
    const KV *find_kv(const char *key) const {
        if (!key) return nullptr;
        auto it = kv.find(key);
        return it == kv.end() ? nullptr : &it->second;
    }
};

extern "C" {

int sinter_gguf_open(const char *path, sinter_gguf **out) {
    if (!path || !out) return set_error(SINTER_ERR_ARG, "gguf_open: null argument");
    *out = nullptr;
    sinter_gguf *g = new sinter_gguf();
    g->fd = open(path, O_RDONLY);
    if (g->fd < 0) {
        delete g;
        return set_error(SINTER_ERR_ARG, "gguf_open: cannot open %s", path);
    }
    struct stat st;
    if (fstat(g->fd, &st) != 0 || st.st_size <= 0) {
        delete g;
        return set_error(SINTER_ERR_ARG, "gguf_open: cannot stat %s (or it is empty)", path);
    }
    g->size = (uint64_t)st.st_size;
    void *p = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (p == MAP_FAILED) {
        delete g;
        return set_error(SINTER_ERR_ARG, "gguf_open: mmap of %s failed", path);
    }
    g->map = (const uint8_t *)p;
    if (!g->parse()) {
        const std::string e = g->err;
        delete g;
        return set_error(SINTER_ERR_ARG, "gguf_open: %s: %s", path, e.c_str());
    }
    *out = g;
    return SINTER_OK;
}

void sinter_gguf_close(sinter_gguf *g) { delete g; }

int sinter_gguf_info(sinter_gguf *g, uint32_t *version, uint64_t *n_tensors, uint64_t *n_kv, uint64_t *alignment) {
    if (!g) return set_error(SINTER_ERR_ARG, "gguf_info: null handle");
    if (version) *version = g->version;
    if (n_tensors) *n_tensors = g->tensors.size();
    if (n_kv) *n_kv = g->kv.size();
    if (alignment) *alignment = g->alignment;
    return SINTER_OK;
}

int sinter_gguf_get_tensor(sinter_gguf *g, uint64_t i, sinter_gguf_tensor *out) {
    if (!g || !out || i >= g->tensors.size()) return set_error(SINTER_ERR_ARG, "gguf_tensor: index out of range");
    *out = g->tensors[i];
    return SINTER_OK;
}

int64_t sinter_gguf_find(sinter_gguf *g, const char *name) {
    if (!g || !name) return -1;
    auto it = g->by_name.find(name);
    return it == g->by_name.end() ? -1 : (int64_t)it->second;
}

int sinter_gguf_kv_i64(sinter_gguf *g, const char *key, int64_t *out) {
    const KV *v = g ? g->find_kv(key) : nullptr;
    if (!v) return set_error(SINTER_ERR_ARG, "gguf: no key %s", key ? key : "(null)");
    if (v->kind == K_STRING || v->kind == K_ARRAY || v->kind == K_F32 || v->kind == K_F64)
        return set_error(SINTER_ERR_ARG, "gguf: key %s is not an integer", key);
    if (out) *out = v->i;
    return SINTER_OK;
}

int sinter_gguf_kv_f64(sinter_gguf *g, const char *key, double *out) {
    const KV *v = g ? g->find_kv(key) : nullptr;
    if (!v) return set_error(SINTER_ERR_ARG, "gguf: no key %s", key ? key : "(null)");
    if (v->kind == K_STRING || v->kind == K_ARRAY) return set_error(SINTER_ERR_ARG, "gguf: key %s is not a number", key);
    if (out) *out = (v->kind == K_F32 || v->kind == K_F64) ? v->f : (double)v->i;
    return SINTER_OK;
}

int sinter_gguf_kv_str(sinter_gguf *g, const char *key, char *buf, size_t n) {
    const KV *v = g ? g->find_kv(key) : nullptr;
    if (!v) return set_error(SINTER_ERR_ARG, "gguf: no key %s", key ? key : "(null)");
    if (v->kind != K_STRING) return set_error(SINTER_ERR_ARG, "gguf: key %s is not a string", key);
    if (!buf || n <= v->s.size()) return set_error(SINTER_ERR_ARG, "gguf: buffer too small for %s", key);
    std::memcpy(buf, v->s.c_str(), v->s.size() + 1);
    return SINTER_OK;
}

int sinter_gguf_kv_arr_i64(sinter_gguf *g, const char *key, int64_t *out, size_t cap, size_t *n) {
    const KV *v = g ? g->find_kv(key) : nullptr;
    if (!v) return set_error(SINTER_ERR_ARG, "gguf: no key %s", key ? key : "(null)");
    if (v->kind != K_ARRAY || v->arr_kind == K_STRING || v->arr_kind == K_F32 || v->arr_kind == K_F64)
        return set_error(SINTER_ERR_ARG, "gguf: key %s is not an integer array", key);
    if (n) *n = v->ai.size();
    for (size_t j = 0; j < v->ai.size() && j < cap && out; j++) out[j] = v->ai[j];
    return SINTER_OK;
}

}  // extern "C"
