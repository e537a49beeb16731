// fgh_gguf.hip - GGUF file ingestion for the device path (host code only): maps a GGUF file
// read-only, parses its header, metadata and tensor table with the rules of the reference's
// gguf_open (fastgguf.c:342-440), and uploads a tensor of it through fgh_upload, the way
// gpu_upload_tensor (2060-2081) uploads a tensor_t that points into the mapped file.
//
// Layout read (GGUF v2/v3, little-endian): "GGUF", u32 version, u64 tensor count, u64 metadata
// count; metadata entries {string key, u32 value type, value}; tensor infos {string name, u32
// n_dims, u64 dims[n_dims], u32 type, u64 offset}; then the data section at the next multiple of
// general.alignment (default 32), each tensor at data start + its offset. Strings are u64 length
// + bytes. Value types: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 8 string, 9 array
// (u32 element type, u64 count, elements), 10 u64, 11 i64, 12 f64.
//
// Kept from the reference: what fails an open (no "GGUF" magic or fewer than 16 bytes, a
// truncated metadata or tensor table, an unknown value type, a tensor type without a block size,
// a tensor extending past the end of the file); a tensor's byte count ceil(elements / block
// elements) * block bytes (tensor_nbytes, 255-259); alignment from a positive numeric
// general.alignment; keys kept to 95 characters and names to 127 (the reference's fixed buffers,
// so lookups see the same strings); kv_num's answer for numbers and integer arrays (441-448).
// Added: element counts are checked against the file size before anything is allocated, and a
// tensor with more than 4 dimensions fails the open (the reference reads only 4 and then
// misreads the rest of its entry).
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <vector>

#include "fastgguf_hip.h"

namespace {

struct Kv {
    std::string key;
    int kind = 0;  // 0 number, 1 string, 2 integer array, 3 string array
    double num = 0.0;
    std::string str;
    std::vector<int> iarr;
};

// bytes per block and elements per block of a GGML type (block_size_of, fastgguf.c:235-253)
bool block_size_of(uint32_t t, uint64_t *elems, uint64_t *bytes) {
    switch (t) {
    case 0: *elems = 1; *bytes = 4; return true;                 // F32
    case 1: case 30: *elems = 1; *bytes = 2; return true;        // F16, BF16
    case 2: *elems = 32; *bytes = 18; return true;               // Q4_0
    case 3: *elems = 32; *bytes = 20; return true;               // Q4_1
    case 6: *elems = 32; *bytes = 22; return true;               // Q5_0
    case 7: *elems = 32; *bytes = 24; return true;               // Q5_1
    case 8: *elems = 32; *bytes = 34; return true;               // Q8_0
    case 10: *elems = 256; *bytes = 84; return true;             // Q2_K
    case 11: *elems = 256; *bytes = 110; return true;            // Q3_K
    case 12: *elems = 256; *bytes = 144; return true;            // Q4_K
    case 13: *elems = 256; *bytes = 176; return true;            // Q5_K
    case 14: *elems = 256; *bytes = 210; return true;            // Q6_K
    case 20: *elems = 32; *bytes = 18; return true;              // IQ4_NL
    case 23: *elems = 256; *bytes = 136; return true;            // IQ4_XS
    default: return false;
    }
}

// bounds-checked little-endian reader over the mapped file; any overrun sets err
struct Reader {
    const uint8_t *b;
    uint64_t pos, size;
    bool err = false;
    bool need(uint64_t n) {
        if (err || n > size - pos) err = true;
        return !err;
    }
    template <typename T>
    T get() {
        T v{};
        if (need(sizeof(T))) {
            memcpy(&v, b + pos, sizeof(T));
            pos += sizeof(T);
        }
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!need(n)) return std::string();
        std::string s((const char *)b + pos, (size_t)n);
        pos += n;
        return s;
    }
    // one scalar of value type vt as a double (read_scalar, fastgguf.c:322-338)
    double scalar(uint32_t vt) {
        switch (vt) {
        case 0: return (double)get<uint8_t>();
        case 1: return (double)get<int8_t>();
        case 2: return (double)get<uint16_t>();
        case 3: return (double)get<int16_t>();
        case 4: return (double)get<uint32_t>();
        case 5: return (double)get<int32_t>();
        case 6: return (double)get<float>();
        case 7: return (double)get<uint8_t>();
        case 10: return (double)get<uint64_t>();
        case 11: return (double)get<int64_t>();
        case 12: return get<double>();
        default: err = true; return 0.0;
        }
    }
};

std::string clip(const std::string &s, size_t n) { return s.size() > n ? s.substr(0, n) : s; }

}  // namespace

struct fgh_gguf {
    int fd = -1;
    const uint8_t *data = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32;
    std::vector<Kv> kvs;
    std::vector<fgh_gguf_tensor_info> tensors;
    ~fgh_gguf() {
        if (data) munmap((void *)data, size);
        if (fd >= 0) close(fd);
    }
};

static int gguf_fail(char *err, size_t err_len, int rc, const char *fmt, ...) {
    if (err && err_len) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(err, err_len, fmt, ap);
        va_end(ap);
    }
    return rc;
}

extern "C" {

int fgh_gguf_open(const char *path, fgh_gguf **out, char *err, size_t err_len) {
    if (!out) return FGH_ERR_ARG;
    *out = nullptr;
    if (err && err_len) err[0] = 0;
    if (!path) return gguf_fail(err, err_len, FGH_ERR_ARG, "no path");
    fgh_gguf *g = new fgh_gguf();
    auto bail = [&](const char *fmt, const char *arg) {
        char m[256];
        snprintf(m, sizeof(m), fmt, arg);
        delete g;
        return gguf_fail(err, err_len, FGH_ERR_ARG, "%s", m);
    };
    g->fd = open(path, O_RDONLY);
    if (g->fd < 0) return bail("cannot open %s", path);
    struct stat st;
    if (fstat(g->fd, &st) != 0) return bail("cannot open %s", path);
    g->size = (uint64_t)st.st_size;
    if (g->size < 16) return bail("%s: not a GGUF file", path);
    void *m = mmap(nullptr, (size_t)g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) return bail("cannot map %s", path);
    g->data = (const uint8_t *)m;
    if (memcmp(g->data, "GGUF", 4) != 0) return bail("%s: not a GGUF file", path);

    Reader r{g->data, 4, g->size};
    g->version = r.get<uint32_t>();
    const uint64_t n_tensors = r.get<uint64_t>();
    const uint64_t n_kvs = r.get<uint64_t>();
    // every entry takes at least 12 (metadata) or 24 (tensor) bytes of the file
    if (n_kvs > g->size / 12 || n_tensors > g->size / 24) return bail("%s: metadata parse error", path);

    g->kvs.resize((size_t)n_kvs);
    for (uint64_t i = 0; i < n_kvs && !r.err; i++) {
        Kv &kv = g->kvs[(size_t)i];
        kv.key = clip(r.str(), 95);
        const uint32_t vt = r.get<uint32_t>();
        if (vt == 8) {
            kv.kind = 1;
            kv.str = r.str();
        } else if (vt == 9) {
            const uint32_t et = r.get<uint32_t>();
            const uint64_t n = r.get<uint64_t>();
            if (r.err || n > g->size - r.pos) {  // each element takes at least a byte
                r.err = true;
                break;
            }
            if (et == 8) {
                kv.kind = 3;
                for (uint64_t j = 0; j < n && !r.err; j++) r.str();
                kv.num = (double)n;
            } else if (et == 4 || et == 5 || et == 7 || et == 0 || et == 1) {
                kv.kind = 2;
                kv.iarr.reserve((size_t)n);
                for (uint64_t j = 0; j < n && !r.err; j++) kv.iarr.push_back((int)r.scalar(et));
            } else {  // an array of another type: skipped, its length kept as the value
                kv.kind = 0;
                kv.num = (double)n;
                for (uint64_t j = 0; j < n && !r.err; j++) r.scalar(et);
            }
        } else {
            kv.kind = 0;
            kv.num = r.scalar(vt);
        }
    }
    if (r.err) return bail("%s: metadata parse error", path);
    for (const Kv &kv : g->kvs)
        if (kv.key == "general.alignment" && kv.kind == 0 && kv.num > 0) {
            // the reference divides by (uint64_t)kv_num: a value below 1 would be a division by
            // zero there, and one past 2^32 makes the data start overflow; both are refused
            if (!(kv.num >= 1.0 && kv.num <= 4294967296.0)) return bail("%s: bad general.alignment", path);
            g->alignment = (uint64_t)kv.num;
        }

    g->tensors.resize((size_t)n_tensors);
    std::vector<uint64_t> offsets((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors && !r.err; i++) {
        fgh_gguf_tensor_info &t = g->tensors[(size_t)i];
        memset(&t, 0, sizeof(t));
        const std::string name = clip(r.str(), 127);
        memcpy(t.name, name.data(), name.size());
        const uint32_t nd = r.get<uint32_t>();
        if (r.err) break;
        if (nd > 4) return bail("tensor %s: more than 4 dimensions", t.name);
        t.n_dims = (int32_t)nd;
        uint64_t elems = 1;
        bool wraps = false;
        for (uint32_t j = 0; j < nd; j++) {
            t.ne[j] = r.get<uint64_t>();
            wraps |= __builtin_mul_overflow(elems, t.ne[j], &elems);
        }
        if (wraps && !r.err) return bail("tensor %s: element count overflows", t.name);
        t.type = r.get<uint32_t>();
        offsets[(size_t)i] = r.get<uint64_t>();
        if (r.err) break;
        uint64_t be, bb;
        if (!block_size_of(t.type, &be, &bb)) {
            char m2[64];
            snprintf(m2, sizeof(m2), "unsupported type %u", t.type);
            delete g;
            return gguf_fail(err, err_len, FGH_ERR_ARG, "tensor %s: %s", name.c_str(), m2);
        }
        if (__builtin_mul_overflow(elems / be + (elems % be != 0), bb, &t.nbytes))
            return bail("tensor %s: byte count overflows", t.name);
    }
    if (r.err) return bail("%s: tensor header parse error", path);

    const uint64_t data_start = (r.pos + g->alignment - 1) / g->alignment * g->alignment;
    for (size_t i = 0; i < g->tensors.size(); i++) {
        fgh_gguf_tensor_info &t = g->tensors[i];
        t.offset = data_start + offsets[i];
        if (offsets[i] > g->size || t.offset > g->size || t.nbytes > g->size - t.offset)
            return bail("tensor %s extends past EOF", t.name);
    }
    *out = g;
    return FGH_OK;
}

void fgh_gguf_close(fgh_gguf *g) { delete g; }

int fgh_gguf_summary(const fgh_gguf *g, uint32_t *version, uint64_t *alignment, int64_t *n_kvs,
                     int64_t *n_tensors) {
    if (!g) return FGH_ERR_ARG;
    if (version) *version = g->version;
    if (alignment) *alignment = g->alignment;
    if (n_kvs) *n_kvs = (int64_t)g->kvs.size();
    if (n_tensors) *n_tensors = (int64_t)g->tensors.size();
    return FGH_OK;
}

int fgh_gguf_tensor(const fgh_gguf *g, int64_t index, fgh_gguf_tensor_info *out) {
    if (!g || !out || index < 0 || index >= (int64_t)g->tensors.size()) return FGH_ERR_ARG;
    *out = g->tensors[(size_t)index];
    return FGH_OK;
}

int64_t fgh_gguf_find(const fgh_gguf *g, const char *name) {
    if (!g || !name) return -1;
    for (size_t i = 0; i < g->tensors.size(); i++)
        if (strcmp(g->tensors[i].name, name) == 0) return (int64_t)i;
    return -1;
}

int fgh_gguf_kv_num(const fgh_gguf *g, const char *key, double def, double *out) {
    if (!g || !key || !out) return FGH_ERR_ARG;
    *out = def;
    for (const Kv &kv : g->kvs)
        if (kv.key == key) {  // the first entry of that key, as kv_find
            if (kv.kind == 0) *out = kv.num;
            else if (kv.kind == 2 && !kv.iarr.empty()) *out = (double)kv.iarr[0];
            break;
        }
    return FGH_OK;
}

const char *fgh_gguf_kv_str(const fgh_gguf *g, const char *key) {
    if (!g || !key) return nullptr;
    for (const Kv &kv : g->kvs)
        if (kv.key == key) return kv.kind == 1 ? kv.str.c_str() : nullptr;
    return nullptr;
}

const void *fgh_gguf_data(const fgh_gguf *g, int64_t index) {
    if (!g || index < 0 || index >= (int64_t)g->tensors.size()) return nullptr;
    return g->data + g->tensors[(size_t)index].offset;
}

int fgh_upload_gguf(fgh_ctx *ctx, const fgh_gguf *g, int64_t index, int order, fgh_tensor **out) {
    if (!ctx || !out) return FGH_ERR_ARG;
    *out = nullptr;
    if (!g || index < 0 || index >= (int64_t)g->tensors.size()) return FGH_ERR_ARG;
    const fgh_gguf_tensor_info &t = g->tensors[(size_t)index];
    const int64_t cols = (int64_t)t.ne[0];
    const int64_t rows = t.n_dims >= 2 ? (int64_t)t.ne[1] : 1;
    int64_t n_mats = 1;
    for (int j = 2; j < t.n_dims; j++) n_mats *= (int64_t)t.ne[j];
    return fgh_upload(ctx, t.type, cols, rows, n_mats, order, g->data + t.offset, t.nbytes, out);
}

}  // extern "C"
