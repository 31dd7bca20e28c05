// gguf.cpp -- GGUF (v2/v3) container reader, host only: the header, the
// metadata key/value table, the tensor directory and the tensor bytes, with
// the semantics of the reference's GgufFile (crates/mrml-tensor/src/gguf.rs):
//  * magic "GGUF", version 2 or 3 (gguf.rs:83-92);
//  * u64 tensor and key/value counts; keys and strings are a u64 length plus
//    UTF-8 bytes (gguf.rs:190-201); value type ids 0..12, arrays nested by
//    item type (gguf.rs:203-228);
//  * a tensor entry is name, u32 n_dims, the first min(n_dims, 4) dims as u64
//    (missing dims are 1, extra dims are read and dropped), u32 type id,
//    u64 offset; its byte size is numel / block_size * type_size
//    (gguf.rs:106-151, types.rs:32-70, 179-181);
//  * tensor data starts at the end of the directory rounded up to
//    general.alignment (default 32; gguf.rs:153-163) and each tensor sits at
//    data_offset + offset (gguf.rs:174-183);
//  * both tables are ordered maps sorted by key bytes, a repeated key keeping
//    its last value (mrml-runtime map.rs:38-49).
// Lengths are checked against the file size before anything is allocated, so
// a corrupt header yields an error instead of a huge allocation.

#include <algorithm>
#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "../../include/mrml_hip.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

struct Value {
    int32_t type = 0;
    uint64_t u = 0;  // unsigned and bool payloads
    int64_t i = 0;   // signed payloads
    double f = 0.0;  // float payloads (f32 values stored exactly)
    std::string s;
    int32_t item_type = -1;
    std::vector<Value> items;
};

struct Tensor {
    std::string name;
    int32_t type = 0;
    int32_t n_dims = 0;
    uint64_t dims[4] = {1, 1, 1, 1};
    uint64_t offset = 0;
    uint64_t size_bytes = 0;
};

// types.rs:32-70 for the ids gguf.rs:121-133 accepts
bool type_layout(uint32_t id, uint64_t &block, uint64_t &bytes)
{
    switch (id) {
    case 0: block = 1, bytes = 4; return true;     // F32
    case 1: block = 1, bytes = 2; return true;     // F16
    case 2: block = 32, bytes = 18; return true;   // Q4_0
    case 3: block = 32, bytes = 20; return true;   // Q4_1
    case 8: block = 32, bytes = 34; return true;   // Q8_0
    case 12: block = 256, bytes = 144; return true;  // Q4_K
    case 13: block = 256, bytes = 176; return true;  // Q5_K
    case 14: block = 256, bytes = 210; return true;  // Q6_K
    case 16: block = 256, bytes = 136; return true;  // IQ4_XS
    case 30: block = 1, bytes = 2; return true;    // BF16
    default: return false;
    }
}

bool valid_utf8(const std::string &s)
{
    const auto *p = reinterpret_cast<const unsigned char *>(s.data());
    size_t i = 0, n = s.size();
    while (i < n) {
        const unsigned c = p[i];
        int len;
        uint32_t cp;
        if (c < 0x80) { ++i; continue; }
        if (c >= 0xC2 && c <= 0xDF) len = 2, cp = c & 0x1F;
        else if (c >= 0xE0 && c <= 0xEF) len = 3, cp = c & 0x0F;
        else if (c >= 0xF0 && c <= 0xF4) len = 4, cp = c & 0x07;
        else return false;
        if (i + len > n) return false;
        for (int k = 1; k < len; ++k) {
            const unsigned cc = p[i + k];
            if ((cc & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (cc & 0x3F);
        }
        if ((len == 3 && (cp < 0x800 || (cp >= 0xD800 && cp <= 0xDFFF))) || (len == 4 && (cp < 0x10000 || cp > 0x10FFFF)))
            return false;
        i += len;
    }
    return true;
}

class Reader {
public:
    Reader(FILE *f, uint64_t size) : f_(f), size_(size) {}
    uint64_t pos() const { return pos_; }
    uint64_t left() const { return size_ - pos_; }

    int bytes(void *dst, uint64_t n)
    {
        if (n > left()) return fail(MRML_HIP_E_FORMAT, "GGUF: unexpected end of file at byte %llu (need %llu more)",
                                    (unsigned long long)pos_, (unsigned long long)n);
        if (n && fread(dst, 1, n, f_) != n) return fail(MRML_HIP_E_IO, "GGUF: read error at byte %llu", (unsigned long long)pos_);
        pos_ += n;
        return MRML_HIP_OK;
    }
    template <class T>
    int le(T &v)
    {
        unsigned char b[sizeof(T)];
        if (int rc = bytes(b, sizeof b)) return rc;
        uint64_t x = 0;
        for (size_t k = 0; k < sizeof(T); ++k) x |= (uint64_t)b[k] << (8 * k);
        std::memcpy(&v, &x, sizeof(T));  // little-endian host
        return MRML_HIP_OK;
    }
    int str(std::string &s)
    {
        uint64_t n;
        if (int rc = le(n)) return rc;
        if (n > left()) return fail(MRML_HIP_E_FORMAT, "GGUF: string of %llu bytes at byte %llu runs past the end of file",
                                    (unsigned long long)n, (unsigned long long)pos_);
        s.resize(n);
        if (int rc = bytes(&s[0], n)) return rc;
        if (!valid_utf8(s)) return fail(MRML_HIP_E_FORMAT, "GGUF string is not valid UTF-8");
        return MRML_HIP_OK;
    }
    // Smallest encoding of one value of a type id: the scalar's width, a
    // string's u64 length, an array's u32 item type and u64 count.  An
    // unknown id counts 1 byte (it fails when the first item is read).
    static uint64_t min_encoded_bytes(uint32_t type)
    {
        switch (type) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 8: case 10: case 11: case 12: return 8;
        case 9: return 12;
        default: return 1;
        }
    }
    int value(Value &v, uint32_t type, int depth)
    {
        v.type = (int32_t)type;
        switch (type) {
        case 0: { uint8_t x; if (int rc = le(x)) return rc; v.u = x; return 0; }
        case 1: { int8_t x; if (int rc = le(x)) return rc; v.i = x; return 0; }
        case 2: { uint16_t x; if (int rc = le(x)) return rc; v.u = x; return 0; }
        case 3: { int16_t x; if (int rc = le(x)) return rc; v.i = x; return 0; }
        case 4: { uint32_t x; if (int rc = le(x)) return rc; v.u = x; return 0; }
        case 5: { int32_t x; if (int rc = le(x)) return rc; v.i = x; return 0; }
        case 6: { float x; if (int rc = le(x)) return rc; v.f = x; return 0; }
        case 7: { uint8_t x; if (int rc = le(x)) return rc; v.u = x != 0; return 0; }
        case 8: return str(v.s);
        case 9: {
            if (depth > 64) return fail(MRML_HIP_E_FORMAT, "GGUF: arrays nested deeper than 64 levels");
            uint32_t it;
            uint64_t n;
            if (int rc = le(it)) return rc;
            if (int rc = le(n)) return rc;
            v.item_type = (int32_t)it;  // an unknown item type fails at the first item, as in gguf.rs:213-219
            // Every item takes at least min_encoded_bytes(it) bytes of the
            // file, so a count the file cannot hold is an error before any
            // item is allocated, and the item list grows as items parse.
            if (n > left() / min_encoded_bytes(it))
                return fail(MRML_HIP_E_FORMAT, "GGUF: array of %llu items at byte %llu runs past the end of file",
                            (unsigned long long)n, (unsigned long long)pos_);
            v.items.clear();
            for (uint64_t k = 0; k < n; ++k) {
                v.items.emplace_back();
                if (int rc = value(v.items.back(), it, depth + 1)) return rc;
            }
            return 0;
        }
        case 10: { uint64_t x; if (int rc = le(x)) return rc; v.u = x; return 0; }
        case 11: { int64_t x; if (int rc = le(x)) return rc; v.i = x; return 0; }
        case 12: { double x; if (int rc = le(x)) return rc; v.f = x; return 0; }
        default: return fail(MRML_HIP_E_FORMAT, "Unknown GGUF value type ID: %u", type);
        }
    }

private:
    FILE *f_;
    uint64_t size_, pos_ = 0;
};

// Sorted insert, a repeated key replacing the value in place (map.rs:38-49).
template <class T>
void map_insert(std::vector<std::pair<std::string, T>> &m, const std::string &key, T &&v)
{
    auto it = std::lower_bound(m.begin(), m.end(), key,
                               [](const std::pair<std::string, T> &e, const std::string &k) { return e.first < k; });
    if (it != m.end() && it->first == key) it->second = std::move(v);
    else m.insert(it, {key, std::move(v)});
}

template <class T>
const T *map_get(const std::vector<std::pair<std::string, T>> &m, const char *key, int64_t *index = nullptr)
{
    const std::string k(key);
    auto it = std::lower_bound(m.begin(), m.end(), k,
                               [](const std::pair<std::string, T> &e, const std::string &q) { return e.first < q; });
    if (it == m.end() || it->first != k) return nullptr;
    if (index) *index = it - m.begin();
    return &it->second;
}

// GgufValue::as_u32 / as_f32 (gguf.rs:25-46): Rust `as` casts truncate the
// integers and round the f64.
bool as_u32(const Value &v, uint32_t &out)
{
    switch (v.type) {
    case 4: case 10: case 2: case 0: out = (uint32_t)v.u; return true;
    case 5: case 11: if (v.i < 0) return false; out = (uint32_t)v.i; return true;
    default: return false;
    }
}

bool as_f32(const Value &v, float &out)
{
    switch (v.type) {
    case 6: case 12: out = (float)v.f; return true;
    case 4: out = (float)(uint32_t)v.u; return true;
    default: return false;
    }
}

}  // namespace

struct mrml_gguf {
    std::string path;
    uint32_t version = 0;
    uint64_t data_offset = 0, file_size = 0;
    std::vector<std::pair<std::string, Value>> meta;
    std::vector<std::pair<std::string, Tensor>> tensors;
};

namespace {

int open_file(const char *path, mrml_gguf **out)
{
    std::unique_ptr<FILE, int (*)(FILE *)> f(fopen(path, "rb"), fclose);
    if (!f) return fail(MRML_HIP_E_IO, "GGUF: cannot open %s: %s", path, strerror(errno));
    if (fseeko(f.get(), 0, SEEK_END) != 0) return fail(MRML_HIP_E_IO, "GGUF: cannot seek %s", path);
    const off_t size = ftello(f.get());
    if (size < 0 || fseeko(f.get(), 0, SEEK_SET) != 0) return fail(MRML_HIP_E_IO, "GGUF: cannot size %s", path);
    auto g = std::make_unique<mrml_gguf>();
    g->path = path;
    g->file_size = (uint64_t)size;
    Reader r(f.get(), (uint64_t)size);
    uint32_t magic;
    if (int rc = r.le(magic)) return rc;
    if (magic != 0x46554747u) return fail(MRML_HIP_E_FORMAT, "Invalid GGUF magic number: 0x%08X", magic);
    if (int rc = r.le(g->version)) return rc;
    if (g->version < 2 || g->version > 3) return fail(MRML_HIP_E_FORMAT, "Unsupported GGUF version: %u", g->version);
    uint64_t n_tensors, n_kv;
    if (int rc = r.le(n_tensors)) return rc;
    if (int rc = r.le(n_kv)) return rc;
    for (uint64_t k = 0; k < n_kv; ++k) {
        std::string key;
        uint32_t type;
        Value v;
        if (int rc = r.str(key)) return rc;
        if (int rc = r.le(type)) return rc;
        if (int rc = r.value(v, type, 0)) return rc;
        map_insert(g->meta, key, std::move(v));
    }
    for (uint64_t k = 0; k < n_tensors; ++k) {
        Tensor t;
        uint32_t n_dims, type;
        if (int rc = r.str(t.name)) return rc;
        if (int rc = r.le(n_dims)) return rc;
        for (uint32_t d = 0; d < n_dims; ++d) {
            uint64_t x;
            if (int rc = r.le(x)) return rc;
            if (d < 4) t.dims[d] = x;
        }
        if (int rc = r.le(type)) return rc;
        uint64_t block, bytes;
        if (!type_layout(type, block, bytes)) return fail(MRML_HIP_E_FORMAT, "Unsupported GGUF dtype ID: %u", type);
        if (int rc = r.le(t.offset)) return rc;
        t.type = (int32_t)type;
        t.n_dims = (int32_t)std::min<uint32_t>(n_dims, 4);
        uint64_t numel = 1;
        for (int d = 0; d < 4; ++d) {
            if (t.dims[d] && numel > UINT64_MAX / t.dims[d])
                return fail(MRML_HIP_E_FORMAT, "GGUF: tensor %s has more than 2^64 elements", t.name.c_str());
            numel *= t.dims[d];
        }
        t.size_bytes = numel / block * bytes;
        std::string name = t.name;
        map_insert(g->tensors, name, std::move(t));
    }
    uint32_t align = 32;
    if (const Value *a = map_get(g->meta, "general.alignment")) {
        uint32_t x;
        if (as_u32(*a, x)) align = x;
    }
    if (align == 0) return fail(MRML_HIP_E_FORMAT, "GGUF: general.alignment is 0");
    const uint64_t pos = r.pos();
    g->data_offset = pos % align == 0 ? pos : pos + (align - pos % align);
    *out = g.release();
    return MRML_HIP_OK;
}

}  // namespace

extern "C" {

const char *mrml_gguf_last_error(void) { return g_last_error.c_str(); }

int mrml_gguf_open(const char *path, mrml_gguf **out)
{
    if (!path || !out) return fail(MRML_HIP_E_INVALID, "mrml_gguf_open: null argument");
    *out = nullptr;
    // The directory's strings, tables and arrays are host allocations; none
    // of their exceptions may cross the C boundary.
    try {
        return open_file(path, out);
    } catch (const std::bad_alloc &) {
        return fail(MRML_HIP_E_ALLOC, "GGUF: out of host memory reading %s", path);
    } catch (...) {
        return fail(MRML_HIP_E_FORMAT, "GGUF: unexpected error reading %s", path);
    }
}

int mrml_gguf_close(mrml_gguf *g)
{
    delete g;
    return MRML_HIP_OK;
}

int mrml_gguf_header(const mrml_gguf *g, uint32_t *version, uint64_t *data_offset, int64_t *n_tensors, int64_t *n_meta)
{
    if (!g) return fail(MRML_HIP_E_INVALID, "mrml_gguf_header: null handle");
    if (version) *version = g->version;
    if (data_offset) *data_offset = g->data_offset;
    if (n_tensors) *n_tensors = (int64_t)g->tensors.size();
    if (n_meta) *n_meta = (int64_t)g->meta.size();
    return MRML_HIP_OK;
}

int mrml_gguf_tensor(const mrml_gguf *g, int64_t index, mrml_gguf_tensor_info *info)
{
    if (!g || !info) return fail(MRML_HIP_E_INVALID, "mrml_gguf_tensor: null argument");
    if (index < 0 || index >= (int64_t)g->tensors.size())
        return fail(MRML_HIP_E_INVALID, "mrml_gguf_tensor: index %lld out of range", (long long)index);
    const Tensor &t = g->tensors[index].second;
    info->name = t.name.c_str();
    info->type = t.type;
    info->n_dims = t.n_dims;
    for (int d = 0; d < 4; ++d) info->dims[d] = t.dims[d];
    info->offset = t.offset;
    info->size_bytes = t.size_bytes;
    return MRML_HIP_OK;
}

int mrml_gguf_find_tensor(const mrml_gguf *g, const char *name, int64_t *index)
{
    if (!g || !name || !index) return fail(MRML_HIP_E_INVALID, "mrml_gguf_find_tensor: null argument");
    if (!map_get(g->tensors, name, index)) return fail(MRML_HIP_E_NOTFOUND, "GGUF: no tensor named %s", name);
    return MRML_HIP_OK;
}

int mrml_gguf_read_tensor(const mrml_gguf *g, int64_t index, void *h_dst, uint64_t dst_bytes)
{
    if (!g || !h_dst) return fail(MRML_HIP_E_INVALID, "mrml_gguf_read_tensor: null argument");
    if (index < 0 || index >= (int64_t)g->tensors.size())
        return fail(MRML_HIP_E_INVALID, "mrml_gguf_read_tensor: index %lld out of range", (long long)index);
    const Tensor &t = g->tensors[index].second;
    if (dst_bytes < t.size_bytes)
        return fail(MRML_HIP_E_INVALID, "mrml_gguf_read_tensor: %s needs %llu bytes, buffer holds %llu", t.name.c_str(),
                    (unsigned long long)t.size_bytes, (unsigned long long)dst_bytes);
    const uint64_t start = g->data_offset + t.offset;
    if (start < g->data_offset || start > g->file_size || t.size_bytes > g->file_size - start)
        return fail(MRML_HIP_E_FORMAT, "GGUF: tensor %s (bytes %llu..%llu) lies past the end of the %llu-byte file",
                    t.name.c_str(), (unsigned long long)start, (unsigned long long)(start + t.size_bytes),
                    (unsigned long long)g->file_size);
    std::unique_ptr<FILE, int (*)(FILE *)> f(fopen(g->path.c_str(), "rb"), fclose);
    if (!f) return fail(MRML_HIP_E_IO, "GGUF: cannot open %s: %s", g->path.c_str(), strerror(errno));
    if (fseeko(f.get(), (off_t)start, SEEK_SET) != 0 || fread(h_dst, 1, t.size_bytes, f.get()) != t.size_bytes)
        return fail(MRML_HIP_E_IO, "GGUF: short read of tensor %s", t.name.c_str());
    return MRML_HIP_OK;
}

int mrml_gguf_meta_key(const mrml_gguf *g, int64_t index, const char **key, int32_t *type)
{
    if (!g || !key) return fail(MRML_HIP_E_INVALID, "mrml_gguf_meta_key: null argument");
    if (index < 0 || index >= (int64_t)g->meta.size())
        return fail(MRML_HIP_E_INVALID, "mrml_gguf_meta_key: index %lld out of range", (long long)index);
    *key = g->meta[index].first.c_str();
    if (type) *type = g->meta[index].second.type;
    return MRML_HIP_OK;
}

static int meta_lookup(const mrml_gguf *g, const char *key, const Value *&v)
{
    if (!g || !key) return fail(MRML_HIP_E_INVALID, "GGUF metadata lookup: null argument");
    v = map_get(g->meta, key);
    if (!v) return fail(MRML_HIP_E_NOTFOUND, "GGUF: no metadata key %s", key);
    return MRML_HIP_OK;
}

int mrml_gguf_meta_u32(const mrml_gguf *g, const char *key, uint32_t *out)
{
    const Value *v;
    if (int rc = meta_lookup(g, key, v)) return rc;
    if (!out || !as_u32(*v, *out)) return fail(MRML_HIP_E_INVALID, "GGUF: %s (type %d) is not a u32", key, v->type);
    return MRML_HIP_OK;
}

int mrml_gguf_meta_f32(const mrml_gguf *g, const char *key, float *out)
{
    const Value *v;
    if (int rc = meta_lookup(g, key, v)) return rc;
    if (!out || !as_f32(*v, *out)) return fail(MRML_HIP_E_INVALID, "GGUF: %s (type %d) is not an f32", key, v->type);
    return MRML_HIP_OK;
}

int mrml_gguf_meta_str(const mrml_gguf *g, const char *key, const char **out, uint64_t *len)
{
    const Value *v;
    if (int rc = meta_lookup(g, key, v)) return rc;
    if (!out || v->type != 8) return fail(MRML_HIP_E_INVALID, "GGUF: %s (type %d) is not a string", key, v->type);
    *out = v->s.c_str();
    if (len) *len = v->s.size();
    return MRML_HIP_OK;
}

int mrml_gguf_meta_array(const mrml_gguf *g, const char *key, int32_t *item_type, uint64_t *len)
{
    const Value *v;
    if (int rc = meta_lookup(g, key, v)) return rc;
    if (v->type != 9) return fail(MRML_HIP_E_INVALID, "GGUF: %s (type %d) is not an array", key, v->type);
    if (item_type) *item_type = v->item_type;
    if (len) *len = v->items.size();
    return MRML_HIP_OK;
}

}  // extern "C"
