// GGUF reader and raw-block weight loader (host code).
//
// Replaces the load path GgufFile::open -> parse (src/model/inference/gguf.rs:1357-1364,
// 1658-2032) -> get_tensor_data_by_ref (:2062-2110) -> quant::dequantize, driven by
// QuantizedWeightLoader::load_tensor{,_data} (quant_loader.rs:66-92), which
// dequantizes every projection to f32 at load.  Here the file is mapped once, tensor
// bytes are handed out as views of the mapping, and a Q4_0 / Q8_0 projection goes to
// the GPU as its raw blocks (repacked there, never dequantized).
//
// Two on-disk dialects:
//   * the reference's: value, array-element and tensor types are one byte each
//     (gguf.rs:1795-1797, 1843-1845, 2009-2011) and tensor offsets are absolute file
//     offsets (:2037, :2064); no alignment is applied.  Its own fixtures are written
//     this way (gguf.rs:2687-2752).
//   * standard GGUF (v2/v3): those types are uint32 and tensor offsets are relative to
//     the data section, which starts at the end of the tensor infos rounded up to
//     `general.alignment` (default 32).
// AUTO tries the standard layout and falls back to the reference's when the file does
// not parse or its tensors do not fit in it.
//
// Every read is bounds-checked against the mapping: a malformed file is an error
// (status + message), never a crash.  The reference's messages are kept where it has
// them ("File too small", "Invalid GGUF magic number", "Unexpected EOF", "String too
// long", "Invalid UTF-8 string", "Unknown value type", "Too many dimensions", "Unknown
// tensor type", "Tensor data out of bounds", "Tensor not found").
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

#include "qmm_internal.hpp"

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF", gguf.rs:42
constexpr size_t kMaxString = 1024 * 1024;  // gguf.rs:1777
constexpr uint32_t kMaxDims = 8;            // gguf.rs:1996
enum : int { kU8 = 0, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kString, kArray, kU64, kI64, kF64 };

struct Value {
    int type = -1;
    uint64_t u = 0;  // unsigned / bool
    int64_t i = 0;   // signed
    double f = 0.0;  // float
    std::string s;
    std::vector<Value> arr;
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    int type = 0;
    uint64_t offset = 0;  // absolute file offset of the data
};

// GgufTensorType::{block_size, bytes_per_block} (gguf.rs:348-379) for every id
// GgufTensorType::from_u8 accepts; 0 = unknown id.
void type_geometry(int t, uint64_t* bs, uint64_t* bpb) {
    static const int kTable[][3] = {
        {0, 1, 4},     {1, 1, 2},      {2, 32, 18},    {3, 32, 20},   {4, 32, 18},   {5, 32, 20},
        {7, 32, 34},   {8, 32, 36},    {10, 256, 68},  {11, 256, 162}, {12, 256, 144}, {13, 256, 176},
        {14, 256, 210}, {15, 256, 258}, {16, 256, 64},  {17, 256, 64},  {18, 256, 96},  {19, 256, 132},
        {20, 256, 130}, {21, 256, 96},  {22, 256, 64},  {23, 256, 130}, {24, 1, 1},     {25, 1, 2},
        {26, 1, 4},    {27, 1, 8},     {28, 1, 8},     {29, 1, 2}};
    for (const auto& r : kTable)
        if (r[0] == t) {
            *bs = (uint64_t)r[1];
            *bpb = (uint64_t)r[2];
            return;
        }
    *bs = *bpb = 0;
}

}  // namespace

struct openmini_qmm_gguf {
    int dialect = 0;
    const uint8_t* base = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t tensor_count = 0;
    uint64_t kv_count = 0;
    uint32_t alignment = 0;  // standard dialect only
    std::vector<std::string> keys;                       // file order
    std::unordered_map<std::string, Value> kv;           // last definition wins (HashMap insert)
    std::vector<Tensor> tensors;                          // file order
    std::unordered_map<std::string, size_t> by_name;      // last definition wins
};

namespace {

thread_local std::string g_gguf_error;

int gfail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    qmm::set_last_error(buf);
    return code;
}

// Bounds-checked little-endian cursor over the mapping.
struct Cursor {
    const uint8_t* p;
    size_t size;
    size_t off;
    std::string err;
    bool need(size_t n, const char* what) {
        if (off > size || size - off < n) {
            if (err.empty()) err = std::string("Unexpected EOF while reading ") + what;
            return false;
        }
        return true;
    }
    template <typename T>
    bool read(T* v, const char* what) {
        if (!need(sizeof(T), what)) return false;
        std::memcpy(v, p + off, sizeof(T));
        off += sizeof(T);
        return true;
    }
    bool string(std::string* s) {
        uint64_t len = 0;
        if (!read(&len, "string length")) return false;
        if (len > kMaxString) {
            char b[128];
            snprintf(b, sizeof(b), "String too long: %llu bytes (max %zu)", (unsigned long long)len, kMaxString);
            err = b;
            return false;
        }
        if (!need((size_t)len, "string data")) return false;
        size_t valid_up_to = 0;
        int error_len = 0;
        if (!utf8_valid(p + off, (size_t)len, &valid_up_to, &error_len)) {
            // String::from_utf8 -> "Invalid UTF-8 string: {Utf8Error}" (gguf.rs:1780)
            char b[160];
            if (error_len > 0)
                snprintf(b, sizeof(b), "Invalid UTF-8 string: invalid utf-8 sequence of %d bytes from index %zu",
                         error_len, valid_up_to);
            else
                snprintf(b, sizeof(b), "Invalid UTF-8 string: incomplete utf-8 byte sequence from index %zu",
                         valid_up_to);
            err = b;
            return false;
        }
        s->assign(reinterpret_cast<const char*>(p + off), (size_t)len);
        off += (size_t)len;
        return true;
    }
    // UTF-8 well-formedness as String::from_utf8 checks it (RFC 3629: no overlong
    // forms, no surrogates, nothing above U+10FFFF).  On failure: the index of the
    // first bad sequence and the number of bytes that make it invalid (1-3), or 0
    // when the input ends inside a sequence.
    static bool utf8_valid(const uint8_t* s, size_t n, size_t* valid_up_to, int* error_len) {
        size_t i = 0;
        auto cont = [&](size_t j) { return (s[j] & 0xC0) == 0x80; };
        auto fail = [&](int len) {
            *valid_up_to = i;
            *error_len = len;
            return false;
        };
        while (i < n) {
            const uint8_t b = s[i];
            if (b < 0x80) {
                ++i;
                continue;
            }
            int width = 0;
            uint8_t lo = 0x80, hi = 0xBF;  // allowed range of the second byte
            if (b >= 0xC2 && b <= 0xDF) {
                width = 2;
            } else if (b >= 0xE0 && b <= 0xEF) {
                width = 3;
                if (b == 0xE0) lo = 0xA0;
                if (b == 0xED) hi = 0x9F;
            } else if (b >= 0xF0 && b <= 0xF4) {
                width = 4;
                if (b == 0xF0) lo = 0x90;
                if (b == 0xF4) hi = 0x8F;
            } else {
                return fail(1);
            }
            if (i + 1 >= n) return fail(0);
            if (s[i + 1] < lo || s[i + 1] > hi) return fail(1);
            for (int j = 2; j < width; ++j) {
                if (i + j >= n) return fail(0);
                if (!cont(i + j)) return fail(j);
            }
            i += (size_t)width;
        }
        return true;
    }
    bool type_id(bool one_byte, uint32_t* t, const char* what) {
        if (one_byte) {
            uint8_t b = 0;
            if (!read(&b, what)) return false;
            *t = b;
            return true;
        }
        return read(t, what);
    }
};

bool parse_value_of(Cursor& c, uint32_t type, bool one_byte, bool allow_array, Value* v) {
    v->type = (int)type;
    switch (type) {
    case kU8: { uint8_t x; if (!c.read(&x, "value")) return false; v->u = x; return true; }
    case kI8: { int8_t x; if (!c.read(&x, "value")) return false; v->i = x; return true; }
    case kU16: { uint16_t x; if (!c.read(&x, "value")) return false; v->u = x; return true; }
    case kI16: { int16_t x; if (!c.read(&x, "value")) return false; v->i = x; return true; }
    case kU32: { uint32_t x; if (!c.read(&x, "value")) return false; v->u = x; return true; }
    case kI32: { int32_t x; if (!c.read(&x, "value")) return false; v->i = x; return true; }
    case kF32: { float x; if (!c.read(&x, "value")) return false; v->f = x; return true; }
    case kBool: { uint8_t x; if (!c.read(&x, "value")) return false; v->u = x != 0; return true; }
    case kString: return c.string(&v->s);
    case kU64: { uint64_t x; if (!c.read(&x, "value")) return false; v->u = x; return true; }
    case kI64: { int64_t x; if (!c.read(&x, "value")) return false; v->i = x; return true; }
    case kF64: { double x; if (!c.read(&x, "value")) return false; v->f = x; return true; }
    case kArray: {
        if (!allow_array) {
            c.err = "Nested arrays are not supported by GGUF specification";
            return false;
        }
        uint32_t et = 0;
        uint64_t count = 0;
        if (!c.type_id(one_byte, &et, "array element type") || !c.read(&count, "array length")) return false;
        // every element takes at least one byte: a count past the file is malformed
        if (count > c.size - c.off) {
            c.err = "Unexpected EOF while reading array";
            return false;
        }
        // the count is bounded only by the bytes left, which a corrupt file can make huge:
        // reserve at most 64 Ki elements up front and let the vector grow past that
        v->arr.reserve((size_t)(count < ((uint64_t)1 << 16) ? count : ((uint64_t)1 << 16)));
        for (uint64_t k = 0; k < count; ++k) {
            Value e;
            if (!parse_value_of(c, et, one_byte, false, &e)) return false;
            v->arr.push_back(std::move(e));
        }
        return true;
    }
    default: {
        char b[64];
        snprintf(b, sizeof(b), "Unknown value type: %u", type);
        c.err = b;
        return false;
    }
    }
}

// Parses header, metadata and tensor infos in one dialect.  On failure returns false
// with the message in *err.
bool parse(openmini_qmm_gguf& g, bool reference_dialect, std::string* err) {
    Cursor c{g.base, g.size, 0, {}};
    uint32_t magic = 0;
    c.read(&magic, "magic");
    if (magic != kMagic) {
        char b[128];
        snprintf(b, sizeof(b), "Invalid GGUF magic number: expected %#x, got %#x", kMagic, magic);
        *err = b;
        return false;
    }
    c.read(&g.version, "version");
    c.read(&g.tensor_count, "tensor count");
    c.read(&g.kv_count, "metadata count");
    g.keys.clear();
    g.kv.clear();
    g.tensors.clear();
    g.by_name.clear();
    for (uint64_t k = 0; k < g.kv_count; ++k) {
        std::string key;
        uint32_t t = 0;
        Value v;
        if (!c.string(&key) || !c.type_id(reference_dialect, &t, "value type") ||
            !parse_value_of(c, t, reference_dialect, true, &v)) {
            *err = c.err;
            return false;
        }
        if (!g.kv.count(key)) g.keys.push_back(key);
        g.kv[key] = std::move(v);
    }
    for (uint64_t k = 0; k < g.tensor_count; ++k) {
        Tensor t;
        uint32_t nd = 0;
        if (!c.string(&t.name) || !c.read(&nd, "dimension count")) {
            *err = c.err;
            return false;
        }
        if (nd > kMaxDims) {
            char b[96];
            snprintf(b, sizeof(b), "Too many dimensions: %u (max %u)", nd, kMaxDims);
            *err = b;
            return false;
        }
        t.dims.resize(nd);
        for (uint32_t d = 0; d < nd; ++d)
            if (!c.read(&t.dims[d], "dimension")) {
                *err = c.err;
                return false;
            }
        uint32_t tt = 0;
        if (!c.type_id(reference_dialect, &tt, "tensor type") || !c.read(&t.offset, "tensor offset")) {
            *err = c.err;
            return false;
        }
        uint64_t bs = 0, bpb = 0;
        type_geometry((int)tt, &bs, &bpb);
        if (!bs) {
            char b[64];
            snprintf(b, sizeof(b), "Unknown tensor type: %u", tt);
            *err = b;
            return false;
        }
        t.type = (int)tt;
        if (g.by_name.count(t.name)) {
            g.tensors[g.by_name[t.name]] = t;  // a later definition replaces an earlier one
        } else {
            g.by_name[t.name] = g.tensors.size();
            g.tensors.push_back(std::move(t));
        }
    }
    if (!reference_dialect) {
        g.alignment = 32;
        auto it = g.kv.find("general.alignment");
        if (it != g.kv.end() && it->second.type == kU32 && it->second.u) g.alignment = (uint32_t)it->second.u;
        const uint64_t data = (c.off + g.alignment - 1) / g.alignment * g.alignment;
        for (auto& t : g.tensors) {
            if (t.offset > UINT64_MAX - data) {
                *err = "Tensor data out of bounds";
                return false;
            }
            t.offset += data;
        }
    }
    return true;
}

// Element count, saturating: UINT64_MAX when the product of the dims overflows.
uint64_t elements_of(const Tensor& t) {
    uint64_t n = 1;
    for (uint64_t d : t.dims) {
        if (d != 0 && n > UINT64_MAX / d) return UINT64_MAX;
        n *= d;
    }
    return n;
}

// Data bytes (GgufTensor::data_size, gguf.rs:431-438).  Tensors of more than 2^48
// elements get UINT64_MAX, which no file holds, so they report "Tensor data out of
// bounds" instead of a size that wrapped around.
uint64_t data_size_of(const Tensor& t) {
    uint64_t bs = 0, bpb = 0;
    type_geometry(t.type, &bs, &bpb);
    const uint64_t n = elements_of(t);
    if (n > ((uint64_t)1 << 48)) return UINT64_MAX;
    return (n + bs - 1) / bs * bpb;
}

bool fits(const openmini_qmm_gguf& g, const Tensor& t) {
    const uint64_t sz = data_size_of(t);
    return t.offset <= g.size && sz <= g.size - t.offset;
}

const Tensor* find(const openmini_qmm_gguf* g, const char* name) {
    if (!g || !name) return nullptr;
    auto it = g->by_name.find(name);
    return it == g->by_name.end() ? nullptr : &g->tensors[it->second];
}

int not_found(const char* name) {
    return gfail(OPENMINI_QMM_ERR_NOT_FOUND, "Tensor not found: %s", name ? name : "(null)");
}

const Value* meta(const openmini_qmm_gguf* g, const char* key) {
    if (!g || !key) return nullptr;
    auto it = g->kv.find(key);
    return it == g->kv.end() ? nullptr : &it->second;
}

}  // namespace

extern "C" {

int openmini_qmm_gguf_open(const char* path, int dialect, openmini_qmm_gguf_t** out) {
    if (!out) return gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "null out");
    *out = nullptr;
    if (!path) return gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "null path");
    if (dialect < OPENMINI_QMM_GGUF_AUTO || dialect > OPENMINI_QMM_GGUF_STANDARD)
        return gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "unknown dialect %d", dialect);
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return gfail(OPENMINI_QMM_ERR_MODEL_LOAD, "%s: %s (os error %d)", path, strerror(errno), errno);
    struct stat st;
    if (fstat(fd, &st) != 0) {
        const int e = errno;
        ::close(fd);
        return gfail(OPENMINI_QMM_ERR_MODEL_LOAD, "%s: %s (os error %d)", path, strerror(e), e);
    }
    const size_t size = (size_t)st.st_size;
    if (size < 24) {
        ::close(fd);
        return gfail(OPENMINI_QMM_ERR_MODEL_LOAD, "File too small to be a valid GGUF file");
    }
    void* map = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    const int map_errno = errno;
    ::close(fd);
    if (map == MAP_FAILED)
        return gfail(OPENMINI_QMM_ERR_MODEL_LOAD, "mmap %s: %s", path, strerror(map_errno));
    openmini_qmm_gguf* g = new (std::nothrow) openmini_qmm_gguf();
    if (!g) {
        munmap(map, size);
        return gfail(OPENMINI_QMM_ERR_MEMORY, "host allocation failed");
    }
    g->base = static_cast<const uint8_t*>(map);
    g->size = size;
    std::string err;
    bool ok = false;
    try {  // a file whose counts outrun host memory fails with MEMORY; nothing escapes the C ABI
        if (dialect == OPENMINI_QMM_GGUF_REFERENCE) {
            ok = parse(*g, true, &err);
            g->dialect = OPENMINI_QMM_GGUF_REFERENCE;
        } else {
            ok = parse(*g, false, &err);
            g->dialect = OPENMINI_QMM_GGUF_STANDARD;
            if (dialect == OPENMINI_QMM_GGUF_AUTO) {
                bool all_fit = ok;
                for (const auto& t : g->tensors) all_fit = all_fit && fits(*g, t);
                if (!all_fit) {
                    std::string err2;
                    if (parse(*g, true, &err2)) {
                        ok = true;
                        g->dialect = OPENMINI_QMM_GGUF_REFERENCE;
                    } else if (ok) {
                        parse(*g, false, &err);  // keep the standard reading
                    }
                }
            }
        }
    } catch (const std::bad_alloc&) {
        openmini_qmm_gguf_close(g);
        return gfail(OPENMINI_QMM_ERR_MEMORY, "host allocation failed while parsing %s", path);
    }
    if (!ok) {
        openmini_qmm_gguf_close(g);
        return gfail(OPENMINI_QMM_ERR_MODEL_LOAD, "%s", err.c_str());
    }
    *out = g;
    qmm::set_last_error("");
    return OPENMINI_QMM_OK;
}

void openmini_qmm_gguf_close(openmini_qmm_gguf_t* g) {
    if (!g) return;
    if (g->base) munmap(const_cast<uint8_t*>(g->base), g->size);
    delete g;
}

int openmini_qmm_gguf_header(const openmini_qmm_gguf_t* g, openmini_qmm_gguf_header_t* h) {
    if (!g || !h) return gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "null argument");
    h->version = g->version;
    h->dialect = g->dialect;
    h->tensor_count = g->tensor_count;
    h->metadata_kv_count = g->kv_count;
    h->distinct_tensors = g->tensors.size();
    h->distinct_keys = g->keys.size();
    h->alignment = g->alignment;
    h->file_size = g->size;
    return OPENMINI_QMM_OK;
}

int openmini_qmm_gguf_tensor_name(const openmini_qmm_gguf_t* g, size_t index, char* buf, size_t buf_len) {
    if (!g || !buf || !buf_len) return gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "null argument");
    if (index >= g->tensors.size())
        return gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "tensor index %zu out of range (%zu)", index, g->tensors.size());
    snprintf(buf, buf_len, "%s", g->tensors[index].name.c_str());
    return g->tensors[index].name.size() < buf_len ? OPENMINI_QMM_OK
                                                   : gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "buffer too small");
}

int openmini_qmm_gguf_tensor_info(const openmini_qmm_gguf_t* g, const char* name,
                                  openmini_qmm_gguf_tensor_info_t* info) {
    if (!info) return gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "null info");
    const Tensor* t = find(g, name);
    if (!t) return not_found(name);
    std::memset(info, 0, sizeof(*info));
    info->type = t->type;
    info->n_dims = (uint32_t)t->dims.size();
    for (size_t d = 0; d < t->dims.size(); ++d) info->dims[d] = t->dims[d];
    info->offset = t->offset;
    info->n_elements = elements_of(*t);
    info->data_size = data_size_of(*t);
    return OPENMINI_QMM_OK;
}

int openmini_qmm_gguf_tensor_data(const openmini_qmm_gguf_t* g, const char* name, const void** data,
                                  size_t* bytes) {
    if (!data || !bytes) return gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "null argument");
    *data = nullptr;
    *bytes = 0;
    const Tensor* t = find(g, name);
    if (!t) return not_found(name);
    if (!fits(*g, *t)) return gfail(OPENMINI_QMM_ERR_MODEL_LOAD, "Tensor data out of bounds");
    *data = g->base + t->offset;
    *bytes = (size_t)data_size_of(*t);
    return OPENMINI_QMM_OK;
}

int openmini_qmm_gguf_meta_type(const openmini_qmm_gguf_t* g, const char* key, int* value_type,
                                uint64_t* array_len) {
    const Value* v = meta(g, key);
    if (!v) return gfail(OPENMINI_QMM_ERR_NOT_FOUND, "metadata key not found: %s", key ? key : "(null)");
    if (value_type) *value_type = v->type;
    if (array_len) *array_len = v->type == kArray ? v->arr.size() : 0;
    return OPENMINI_QMM_OK;
}

int openmini_qmm_gguf_meta_key(const openmini_qmm_gguf_t* g, size_t index, char* buf, size_t buf_len) {
    if (!g || !buf || !buf_len) return gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "null argument");
    if (index >= g->keys.size())
        return gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "key index %zu out of range (%zu)", index, g->keys.size());
    snprintf(buf, buf_len, "%s", g->keys[index].c_str());
    return g->keys[index].size() < buf_len ? OPENMINI_QMM_OK
                                           : gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "buffer too small");
}

// GgufMetadata::get_u32 (gguf.rs:157-163): UInt32, or Int32 reinterpreted.
int openmini_qmm_gguf_get_u32(const openmini_qmm_gguf_t* g, const char* key, uint32_t* out) {
    const Value* v = meta(g, key);
    if (!out) return gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "null out");
    if (v && v->type == kU32) { *out = (uint32_t)v->u; return OPENMINI_QMM_OK; }
    if (v && v->type == kI32) { *out = (uint32_t)(int32_t)v->i; return OPENMINI_QMM_OK; }
    return gfail(OPENMINI_QMM_ERR_NOT_FOUND, "no u32 value for %s", key ? key : "(null)");
}

// GgufMetadata::get_u64 (gguf.rs:172-180): UInt64, Int64, UInt32, Int32.
int openmini_qmm_gguf_get_u64(const openmini_qmm_gguf_t* g, const char* key, uint64_t* out) {
    const Value* v = meta(g, key);
    if (!out) return gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "null out");
    if (v && (v->type == kU64 || v->type == kU32)) { *out = v->u; return OPENMINI_QMM_OK; }
    if (v && (v->type == kI64 || v->type == kI32)) { *out = (uint64_t)v->i; return OPENMINI_QMM_OK; }
    return gfail(OPENMINI_QMM_ERR_NOT_FOUND, "no u64 value for %s", key ? key : "(null)");
}

// GgufMetadata::get_f32 (gguf.rs:189-194): Float32 only.
int openmini_qmm_gguf_get_f32(const openmini_qmm_gguf_t* g, const char* key, float* out) {
    const Value* v = meta(g, key);
    if (!out) return gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "null out");
    if (v && v->type == kF32) { *out = (float)v->f; return OPENMINI_QMM_OK; }
    return gfail(OPENMINI_QMM_ERR_NOT_FOUND, "no f32 value for %s", key ? key : "(null)");
}

// GgufMetadata::get_string (gguf.rs:143-148).  *out_len = the string's length; the
// copy in buf is NUL-terminated and truncated to buf_len - 1 bytes.
int openmini_qmm_gguf_get_string(const openmini_qmm_gguf_t* g, const char* key, char* buf, size_t buf_len,
                                 size_t* out_len) {
    const Value* v = meta(g, key);
    if (!v || v->type != kString)
        return gfail(OPENMINI_QMM_ERR_NOT_FOUND, "no string value for %s", key ? key : "(null)");
    if (out_len) *out_len = v->s.size();
    if (buf && buf_len) snprintf(buf, buf_len, "%s", v->s.c_str());
    return OPENMINI_QMM_OK;
}

int openmini_qmm_gguf_upload_weight(const openmini_qmm_gguf_t* g, const char* name, void* stream,
                                    openmini_qweight_t** out_weight) {
    if (!out_weight) return gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "null out_weight");
    *out_weight = nullptr;
    const Tensor* t = find(g, name);
    if (!t) return not_found(name);
    if (t->dims.size() != 2)
        return gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "%s has %zu dimensions; a linear weight has 2 ([K, N])",
                     name, t->dims.size());
    if (t->type != OPENMINI_QMM_Q4_0 && t->type != OPENMINI_QMM_Q4_1 && t->type != OPENMINI_QMM_Q8_0 &&
        !qmm::is_kquant(t->type) && t->type != OPENMINI_QMM_Q8_K)
        return gfail(OPENMINI_QMM_ERR_UNSUPPORTED,
                     "%s is tensor type %d; weights upload as Q4_0 (2), Q4_1 (3), Q8_0 (7), Q4_K (12), Q5_K (13), "
                     "Q6_K (14) or Q8_K (15)", name, t->type);
    if (!fits(*g, *t)) return gfail(OPENMINI_QMM_ERR_MODEL_LOAD, "Tensor data out of bounds");
    // GGUF dims [ne0, ne1] = [K, N]: row n of W is ne0 = K consecutive elements.
    const int64_t k = (int64_t)t->dims[0], n = (int64_t)t->dims[1];
    return qmm::upload_from_host(t->type, g->base + t->offset, (size_t)data_size_of(*t), n, k, stream,
                                 out_weight);
}

int openmini_qmm_gguf_dequantize_tensor(const openmini_qmm_gguf_t* g, const char* name, float* d_out,
                                        void* stream) {
    const Tensor* t = find(g, name);
    if (!t) return not_found(name);
    if (!d_out) return gfail(OPENMINI_QMM_ERR_INVALID_PARAM, "null out");
    if (!fits(*g, *t)) return gfail(OPENMINI_QMM_ERR_MODEL_LOAD, "Tensor data out of bounds");
    if (!qmm::layout_block_size(t->type))
        return gfail(OPENMINI_QMM_ERR_UNSUPPORTED, "%s is tensor type %d, which is not implemented", name, t->type);
    // the reference casts F32 / F16 data in place and refuses a misaligned start (the
    // mapping itself is page-aligned, so the file offset decides; gguf.rs:2074-2095)
    if (t->type == OPENMINI_QMM_F32 && t->offset % 4 != 0)
        return gfail(OPENMINI_QMM_ERR_MODEL_LOAD, "F32 data is not properly aligned");
    if (t->type == OPENMINI_QMM_F16 && t->offset % 2 != 0)
        return gfail(OPENMINI_QMM_ERR_MODEL_LOAD, "F16 data is not properly aligned");
    return qmm::dequantize_from_host(t->type, g->base + t->offset, (size_t)data_size_of(*t),
                                     (size_t)elements_of(*t), d_out, stream);
}

}  // extern "C"
