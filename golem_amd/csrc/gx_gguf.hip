// gx_gguf.hip - the GGUF container, read in place (host code only).
//
// golem's tensors/gguf.go (OpenGGUF, readHeader, readTensorTable, Get,
// Close), tensors/gguf_meta.go (the typed metadata accessors) and
// tensors/mmap.go (the whole file mapped, nothing copied).  A GGUF is a
// header, a table of typed metadata, a table of tensor descriptions and then
// the tensor data at the next multiple of the alignment.  Every tensor is a
// view into the mapping; gx_weight_upload takes such a view directly, so a
// checkpoint goes from the page cache to HBM without a host copy.
//
// The checks and their wording follow golem's reader: a file that golem
// refuses is refused here with the same message, and one it accepts reads the
// same tensors at the same offsets.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "gx_internal.hpp"

namespace {

// The thirteen metadata value types, numbered as the format numbers them
// (tensors/gguf.go:17-31).
enum : uint32_t {
    kU8 = 0, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kString, kArray, kU64, kI64, kF64, kTypes
};

const char *type_name(uint32_t t) {  // as golem's %T prints the decoded value
    static const char *names[kTypes] = {"uint8", "int8",  "uint16", "int16", "uint32", "int32",  "float32",
                                        "bool",  "string", "[]interface {}", "uint64", "int64", "float64"};
    return t < kTypes ? names[t] : "?";
}

struct Value {
    uint32_t type = 0;
    uint64_t u = 0;  // unsigned and bool values
    int64_t i = 0;   // signed values
    double f = 0;    // float32 (exactly) and float64 values
    std::string s;
    std::vector<Value> items;
};

struct Tensor {
    std::string name;
    int ggml_type = 0;
    int ndims = 0;
    int64_t shape[4] = {0, 0, 0, 0};
    size_t start = 0, bytes = 0;
};

// The ggml type numbers golem reads, and their block geometry (weights per
// block, bytes per block), tensors/gguf.go:200-222.
struct Geometry {
    uint32_t type;
    const char *name;
    int per_block, block_bytes;
};
const Geometry kGeometry[] = {
    {0, "F32", 1, 4}, {1, "F16", 1, 2}, {2, "Q4_0", 32, 18}, {8, "Q8_0", 32, 34}, {14, "Q6_K", 256, 210},
    {30, "BF16", 1, 2},
};

const Geometry *geometry(uint32_t type) {
    for (const Geometry &g : kGeometry)
        if (g.type == type)
            return &g;
    return nullptr;
}

// A bounds-checked cursor over the mapping (golem's reader type): the first
// failure sticks and every later read returns zero.
struct Reader {
    const uint8_t *buf;
    size_t len, pos = 0;
    std::string err;

    const uint8_t *take(uint64_t n) {
        if (!err.empty())
            return nullptr;
        if (n > len - pos) {
            err = "truncated at byte " + std::to_string(pos);
            return nullptr;
        }
        const uint8_t *p = buf + pos;
        pos += n;
        return p;
    }
    uint64_t le(int n) {
        const uint8_t *p = take(n);
        uint64_t v = 0;
        if (p)
            for (int k = n - 1; k >= 0; k--)
                v = v << 8 | p[k];
        return v;
    }
    uint32_t u32() { return (uint32_t)le(4); }
    uint64_t u64() { return le(8); }
    std::string str() {
        const uint64_t n = u64();
        if (!err.empty())
            return "";
        if (n > len) {
            err = "string of " + std::to_string(n) + " bytes at " + std::to_string(pos);
            return "";
        }
        const uint8_t *p = take(n);
        return p ? std::string((const char *)p, n) : std::string();
    }
    // One metadata value of the given type (tensors/gguf.go:92-158).
    Value value(uint32_t kind) {
        Value v;
        v.type = kind;
        switch (kind) {
        case kU8: v.u = le(1); break;
        case kI8: v.i = (int8_t)le(1); break;
        case kU16: v.u = le(2); break;
        case kI16: v.i = (int16_t)le(2); break;
        case kU32: v.u = le(4); break;
        case kI32: v.i = (int32_t)le(4); break;
        case kF32: {
            const uint32_t bits = (uint32_t)le(4);
            float f;
            memcpy(&f, &bits, 4);
            v.f = f;
            break;
        }
        case kBool: v.u = le(1) != 0; break;
        case kString: v.s = str(); break;
        case kArray: {
            const uint32_t elem = u32();
            const uint64_t n = u64();
            if (!err.empty())
                return v;
            if (n > len) {
                err = "array of " + std::to_string(n) + " values at " + std::to_string(pos);
                return v;
            }
            v.u = elem;
            v.items.reserve(n);
            for (uint64_t k = 0; k < n; k++) {
                v.items.push_back(value(elem));
                if (!err.empty())
                    return v;
            }
            break;
        }
        case kU64: v.u = le(8); break;
        case kI64: v.i = (int64_t)le(8); break;
        case kF64: {
            const uint64_t bits = le(8);
            memcpy(&v.f, &bits, 8);
            break;
        }
        default:
            err = "unknown metadata type " + std::to_string(kind) + " at byte " + std::to_string(pos);
        }
        return v;
    }
};

// asUint32 (tensors/gguf_meta.go:56-77): any integer width, converted as Go
// converts it (truncated or wrapped to 32 bits).
bool as_u32(const Value &v, uint32_t *out) {
    switch (v.type) {
    case kU8: case kU16: case kU32: case kU64: *out = (uint32_t)v.u; return true;
    case kI8: case kI16: case kI32: case kI64: *out = (uint32_t)v.i; return true;
    }
    return false;
}

}  // namespace

struct gx_gguf {
    void *map = nullptr;
    size_t size = 0;
    std::vector<std::pair<std::string, Value>> meta;  // in file order; a repeated key keeps its last value
    std::unordered_map<std::string, size_t> meta_at;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> tensor_at;
    size_t data_offset = 0;

    const Value *find(const char *key) const {
        auto it = meta_at.find(key);
        return it == meta_at.end() ? nullptr : &meta[it->second].second;
    }
};

namespace {

int absent(const char *key) { return gx::fail(GX_ERR_INVALID, "metadata \"%s\" is absent", key); }

int wrong(const char *key, const Value &v, const char *want) {
    return gx::fail(GX_ERR_INVALID, "metadata \"%s\" is %s, not %s", key, type_name(v.type), want);
}

// readHeader + readTensorTable (tensors/gguf.go:177-301).  Returns "" or the
// reason the file is refused.
std::string parse(gx_gguf *g) {
    Reader r{(const uint8_t *)g->map, g->size};
    if (r.u32() != 0x46554747u)  // "GGUF", little-endian
        return "not a GGUF file";
    const uint32_t version = r.u32();  // a short file reads as version 0, as golem's does
    if (version != 2 && version != 3)
        return "GGUF version " + std::to_string(version) + ", only 2 and 3 are read";
    const uint64_t tensor_count = r.u64();
    const uint64_t meta_count = r.u64();
    if (!r.err.empty())
        return r.err;
    for (uint64_t k = 0; k < meta_count; k++) {
        std::string key = r.str();
        const uint32_t kind = r.u32();
        Value v = r.value(kind);
        if (!r.err.empty())
            return "metadata " + std::to_string(k) + " (\"" + key + "\"): " + r.err;
        auto it = g->meta_at.find(key);
        if (it != g->meta_at.end()) {
            g->meta[it->second].second = std::move(v);
        } else {
            g->meta_at.emplace(key, g->meta.size());
            g->meta.emplace_back(std::move(key), std::move(v));
        }
    }

    std::vector<Tensor> entries;
    for (uint64_t k = 0; k < tensor_count; k++) {
        Tensor t;
        t.name = r.str();
        const uint32_t dims = r.u32();
        if (!r.err.empty())
            return "tensor " + std::to_string(k) + ": " + r.err;
        if (dims == 0 || dims > 4)
            return "tensor \"" + t.name + "\" has " + std::to_string(dims) + " dimensions";
        t.ndims = (int)dims;
        uint64_t elements = 1;
        for (uint32_t d = 0; d < dims; d++) {
            t.shape[d] = (int64_t)r.u64();
            elements *= (uint64_t)t.shape[d];
        }
        const uint32_t kind = r.u32();
        const uint64_t offset = r.u64();
        if (!r.err.empty())
            return "tensor \"" + t.name + "\": " + r.err;
        const Geometry *geo = geometry(kind);
        if (!geo)
            return "tensor \"" + t.name + "\": unsupported ggml type " + std::to_string(kind);
        // shape[0] is the row length; everything above it counts rows
        if (t.shape[0] <= 0 || t.shape[0] % geo->per_block != 0)
            return "tensor \"" + t.name + "\": a row of " + std::to_string(t.shape[0]) +
                   " does not divide into blocks of " + std::to_string(geo->per_block) + " (" + geo->name + ")";
        const uint64_t row_bytes = (uint64_t)t.shape[0] / geo->per_block * geo->block_bytes;
        t.ggml_type = (int)kind;
        t.bytes = (size_t)(row_bytes * (elements / (uint64_t)t.shape[0]));
        t.start = (size_t)offset;  // relative to the data section until it is known
        entries.push_back(std::move(t));
    }

    // The data section begins at the next multiple of the alignment.
    uint64_t alignment = 32;
    if (const Value *v = g->find("general.alignment")) {
        uint32_t a;
        if (as_u32(*v, &a))
            alignment = a;
    }
    if (alignment == 0 || (alignment & (alignment - 1)) != 0)
        return "alignment " + std::to_string(alignment) + " is not a power of two";
    g->data_offset = (r.pos + alignment - 1) & ~(size_t)(alignment - 1);

    for (Tensor &t : entries) {
        const uint64_t start = g->data_offset + (uint64_t)t.start, end = start + t.bytes;
        if (start < g->data_offset || end > g->size || end < start)
            return "tensor \"" + t.name + "\" runs from " + std::to_string(start) + " to " + std::to_string(end) +
                   ", past the end of the file";
        t.start = (size_t)start;
        auto it = g->tensor_at.find(t.name);
        if (it != g->tensor_at.end()) {
            g->tensors[it->second] = std::move(t);
        } else {
            g->tensor_at.emplace(t.name, g->tensors.size());
            g->tensors.push_back(std::move(t));
        }
    }
    return "";
}

void unmap(gx_gguf *g) {
    if (g->map)
        munmap(g->map, g->size);
    g->map = nullptr;
}

}  // namespace

extern "C" {

int gx_gguf_open(const char *path, gx_gguf **out) {
    GX_CHECK(path != nullptr && out != nullptr, "gx: gguf: no path or no place for the handle");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0)
        return gx::fail(GX_ERR_INVALID, "open %s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        const int e = errno;
        close(fd);
        return gx::fail(GX_ERR_INVALID, "stat %s: %s", path, strerror(e));
    }
    if (st.st_size == 0) {
        close(fd);
        return gx::fail(GX_ERR_INVALID, "%s is empty", path);
    }
    void *map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_SHARED, fd, 0);
    const int e = errno;
    close(fd);  // the mapping outlives the descriptor
    if (map == MAP_FAILED)
        return gx::fail(GX_ERR_INVALID, "mmap %s: %s", path, strerror(e));
    gx_gguf *g = new gx_gguf;
    g->map = map;
    g->size = (size_t)st.st_size;
    const std::string why = parse(g);
    if (!why.empty()) {
        unmap(g);
        delete g;
        return gx::fail(GX_ERR_INVALID, "%s: %s", path, why.c_str());
    }
    *out = g;
    return gx::succeed();
}

int gx_gguf_close(gx_gguf *g) {
    if (g) {
        unmap(g);
        delete g;
    }
    return gx::succeed();
}

int gx_gguf_tensor_count(const gx_gguf *g, int *count) {
    GX_CHECK(g && count, "gx: gguf: no handle or no place for the count");
    *count = (int)g->tensors.size();
    return gx::succeed();
}

int gx_gguf_tensor_name(const gx_gguf *g, int index, const char **name) {
    GX_CHECK(g && name, "gx: gguf: no handle or no place for the name");
    GX_CHECK(index >= 0 && (size_t)index < g->tensors.size(), "gx: gguf: tensor %d of %zu", index,
             g->tensors.size());
    *name = g->tensors[index].name.c_str();
    return gx::succeed();
}

int gx_gguf_tensor(const gx_gguf *g, const char *name, int *ggml_type, int *ndims, int64_t *shape, const void **data,
                   size_t *bytes) {
    GX_CHECK(g && name, "gx: gguf: no handle or no name");
    auto it = g->tensor_at.find(name);
    if (it == g->tensor_at.end())
        return gx::fail(GX_ERR_INVALID, "tensor \"%s\" is absent", name);
    const Tensor &t = g->tensors[it->second];
    if (ggml_type)
        *ggml_type = t.ggml_type;
    if (ndims)
        *ndims = t.ndims;
    if (shape)
        for (int d = 0; d < 4; d++)
            shape[d] = d < t.ndims ? t.shape[d] : 0;
    if (data)
        *data = (const uint8_t *)g->map + t.start;
    if (bytes)
        *bytes = t.bytes;
    return gx::succeed();
}

int gx_gguf_meta_count(const gx_gguf *g, int *count) {
    GX_CHECK(g && count, "gx: gguf: no handle or no place for the count");
    *count = (int)g->meta.size();
    return gx::succeed();
}

int gx_gguf_meta_key(const gx_gguf *g, int index, const char **key, int *type) {
    GX_CHECK(g && key, "gx: gguf: no handle or no place for the key");
    GX_CHECK(index >= 0 && (size_t)index < g->meta.size(), "gx: gguf: metadata %d of %zu", index, g->meta.size());
    *key = g->meta[index].first.c_str();
    if (type)
        *type = (int)g->meta[index].second.type;
    return gx::succeed();
}

int gx_gguf_meta_string(const gx_gguf *g, const char *key, const char **s, size_t *len) {
    GX_CHECK(g && key && s, "gx: gguf: no handle, key or place for the string");
    const Value *v = g->find(key);
    if (!v)
        return absent(key);
    if (v->type != kString)
        return wrong(key, *v, "a string");
    *s = v->s.c_str();
    if (len)
        *len = v->s.size();
    return gx::succeed();
}

int gx_gguf_meta_bool(const gx_gguf *g, const char *key, int *out) {
    GX_CHECK(g && key && out, "gx: gguf: no handle, key or place for the value");
    const Value *v = g->find(key);
    if (!v)
        return absent(key);
    if (v->type != kBool)
        return wrong(key, *v, "a bool");
    *out = (int)v->u;
    return gx::succeed();
}

int gx_gguf_meta_f32(const gx_gguf *g, const char *key, float *out) {
    GX_CHECK(g && key && out, "gx: gguf: no handle, key or place for the value");
    const Value *v = g->find(key);
    if (!v)
        return absent(key);
    if (v->type != kF32 && v->type != kF64)
        return wrong(key, *v, "a float");
    *out = (float)v->f;
    return gx::succeed();
}

int gx_gguf_meta_u32(const gx_gguf *g, const char *key, uint32_t *out) {
    GX_CHECK(g && key && out, "gx: gguf: no handle, key or place for the value");
    const Value *v = g->find(key);
    if (!v)
        return absent(key);
    if (!as_u32(*v, out))
        return wrong(key, *v, "an integer");
    return gx::succeed();
}

int gx_gguf_meta_u32s(const gx_gguf *g, const char *key, uint32_t *out, size_t cap, size_t *count) {
    GX_CHECK(g && key && count, "gx: gguf: no handle, key or place for the count");
    const Value *v = g->find(key);
    if (!v)
        return absent(key);
    if (v->type != kArray) {  // a scalar reads as an array of one
        uint32_t n;
        if (!as_u32(*v, &n))
            return wrong(key, *v, "an integer");
        *count = 1;
        if (out && cap >= 1)
            out[0] = n;
        return gx::succeed();
    }
    for (size_t k = 0; k < v->items.size(); k++) {
        uint32_t n;
        if (!as_u32(v->items[k], &n))
            return wrong(key, v->items[k], "an integer");
        if (out && k < cap)
            out[k] = n;
    }
    *count = v->items.size();
    return gx::succeed();
}

int gx_gguf_meta_bools(const gx_gguf *g, const char *key, uint8_t *out, size_t cap, size_t *count) {
    GX_CHECK(g && key && count, "gx: gguf: no handle, key or place for the count");
    const Value *v = g->find(key);
    if (!v)
        return absent(key);
    if (v->type != kArray) {
        if (v->type != kBool)
            return wrong(key, *v, "a bool");
        *count = 1;
        if (out && cap >= 1)
            out[0] = (uint8_t)v->u;
        return gx::succeed();
    }
    for (size_t k = 0; k < v->items.size(); k++) {
        if (v->items[k].type != kBool)
            return gx::fail(GX_ERR_INVALID, "metadata \"%s\" holds a %s, not a bool", key,
                            type_name(v->items[k].type));
        if (out && k < cap)
            out[k] = (uint8_t)v->items[k].u;
    }
    *count = v->items.size();
    return gx::succeed();
}

int gx_gguf_meta_strings(const gx_gguf *g, const char *key, size_t index, const char **s, size_t *len,
                         size_t *count) {
    GX_CHECK(g && key && count, "gx: gguf: no handle, key or place for the count");
    const Value *v = g->find(key);
    if (!v)
        return absent(key);
    if (v->type != kArray)
        return wrong(key, *v, "an array");
    for (const Value &item : v->items)
        if (item.type != kString)
            return gx::fail(GX_ERR_INVALID, "metadata \"%s\" holds a %s, not a string", key, type_name(item.type));
    *count = v->items.size();
    if (s) {
        GX_CHECK(index < v->items.size(), "gx: gguf: string %zu of %zu in \"%s\"", index, v->items.size(), key);
        *s = v->items[index].s.c_str();
        if (len)
            *len = v->items[index].s.size();
    }
    return gx::succeed();
}

}  // extern "C"
