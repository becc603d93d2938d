// ns_gguf.cpp -- GGUF v3 reader (host side): the engine's GGUF class
// (src/native/gguf.cpp:71-122, include/neutron/native/gguf.hpp) behind the C ABI,
// plus the FFN tensor table that .nsmffn conversion takes (ffn_tensors,
// src/native/metal_ffn.cpp:63-71, with Gemma4Model's tensor names, model.cpp:17).
//
// File layout (GGUF v3, little endian): magic "GGUF", u32 version, u64 tensor
// count, u64 metadata count; metadata entries (string key, u32 value type,
// value; arrays carry an element type and a u64 length); tensor entries
// (string name, u32 rank, u64 dims, u32 type, u64 offset from the data
// section); the data section starts at the next multiple of general.alignment
// (32 by default).  Strings are a u64 length and that many bytes.
//
// The mapping is private and read-only; tensors are addressed in place.  The
// checks and their messages follow the reference reader, so an engine sees the
// same failures.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "ns_ffn.h"
#include "ns_internal.hpp"

namespace {

enum : uint32_t { kU8, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kString, kArray, kU64, kI64, kF64 };

uint32_t scalar_size(uint32_t t) {
    switch (t) {
        case kU8: case kI8: case kBool: return 1;
        case kU16: case kI16: return 2;
        case kU32: case kI32: case kF32: return 4;
        case kU64: case kI64: case kF64: return 8;
        default: return 0;
    }
}

// One metadata value.  Scalars keep their integer or floating value; arrays keep
// their element type, length and raw little-endian elements (strings separately).
struct MetaValue {
    uint32_t type = 0;       // value type; kArray for arrays
    uint32_t elem = 0;       // element type of an array
    uint64_t count = 0;      // array length
    uint64_t u = 0;          // unsigned scalars and bool
    int64_t i = 0;           // signed scalars
    double f = 0.0;          // kF32 / kF64
    std::string s;           // kString
    std::vector<uint8_t> raw;        // numeric array elements
    std::vector<std::string> strs;   // string array elements
};

class Cursor {
public:
    Cursor(const uint8_t *p, size_t n) : p_(p), n_(n) {}
    template <class T>
    T get() {
        if (pos_ + sizeof(T) > n_) throw std::runtime_error("truncated GGUF header");
        T v;
        std::memcpy(&v, p_ + pos_, sizeof(T));
        pos_ += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t len = get<uint64_t>();
        if (len > n_ - pos_) throw std::runtime_error("invalid GGUF string length");
        std::string s(reinterpret_cast<const char *>(p_ + pos_), size_t(len));
        pos_ += len;
        return s;
    }
    void bytes(void *dst, size_t len) {
        if (len > n_ - pos_) throw std::runtime_error("truncated GGUF header");
        std::memcpy(dst, p_ + pos_, len);
        pos_ += len;
    }
    size_t pos() const { return pos_; }

private:
    const uint8_t *p_;
    size_t n_, pos_ = 0;
};

MetaValue read_scalar(Cursor &c, uint32_t t) {
    MetaValue v;
    v.type = t;
    switch (t) {
        case kU8: v.u = c.get<uint8_t>(); break;
        case kI8: v.i = c.get<int8_t>(); break;
        case kU16: v.u = c.get<uint16_t>(); break;
        case kI16: v.i = c.get<int16_t>(); break;
        case kU32: v.u = c.get<uint32_t>(); break;
        case kI32: v.i = c.get<int32_t>(); break;
        case kU64: v.u = c.get<uint64_t>(); break;
        case kI64: v.i = c.get<int64_t>(); break;
        case kF32: v.f = c.get<float>(); break;
        case kF64: v.f = c.get<double>(); break;
        case kBool: v.u = c.get<uint8_t>() != 0; break;
        case kString: v.s = c.str(); break;
        default: throw std::runtime_error("unsupported GGUF scalar type");
    }
    return v;
}

MetaValue read_array(Cursor &c) {
    MetaValue v;
    v.type = kArray;
    v.elem = c.get<uint32_t>();
    v.count = c.get<uint64_t>();
    if (v.count > (uint64_t(1) << 31)) throw std::runtime_error("unreasonable GGUF array length");
    if (v.elem == kString) {
        v.strs.reserve(size_t(v.count));
        for (uint64_t k = 0; k < v.count; ++k) v.strs.push_back(c.str());
    } else {
        const uint32_t es = scalar_size(v.elem);
        if (es == 0) throw std::runtime_error("nested/invalid GGUF array type");
        v.raw.resize(size_t(v.count) * es);
        c.bytes(v.raw.data(), v.raw.size());
    }
    return v;
}

// Bytes of a tensor of `elements` values (gguf.cpp tensor_type_size / tensor_block_size).
uint64_t tensor_bytes(uint32_t type, uint64_t elements) {
    uint64_t block = 1, size = 0;
    switch (type) {
        case 0: size = 4; break;                  // F32
        case 1: size = 2; break;                  // F16
        case 12: size = 144; block = 256; break;  // Q4_K
        case 14: size = 210; block = 256; break;  // Q6_K
        default: throw std::runtime_error("unsupported tensor type " + std::to_string(type));
    }
    if (elements % block) throw std::runtime_error("invalid quantized tensor shape");
    return elements / block * size;
}

}  // namespace

struct ns_gguf {
    int fd = -1;
    uint8_t *map = nullptr;
    size_t size = 0;
    uint64_t data_offset = 0;
    std::unordered_map<std::string, MetaValue> meta;
    std::vector<std::string> names;
    std::vector<ns_gguf_tensor_info> tensors;
    std::unordered_map<std::string, uint32_t> index;

    ~ns_gguf() {
        if (map) munmap(map, size);
        if (fd >= 0) ::close(fd);
    }

    void parse() {
        Cursor c(map, size);
        if (c.get<uint32_t>() != 0x46554747u) throw std::runtime_error("bad GGUF magic");
        if (c.get<uint32_t>() != 3) throw std::runtime_error("only GGUF v3 is supported");
        const uint64_t ntensors = c.get<uint64_t>(), nmeta = c.get<uint64_t>();
        if (ntensors > 100000 || nmeta > 100000) throw std::runtime_error("invalid GGUF counts");
        for (uint64_t k = 0; k < nmeta; ++k) {
            std::string key = c.str();
            const uint32_t t = c.get<uint32_t>();
            meta.emplace(std::move(key), t == kArray ? read_array(c) : read_scalar(c, t));
        }
        uint64_t align = 32;
        if (meta.count("general.alignment")) align = integer("general.alignment");
        names.reserve(size_t(ntensors));
        tensors.reserve(size_t(ntensors));
        for (uint64_t k = 0; k < ntensors; ++k) {
            names.push_back(c.str());
            ns_gguf_tensor_info t{};
            t.n_dims = c.get<uint32_t>();
            if (t.n_dims == 0 || t.n_dims > 4) throw std::runtime_error("invalid tensor rank");
            uint64_t elements = 1;
            for (uint32_t d = 0; d < t.n_dims; ++d) {
                t.shape[d] = c.get<uint64_t>();
                elements *= t.shape[d];
            }
            t.type = c.get<uint32_t>();
            t.offset = c.get<uint64_t>();
            try {
                t.bytes = tensor_bytes(t.type, elements);
            } catch (const std::exception &e) {
                throw std::runtime_error(std::string(e.what()) + ": " + names.back());
            }
            index.emplace(names.back(), uint32_t(tensors.size()));
            tensors.push_back(t);
        }
        data_offset = (uint64_t(c.pos()) + align - 1) & ~(align - 1);
        for (size_t k = 0; k < tensors.size(); ++k) {
            tensors[k].name = names[k].c_str();
            if (data_offset + tensors[k].offset + tensors[k].bytes > size)
                throw std::runtime_error("tensor outside GGUF mapping: " + names[k]);
        }
    }

    // meta_u64 (gguf.cpp:127): unsigned or signed integers (a bool is neither).
    uint64_t integer(const std::string &key) const {
        const MetaValue &v = meta.at(key);
        switch (v.type) {
            case kU8: case kU16: case kU32: case kU64: return v.u;
            case kI8: case kI16: case kI32: case kI64: return uint64_t(v.i);
            default: throw std::runtime_error("metadata is not integer: " + key);
        }
    }
};

namespace {
template <class F>
int guarded(const char *fn, F &&body) {
    try {
        body();
        return NS_OK;
    } catch (const std::runtime_error &e) {
        ns::set_error(e.what());
        return NS_ERR_FORMAT;
    } catch (const std::exception &e) {
        ns::set_error(std::string(fn) + ": " + e.what());
        return NS_ERR_FORMAT;
    }
}

const MetaValue *find_meta(const ns_gguf *g, const char *key) {
    if (!g || !key) return nullptr;
    const auto it = g->meta.find(key);
    return it == g->meta.end() ? nullptr : &it->second;
}

int missing(const char *key) {
    ns::set_error(std::string("missing GGUF metadata: ") + (key ? key : ""));
    return NS_ERR_ARG;
}
}  // namespace

extern "C" int ns_gguf_open(const char *path, int prefetch, ns_gguf **out) {
    if (!path || !out) {
        ns::set_error("ns_gguf_open: null argument");
        return NS_ERR_ARG;
    }
    *out = nullptr;
    auto *g = new ns_gguf;
    g->fd = ::open(path, O_RDONLY);
    if (g->fd < 0) {
        delete g;
        ns::set_error(std::string("cannot open GGUF: ") + path);
        return NS_ERR_IO;
    }
    struct stat st {};
    if (fstat(g->fd, &st) != 0 || st.st_size < 24) {
        delete g;
        ns::set_error("invalid GGUF file");
        return NS_ERR_FORMAT;
    }
    g->size = size_t(st.st_size);
    void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        delete g;
        ns::set_error("mmap GGUF failed");
        return NS_ERR_IO;
    }
    g->map = static_cast<uint8_t *>(m);
    madvise(g->map, g->size, MADV_RANDOM);
    const int rc = guarded("ns_gguf_open", [&] { g->parse(); });
    if (rc != NS_OK) {
        delete g;
        return rc;
    }
    // page the file in ahead of first use, unless the engine's switch says not to
    if (prefetch && !std::getenv("NEUTRON_NO_SSD_PREFETCH")) madvise(g->map, g->size, MADV_WILLNEED);
    *out = g;
    return NS_OK;
}

extern "C" int ns_gguf_close(ns_gguf *g) {
    delete g;
    return NS_OK;
}

extern "C" uint64_t ns_gguf_data_offset(const ns_gguf *g) { return g ? g->data_offset : 0; }
extern "C" uint64_t ns_gguf_file_size(const ns_gguf *g) { return g ? g->size : 0; }
extern "C" const void *ns_gguf_mapped_data(const ns_gguf *g) { return g ? g->map : nullptr; }
extern "C" uint32_t ns_gguf_tensor_count(const ns_gguf *g) { return g ? uint32_t(g->tensors.size()) : 0; }

extern "C" int ns_gguf_tensor(const ns_gguf *g, uint32_t index, ns_gguf_tensor_info *out) {
    if (!g || !out || index >= g->tensors.size()) {
        ns::set_error("ns_gguf_tensor: no such tensor index");
        return NS_ERR_ARG;
    }
    *out = g->tensors[index];
    return NS_OK;
}

extern "C" int ns_gguf_find_tensor(const ns_gguf *g, const char *name, uint32_t *index) {
    if (!g || !name) {
        ns::set_error("ns_gguf_find_tensor: null argument");
        return NS_ERR_ARG;
    }
    const auto it = g->index.find(name);
    if (it == g->index.end()) {
        ns::set_error(std::string("missing tensor: ") + name);
        return NS_ERR_ARG;
    }
    if (index) *index = it->second;
    return NS_OK;
}

extern "C" int ns_gguf_has_meta(const ns_gguf *g, const char *key) { return find_meta(g, key) != nullptr; }

extern "C" int ns_gguf_meta_u64(const ns_gguf *g, const char *key, uint64_t *out) {
    if (!find_meta(g, key)) return missing(key);
    return guarded("ns_gguf_meta_u64", [&] { *out = g->integer(key); });
}

extern "C" int ns_gguf_meta_number(const ns_gguf *g, const char *key, double *out) {
    const MetaValue *v = find_meta(g, key);
    if (!v) return missing(key);
    if (v->type == kF32 || v->type == kF64) {
        *out = v->f;
        return NS_OK;
    }
    // integers go through meta_u64 as in the reference (gguf.cpp:128), so a negative
    // integer reads as its unsigned 64-bit pattern
    return guarded("ns_gguf_meta_number", [&] { *out = double(g->integer(key)); });
}

extern "C" int ns_gguf_meta_string(const ns_gguf *g, const char *key, const char **out) {
    const MetaValue *v = find_meta(g, key);
    if (!v) return missing(key);
    if (v->type != kString) {
        ns::set_error(std::string("metadata is not a string: ") + key);
        return NS_ERR_ARG;
    }
    *out = v->s.c_str();
    return NS_OK;
}

extern "C" int ns_gguf_meta_array(const ns_gguf *g, const char *key, uint32_t *elem_type, uint64_t *count,
                                  const void **data) {
    const MetaValue *v = find_meta(g, key);
    if (!v) return missing(key);
    if (v->type != kArray) {
        ns::set_error(std::string("metadata is not an array: ") + key);
        return NS_ERR_ARG;
    }
    if (elem_type) *elem_type = v->elem;
    if (count) *count = v->count;
    if (data) *data = v->elem == kString ? nullptr : v->raw.data();
    return NS_OK;
}

extern "C" int ns_gguf_ffn_table(const ns_gguf *g, ns_tensor_desc *out, uint32_t capacity, uint32_t *count) {
    if (!g || !count) {
        ns::set_error("ns_gguf_ffn_table: null argument");
        return NS_ERR_ARG;
    }
    *count = uint32_t(g->tensors.size());
    if (!out) return NS_OK;
    if (capacity < g->tensors.size()) {
        ns::set_error("ns_gguf_ffn_table: output table too small");
        return NS_ERR_ARG;
    }
    for (size_t k = 0; k < g->tensors.size(); ++k) {
        const ns_gguf_tensor_info &t = g->tensors[k];
        ns_tensor_desc d{};
        d.source_offset = t.offset;
        d.bytes = t.bytes;
        d.type = t.type;
        d.cols = uint32_t(t.shape[0]);
        d.rows = t.n_dims > 1 ? uint32_t(t.shape[1]) : 1u;
        d.layer = NS_FFN_NONE;
        d.kind = NS_FFN_NONE;
        // blk.<layer>.ffn_{gate,up,down}.weight (Gemma4Model, model.cpp:17)
        const std::string &n = g->names[k];
        static const char *kinds[3] = {"ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"};
        if (n.compare(0, 4, "blk.") == 0) {
            const size_t dot = n.find('.', 4);
            if (dot != std::string::npos && dot > 4 && n.find_first_not_of("0123456789", 4) == dot) {
                const std::string rest = n.substr(dot + 1);
                for (uint32_t kind = 0; kind < 3; ++kind)
                    if (rest == kinds[kind]) {
                        d.layer = uint32_t(std::stoul(n.substr(4, dot - 4)));
                        d.kind = kind;
                    }
            }
        }
        out[k] = d;
    }
    return NS_OK;
}
