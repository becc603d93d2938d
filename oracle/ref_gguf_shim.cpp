// ref_gguf_shim.cpp -- C entry points over the reference's own GGUF reader.
//
// TEST INFRASTRUCTURE ONLY.  Compiled together with the unmodified reference
// source src/native/gguf.cpp (taken from where it lies under the reference
// checkout, never copied) into oracle/_ref/libns_ref_gguf.so by
// oracle/Makefile.  It opens a file with the reference's GGUF class
// (include/neutron/native/gguf.hpp:29-60) and reports what that class reports,
// turning its exceptions into a status and the exception's message.
#include "neutron/native/gguf.hpp"

#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

using neutron::native::GGUF;

namespace {
void put(char *buf, uint64_t cap, const std::string &s) {
    if (!buf || cap == 0) return;
    const size_t n = s.size() < cap - 1 ? s.size() : size_t(cap - 1);
    std::memcpy(buf, s.data(), n);
    buf[n] = 0;
}

template <class T>
int copy_vec(const GGUF &g, const char *key, void *out, uint64_t cap, uint64_t *count) {
    const auto &v = g.meta<std::vector<T>>(key);
    *count = v.size();
    const uint64_t n = v.size() * sizeof(T);
    if (n > cap) return 2;
    if (n) std::memcpy(out, v.data(), n);
    return 0;
}
}  // namespace

extern "C" void *nsref_gguf_open(const char *path, char *err, uint64_t cap) {
    try {
        return new GGUF(path, false);
    } catch (const std::exception &e) {
        put(err, cap, e.what());
        return nullptr;
    }
}

extern "C" void nsref_gguf_close(void *h) { delete static_cast<GGUF *>(h); }
extern "C" uint64_t nsref_gguf_data_offset(void *h) { return static_cast<GGUF *>(h)->data_offset(); }
extern "C" uint64_t nsref_gguf_file_size(void *h) { return static_cast<GGUF *>(h)->file_size(); }
extern "C" uint32_t nsref_gguf_tensor_count(void *h) { return uint32_t(static_cast<GGUF *>(h)->tensors().size()); }

extern "C" int nsref_gguf_tensor(void *h, uint32_t i, char *name, uint64_t cap, uint32_t *type, uint32_t *ndims,
                                 uint64_t *shape4, uint64_t *offset, uint64_t *bytes) {
    const auto &ts = static_cast<GGUF *>(h)->tensors();
    if (i >= ts.size()) return 1;
    const auto &t = ts[i];
    put(name, cap, t.name);
    *type = uint32_t(t.type);
    *ndims = uint32_t(t.shape.size());
    for (size_t d = 0; d < 4; ++d) shape4[d] = d < t.shape.size() ? t.shape[d] : 0;
    *offset = t.offset;
    *bytes = t.bytes;
    return 0;
}

extern "C" int nsref_gguf_find(void *h, const char *name, char *err, uint64_t cap) {
    try {
        (void)static_cast<GGUF *>(h)->tensor(name);
        return 0;
    } catch (const std::exception &e) {
        put(err, cap, e.what());
        return 1;
    }
}

extern "C" int nsref_gguf_meta_u64(void *h, const char *key, uint64_t *out, char *err, uint64_t cap) {
    try {
        *out = static_cast<GGUF *>(h)->meta_u64(key);
        return 0;
    } catch (const std::exception &e) {
        put(err, cap, e.what());
        return 1;
    }
}

extern "C" int nsref_gguf_meta_number(void *h, const char *key, double *out, char *err, uint64_t cap) {
    try {
        *out = static_cast<GGUF *>(h)->meta_number(key);
        return 0;
    } catch (const std::exception &e) {
        put(err, cap, e.what());
        return 1;
    }
}

extern "C" int nsref_gguf_meta_string(void *h, const char *key, char *out, uint64_t cap) {
    try {
        put(out, cap, static_cast<GGUF *>(h)->meta<std::string>(key));
        return 0;
    } catch (const std::exception &e) {
        put(out, cap, e.what());
        return 1;
    }
}

// Numeric array metadata as raw elements; elem is the GGUF value type
// (0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 10 u64, 11 i64, 12 f64).
extern "C" int nsref_gguf_meta_array(void *h, const char *key, int elem, void *out, uint64_t cap,
                                     uint64_t *count) {
    const GGUF &g = *static_cast<GGUF *>(h);
    try {
        switch (elem) {
            case 0: case 7: return copy_vec<uint8_t>(g, key, out, cap, count);
            case 1: return copy_vec<int8_t>(g, key, out, cap, count);
            case 2: return copy_vec<uint16_t>(g, key, out, cap, count);
            case 3: return copy_vec<int16_t>(g, key, out, cap, count);
            case 4: return copy_vec<uint32_t>(g, key, out, cap, count);
            case 5: return copy_vec<int32_t>(g, key, out, cap, count);
            case 6: return copy_vec<float>(g, key, out, cap, count);
            case 10: return copy_vec<uint64_t>(g, key, out, cap, count);
            case 11: return copy_vec<int64_t>(g, key, out, cap, count);
            case 12: return copy_vec<double>(g, key, out, cap, count);
            default: return 3;
        }
    } catch (const std::exception &) {
        return 1;
    }
}
