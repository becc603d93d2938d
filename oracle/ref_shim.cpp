// ref_shim.cpp -- C entry points over the reference's own CPU quant path.
//
// TEST INFRASTRUCTURE ONLY.  Compiled together with the unmodified reference
// source src/native/quant.cpp (taken from where it lies under the reference
// checkout, never copied) into oracle/_ref/libns_ref_quant.so by
// oracle/Makefile.  It only builds the reference's Tensor descriptor
// (include/neutron/native/gguf.hpp:20-27) and calls dequant()/dot_row()
// (quant.hpp:5-6), turning the reference's std::runtime_error into a status.
#include "neutron/native/quant.hpp"

#include <cstdint>
#include <stdexcept>

using neutron::native::Tensor;
using neutron::native::TensorType;

static Tensor make(int type, const void *data, uint64_t cols, uint64_t rows) {
    Tensor t;
    t.name = "ref";
    t.shape = {cols, rows};
    t.type = static_cast<TensorType>(type);
    t.data = static_cast<const std::byte *>(data);
    return t;
}

extern "C" int nsref_dequant(int type, const void *data, uint64_t cols, uint64_t rows,
                             uint64_t first, uint64_t count, float *out) {
    const Tensor t = make(type, data, cols, rows);
    try {
        for (uint64_t i = 0; i < count; ++i) out[i] = neutron::native::dequant(t, first + i);
    } catch (const std::runtime_error &) {
        return -1;
    }
    return 0;
}

extern "C" int nsref_dot_row(int type, const void *data, uint64_t cols, uint64_t rows,
                             uint64_t row, const float *x, float *out) {
    const Tensor t = make(type, data, cols, rows);
    try {
        *out = neutron::native::dot_row(t, row, x);
    } catch (const std::exception &) {
        return -1;
    }
    return 0;
}
