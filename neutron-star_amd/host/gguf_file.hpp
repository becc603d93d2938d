// gguf_file.hpp -- C++ layer over the GGUF part of the C ABI with the reference's
// interface (include/neutron/native/gguf.hpp:29-60): GGUF(path, prefetch),
// tensor(name), has_tensor, tensors(), has(key), meta_u64, meta_number,
// meta_string, data_offset, file_size, mapped_data.  Failures throw
// std::runtime_error with the reference's messages.  ffn_tensor_table() gives the
// table the .nsmffn functions take (nsmffn_file.hpp), as the reference's
// ffn_tensors() derives it from the model (metal_ffn.cpp:63-71).
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "ffn_path.hpp"
#include "ns_ffn.h"

namespace neutron::amd {

class GGUF {
public:
    explicit GGUF(const std::string &path, bool prefetch = true) {
        if (ns_gguf_open(path.c_str(), prefetch ? 1 : 0, &g_) != NS_OK) throw std::runtime_error(ns_last_error());
        const uint32_t n = ns_gguf_tensor_count(g_);
        tensors_.reserve(n);
        for (uint32_t i = 0; i < n; ++i) {
            ns_gguf_tensor_info t{};
            ns_gguf_tensor(g_, i, &t);
            Tensor d;
            d.name = t.name;
            d.shape.assign(t.shape, t.shape + t.n_dims);
            d.type = TensorType(t.type);
            d.offset = t.offset;
            d.bytes = t.bytes;
            tensors_.push_back(std::move(d));
        }
    }
    ~GGUF() { ns_gguf_close(g_); }
    GGUF(const GGUF &) = delete;
    GGUF &operator=(const GGUF &) = delete;

    const Tensor &tensor(const std::string &name) const {
        uint32_t i = 0;
        if (ns_gguf_find_tensor(g_, name.c_str(), &i) != NS_OK) throw std::runtime_error(ns_last_error());
        return tensors_[i];
    }
    bool has_tensor(const std::string &name) const { return ns_gguf_find_tensor(g_, name.c_str(), nullptr) == NS_OK; }
    const std::vector<Tensor> &tensors() const { return tensors_; }
    bool has(const std::string &key) const { return ns_gguf_has_meta(g_, key.c_str()) != 0; }
    uint64_t meta_u64(const std::string &key) const {
        uint64_t v = 0;
        if (ns_gguf_meta_u64(g_, key.c_str(), &v) != NS_OK) throw std::runtime_error(ns_last_error());
        return v;
    }
    double meta_number(const std::string &key) const {
        double v = 0;
        if (ns_gguf_meta_number(g_, key.c_str(), &v) != NS_OK) throw std::runtime_error(ns_last_error());
        return v;
    }
    std::string meta_string(const std::string &key) const {
        const char *v = nullptr;
        if (ns_gguf_meta_string(g_, key.c_str(), &v) != NS_OK) throw std::runtime_error(ns_last_error());
        return v;
    }
    size_t data_offset() const { return size_t(ns_gguf_data_offset(g_)); }
    size_t file_size() const { return size_t(ns_gguf_file_size(g_)); }
    const std::byte *mapped_data() const { return static_cast<const std::byte *>(ns_gguf_mapped_data(g_)); }

    // The table for convert_metal_ffn / MetalFfnFile: FFN matrices (blk.<i>.ffn_gate / ffn_up /
    // ffn_down.weight) with their layer and kind, every other tensor NS_FFN_NONE.
    std::vector<ns_tensor_desc> ffn_tensor_table() const {
        uint32_t n = 0;
        if (ns_gguf_ffn_table(g_, nullptr, 0, &n) != NS_OK) throw std::runtime_error(ns_last_error());
        std::vector<ns_tensor_desc> t(n);
        if (ns_gguf_ffn_table(g_, t.data(), n, &n) != NS_OK) throw std::runtime_error(ns_last_error());
        return t;
    }

private:
    ns_gguf *g_ = nullptr;
    std::vector<Tensor> tensors_;
};

}  // namespace neutron::amd
