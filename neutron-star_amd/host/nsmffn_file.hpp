// nsmffn_file.hpp -- C++ layer over the .nsmffn part of the C ABI with the
// reference's interface (include/neutron/native/metal_ffn.hpp:43-67):
// metal_ffn_fingerprint, convert_metal_ffn, convert_metal_ffn_in_place and the
// MetalFfnFile reader (mapped_data, file_size, offset, reordered).  The reference
// takes its GGUF and Gemma4Model objects; here the caller passes what those
// provide: the GGUF image (or its size and fingerprint) and the tensor table with
// each FFN tensor's layer and kind.  Failures throw std::runtime_error with the
// C ABI's message, as the reference does.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "ns_ffn.h"

namespace neutron::amd {

inline void check_nsmffn(int rc) {
    if (rc != NS_OK) throw std::runtime_error(std::string("neutron-star-amd: ") + ns_last_error());
}

// metal_ffn_fingerprint(gguf) (metal_ffn.cpp:81-90).
inline uint64_t metal_ffn_fingerprint(const void *gguf_head, uint64_t data_offset, uint64_t gguf_size) {
    return ns_nsmffn_fingerprint(gguf_head, data_offset, gguf_size);
}

// convert_metal_ffn(output_path, gguf, model) (metal_ffn.cpp:92-165).
inline void convert_metal_ffn(const std::string &output_path, const void *gguf, uint64_t gguf_size,
                              uint64_t data_offset, const std::vector<ns_tensor_desc> &tensors) {
    check_nsmffn(ns_nsmffn_convert(output_path.c_str(), gguf, gguf_size, data_offset, tensors.data(),
                                   uint32_t(tensors.size())));
}

// convert_metal_ffn_in_place(model_path, metadata_path, gguf, model) (metal_ffn.cpp:167-251).
inline void convert_metal_ffn_in_place(const std::string &model_path, const std::string &metadata_path,
                                       uint64_t data_offset, const std::vector<ns_tensor_desc> &tensors) {
    check_nsmffn(ns_nsmffn_convert_in_place(model_path.c_str(), metadata_path.c_str(), data_offset, tensors.data(),
                                            uint32_t(tensors.size())));
}

// MetalFfnFile (metal_ffn.cpp:253-311).  Tensors are identified by their GGUF
// data offset, as the reference keys its entries by Tensor::offset.
class MetalFfnFile {
public:
    MetalFfnFile(const std::string &path, uint64_t gguf_size, uint64_t gguf_fingerprint,
                 const std::vector<ns_tensor_desc> &tensors) {
        check_nsmffn(ns_nsmffn_open(path.c_str(), gguf_size, gguf_fingerprint, tensors.data(),
                                    uint32_t(tensors.size()), &f_));
    }
    ~MetalFfnFile() { ns_nsmffn_close(f_); }
    MetalFfnFile(const MetalFfnFile &) = delete;
    MetalFfnFile &operator=(const MetalFfnFile &) = delete;

    const std::byte *mapped_data() const { return static_cast<const std::byte *>(ns_nsmffn_data(f_)); }
    size_t file_size() const { return size_t(ns_nsmffn_size(f_)); }
    uint64_t offset(uint64_t source_offset) const { return lookup(source_offset).first; }
    bool reordered(uint64_t source_offset) const { return lookup(source_offset).second; }

private:
    std::pair<uint64_t, bool> lookup(uint64_t source_offset) const {
        uint64_t off = 0;
        int re = 0;
        check_nsmffn(ns_nsmffn_lookup(f_, source_offset, &off, &re));
        return {off, re != 0};
    }
    ns_nsmffn *f_ = nullptr;
};

}  // namespace neutron::amd
