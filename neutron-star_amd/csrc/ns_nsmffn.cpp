// ns_nsmffn.cpp -- the .nsmffn v3 weight file: fingerprint, converters and the
// validating reader (host code, no GPU).
//
// File format (the reference's include/neutron/native/metal_ffn.hpp:13-40 and
// src/native/metal_ffn.cpp:19-22), kept byte-compatible so files written by
// either side are interchangeable:
//   * a 65,536-byte header page: the 72-byte header (magic "NSMFFN03",
//     version 3, row tile 64, entry count, header size, model size, model
//     fingerprint, file size, 3 reserved words) followed by one 48-byte entry
//     per GGUF tensor, in GGUF tensor-table order;
//   * every tensor at its GGUF position (data offset + tensor offset); FFN
//     tensors (gate/up/down) are re-laid into 64-row slabs of whole blocks,
//     [slab][super-block][row % 64], all other tensors are byte-identical.
// The fingerprint ties the file to its GGUF: the FNV-1a 64 loop over the
// version (u32 LE), the GGUF file size (u64 LE) and the first min(data offset,
// 16 MiB) bytes of the GGUF (metal_ffn.cpp:81-90), from the reference's start value.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "ns_ffn.h"
#include "ns_internal.hpp"

namespace ns {
namespace {

constexpr char kMagic[8] = {'N', 'S', 'M', 'F', 'F', 'N', '0', '3'};
constexpr uint32_t kVersion = 3;
constexpr uint32_t kHeaderBytes = 65536;
constexpr uint64_t kFingerprintSpan = uint64_t(16) << 20;

struct Header {
    char magic[8];
    uint32_t version, row_tile, entry_count, header_bytes;
    uint64_t model_size, model_fingerprint, file_size;
    uint64_t reserved[3];
};
struct Entry {
    uint32_t layer, kind, type, cols, rows, reserved;
    uint64_t source_offset, offset, bytes;
};
static_assert(sizeof(Header) == 72, "header layout");
static_assert(sizeof(Entry) == 48, "entry layout");

static_assert(sizeof(ns_tensor_desc) == 40, "ns_tensor_desc layout");

struct Error {
    int code;
    std::string msg;
};

uint64_t fnv1a(uint64_t h, const void *data, size_t n) {
    const auto *p = static_cast<const uint8_t *>(data);
    for (size_t i = 0; i < n; ++i) {
        h ^= p[i];
        h *= 1099511628211ull;
    }
    return h;
}

// The reference starts from 1469598103934665603 (metal_ffn.cpp:82), one digit
// short of the standard FNV-1a 64 offset basis 14695981039346656037; files are
// only interchangeable if the same start value is used, so it is kept.
uint64_t fingerprint(const void *head, uint64_t head_bytes, uint64_t gguf_size) {
    uint64_t h = 1469598103934665603ull;
    const uint32_t v = kVersion;
    h = fnv1a(h, &v, sizeof v);
    h = fnv1a(h, &gguf_size, sizeof gguf_size);
    return fnv1a(h, head, size_t(std::min(head_bytes, kFingerprintSpan)));
}

bool is_ffn(const ns_tensor_desc &t) { return t.kind != NS_FFN_NONE; }

// An FFN tensor must be a Q4_K/Q6_K matrix of whole 64-row slabs (metal_ffn.cpp:73-77).
void check_ffn_tensor(const ns_tensor_desc &t, uint32_t index) {
    if (t.cols == 0 || t.cols % kQK || t.rows == 0 || t.rows % kRowTile)
        throw Error{NS_ERR_SHAPE, "Metal FFN tensor has unsupported shape: entry " + std::to_string(index)};
    if (t.type != Q4_K && t.type != Q6_K)
        throw Error{NS_ERR_ARG, "Metal FFN tensor has unsupported type: entry " + std::to_string(index)};
    if (t.bytes != uint64_t(t.rows) * (t.cols / kQK) * block_bytes(int(t.type)))
        throw Error{NS_ERR_SHAPE, "Metal FFN tensor byte count does not match its shape: entry " + std::to_string(index)};
}

std::vector<uint8_t> header_page(const ns_tensor_desc *t, uint32_t count, uint64_t gguf_size, uint64_t fp,
                                 uint64_t data_offset) {
    if (sizeof(Header) + uint64_t(count) * sizeof(Entry) > kHeaderBytes)
        throw Error{NS_ERR_ARG, "Metal FFN header capacity exceeded"};
    std::vector<uint8_t> page(kHeaderBytes, 0);
    Header h{};
    std::memcpy(h.magic, kMagic, 8);
    h.version = kVersion;
    h.row_tile = kRowTile;
    h.entry_count = count;
    h.header_bytes = kHeaderBytes;
    h.model_size = gguf_size;
    h.model_fingerprint = fp;
    h.file_size = gguf_size;
    std::memcpy(page.data(), &h, sizeof h);
    for (uint32_t i = 0; i < count; ++i) {
        if (is_ffn(t[i])) check_ffn_tensor(t[i], i);
        const Entry e{is_ffn(t[i]) ? t[i].layer : NS_FFN_NONE, is_ffn(t[i]) ? t[i].kind : NS_FFN_NONE, t[i].type,
                      t[i].cols, t[i].rows, 0, t[i].source_offset, data_offset + t[i].source_offset, t[i].bytes};
        if (e.offset + e.bytes > gguf_size)
            throw Error{NS_ERR_SHAPE, "tensor outside the GGUF image: entry " + std::to_string(i)};
        std::memcpy(page.data() + sizeof(Header) + size_t(i) * sizeof(Entry), &e, sizeof e);
    }
    return page;
}

// [row][kb] -> [slab][kb][row % 64] for `rows` rows starting at a slab boundary.
void reorder_rows(const uint8_t *src, uint8_t *dst, uint64_t rows, uint64_t nb, uint32_t bb) {
    for (uint64_t r0 = 0; r0 < rows; r0 += kRowTile)
        for (uint64_t kb = 0; kb < nb; ++kb)
            for (uint64_t r = 0; r < kRowTile; ++r)
                std::memcpy(dst + ((r0 / kRowTile * nb + kb) * kRowTile + r) * bb, src + ((r0 + r) * nb + kb) * bb, bb);
}

void pwrite_all(int fd, const void *data, size_t n, uint64_t off) {
    const auto *p = static_cast<const uint8_t *>(data);
    while (n) {
        const ssize_t w = ::pwrite(fd, p, n, off_t(off));
        if (w < 0) {
            if (errno == EINTR) continue;
            throw Error{NS_ERR_IO, std::string("Metal FFN write failed: ") + std::strerror(errno)};
        }
        p += w;
        n -= size_t(w);
        off += uint64_t(w);
    }
}

void pread_all(int fd, void *data, size_t n, uint64_t off) {
    auto *p = static_cast<uint8_t *>(data);
    while (n) {
        const ssize_t r = ::pread(fd, p, n, off_t(off));
        if (r < 0) {
            if (errno == EINTR) continue;
            throw Error{NS_ERR_IO, std::string("Metal FFN read failed: ") + std::strerror(errno)};
        }
        if (r == 0) throw Error{NS_ERR_IO, "unexpected end of Metal FFN source"};
        p += r;
        n -= size_t(r);
        off += uint64_t(r);
    }
}

template <class F>
int guard(const char *fn, F &&body) {
    try {
        body();
        return NS_OK;
    } catch (const Error &e) {
        set_error(std::string(fn) + ": " + e.msg);
        return e.code;
    } catch (const std::exception &e) {
        set_error(std::string(fn) + ": " + e.what());
        return NS_ERR_IO;
    }
}

}  // namespace
}  // namespace ns

using namespace ns;

struct ns_nsmffn {
    int fd = -1;
    uint8_t *map = nullptr;
    size_t size = 0;
    std::unordered_map<uint64_t, Entry> entries;  // keyed by GGUF source offset
};

extern "C" uint64_t ns_nsmffn_fingerprint(const void *gguf_head, uint64_t head_bytes, uint64_t gguf_file_size) {
    return fingerprint(gguf_head, gguf_head ? head_bytes : 0, gguf_file_size);
}

extern "C" int ns_nsmffn_convert(const char *out_path, const void *gguf, uint64_t gguf_size, uint64_t data_offset,
                                 const ns_tensor_desc *tensors, uint32_t count) {
    return guard("ns_nsmffn_convert", [&] {
        if (!out_path || !gguf || (!tensors && count)) throw Error{NS_ERR_ARG, "null argument"};
        if (data_offset > gguf_size) throw Error{NS_ERR_ARG, "data offset past the end of the GGUF"};
        const auto *src = static_cast<const uint8_t *>(gguf);
        const std::vector<uint8_t> page =
            header_page(tensors, count, gguf_size, fingerprint(src, data_offset, gguf_size), data_offset);
        const std::string tmp = std::string(out_path) + ".tmp";
        const int fd = ::open(tmp.c_str(), O_CREAT | O_TRUNC | O_RDWR, 0644);
        if (fd < 0) throw Error{NS_ERR_IO, "cannot create Metal FFN file: " + tmp};
        try {
            if (::ftruncate(fd, off_t(gguf_size)) != 0)
                throw Error{NS_ERR_IO, std::string("cannot size Metal FFN file: ") + std::strerror(errno)};
            pwrite_all(fd, page.data(), page.size(), 0);
            std::vector<uint8_t> buf;
            for (uint32_t i = 0; i < count; ++i) {
                const ns_tensor_desc &t = tensors[i];
                const uint8_t *data = src + data_offset + t.source_offset;
                const uint64_t dst = data_offset + t.source_offset;
                if (is_ffn(t)) {
                    buf.resize(t.bytes);
                    reorder_rows(data, buf.data(), t.rows, t.cols / kQK, block_bytes(int(t.type)));
                    pwrite_all(fd, buf.data(), buf.size(), dst);
                } else {
                    pwrite_all(fd, data, t.bytes, dst);
                }
            }
            if (::fsync(fd) != 0) throw Error{NS_ERR_IO, "Metal FFN fsync failed"};
            ::close(fd);
            if (::rename(tmp.c_str(), out_path) != 0)
                throw Error{NS_ERR_IO, std::string("Metal FFN rename failed: ") + std::strerror(errno)};
        } catch (...) {
            ::close(fd);
            ::unlink(tmp.c_str());
            throw;
        }
    });
}

extern "C" int ns_nsmffn_convert_in_place(const char *model_path, const char *metadata_path, uint64_t data_offset,
                                          const ns_tensor_desc *tensors, uint32_t count) {
    return guard("ns_nsmffn_convert_in_place", [&] {
        if (!model_path || !metadata_path || (!tensors && count)) throw Error{NS_ERR_ARG, "null argument"};
        if (data_offset < kHeaderBytes) throw Error{NS_ERR_ARG, "GGUF metadata area is too small for the Metal header"};
        const int fd = ::open(model_path, O_RDWR);
        if (fd < 0) throw Error{NS_ERR_IO, std::string("cannot open model for in-place Metal conversion: ") + model_path};
        try {
            struct stat st {};
            if (::fstat(fd, &st) != 0) throw Error{NS_ERR_IO, "cannot stat model"};
            const uint64_t size = uint64_t(st.st_size);
            if (data_offset > size) throw Error{NS_ERR_ARG, "data offset past the end of the GGUF"};
            // The GGUF metadata area, kept as a sparse GGUF of the same size beside
            // the model (the loader still needs it once the header page is replaced).
            std::vector<uint8_t> head(data_offset);
            pread_all(fd, head.data(), head.size(), 0);
            const std::vector<uint8_t> page =
                header_page(tensors, count, size, fingerprint(head.data(), head.size(), size), data_offset);
            const std::string mtmp = std::string(metadata_path) + ".tmp";
            const int mfd = ::open(mtmp.c_str(), O_CREAT | O_TRUNC | O_RDWR, 0644);
            if (mfd < 0) throw Error{NS_ERR_IO, "cannot create sparse GGUF metadata file"};
            try {
                if (::ftruncate(mfd, off_t(size)) != 0) throw Error{NS_ERR_IO, "cannot size sparse GGUF metadata file"};
                pwrite_all(mfd, head.data(), head.size(), 0);
                if (::fsync(mfd) != 0) throw Error{NS_ERR_IO, "GGUF metadata fsync failed"};
                ::close(mfd);
                if (::rename(mtmp.c_str(), metadata_path) != 0)
                    throw Error{NS_ERR_IO, std::string("GGUF metadata rename failed: ") + std::strerror(errno)};
            } catch (...) {
                ::close(mfd);
                ::unlink(mtmp.c_str());
                throw;
            }
            // One slab at a time, so the extra memory is one slab of one tensor.
            std::vector<uint8_t> src, dst;
            for (uint32_t i = 0; i < count; ++i) {
                const ns_tensor_desc &t = tensors[i];
                if (!is_ffn(t)) continue;
                const uint64_t nb = t.cols / kQK, bb = block_bytes(int(t.type)), slab = kRowTile * nb * bb;
                src.resize(slab);
                dst.resize(slab);
                for (uint64_t r0 = 0; r0 < t.rows; r0 += kRowTile) {
                    const uint64_t off = data_offset + t.source_offset + r0 * nb * bb;
                    pread_all(fd, src.data(), slab, off);
                    reorder_rows(src.data(), dst.data(), kRowTile, nb, uint32_t(bb));
                    pwrite_all(fd, dst.data(), slab, off);
                }
            }
            pwrite_all(fd, page.data(), page.size(), 0);
            if (::fsync(fd) != 0) throw Error{NS_ERR_IO, "in-place Metal model fsync failed"};
            ::close(fd);
        } catch (...) {
            ::close(fd);
            throw;
        }
    });
}

extern "C" int ns_nsmffn_open(const char *path, uint64_t gguf_size, uint64_t gguf_fingerprint,
                              const ns_tensor_desc *expected, uint32_t count, ns_nsmffn **out) {
    if (out) *out = nullptr;
    auto *f = new ns_nsmffn;
    const int rc = guard("ns_nsmffn_open", [&] {
        if (!path || !out || (!expected && count)) throw Error{NS_ERR_ARG, "null argument"};
        f->fd = ::open(path, O_RDONLY);
        if (f->fd < 0) throw Error{NS_ERR_IO, std::string("cannot open Metal FFN file: ") + path};
        struct stat st {};
        if (::fstat(f->fd, &st) != 0 || uint64_t(st.st_size) < kHeaderBytes)
            throw Error{NS_ERR_FORMAT, std::string("invalid Metal FFN file: ") + path};
        f->size = size_t(st.st_size);
        void *m = ::mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
        if (m == MAP_FAILED) throw Error{NS_ERR_IO, "mmap Metal FFN failed"};
        f->map = static_cast<uint8_t *>(m);
        Header h;
        std::memcpy(&h, f->map, sizeof h);
        // metal_ffn.cpp:264-270
        if (std::memcmp(h.magic, kMagic, 8) != 0 || h.version != kVersion || h.row_tile != kRowTile ||
            h.header_bytes != kHeaderBytes || h.entry_count != count || h.file_size != f->size ||
            h.model_size != gguf_size || h.model_fingerprint != gguf_fingerprint ||
            sizeof(Header) + uint64_t(h.entry_count) * sizeof(Entry) > h.header_bytes)
            throw Error{NS_ERR_FORMAT, "Metal FFN file does not match this GGUF"};
        for (uint32_t i = 0; i < count; ++i) {
            Entry e;
            std::memcpy(&e, f->map + sizeof(Header) + size_t(i) * sizeof(Entry), sizeof e);
            const ns_tensor_desc &t = expected[i];
            const uint32_t layer = is_ffn(t) ? t.layer : NS_FFN_NONE, kind = is_ffn(t) ? t.kind : NS_FFN_NONE;
            // metal_ffn.cpp:274-287
            if (e.layer != layer || e.kind != kind || e.type != t.type || e.cols != t.cols || e.rows != t.rows ||
                e.source_offset != t.source_offset || e.bytes != t.bytes || e.offset > f->size ||
                e.bytes > f->size - e.offset)
                throw Error{NS_ERR_FORMAT, "invalid Metal FFN tensor entry " + std::to_string(i)};
            if (!f->entries.emplace(e.source_offset, e).second)
                throw Error{NS_ERR_FORMAT, "duplicate Metal FFN tensor entry"};
        }
        ::madvise(f->map, f->size, MADV_RANDOM);
        *out = f;
    });
    if (rc != NS_OK) ns_nsmffn_close(f);
    return rc;
}

extern "C" int ns_nsmffn_close(ns_nsmffn *f) {
    if (!f) return NS_OK;
    if (f->map) ::munmap(f->map, f->size);
    if (f->fd >= 0) ::close(f->fd);
    delete f;
    return NS_OK;
}

extern "C" const void *ns_nsmffn_data(const ns_nsmffn *f) { return f ? f->map : nullptr; }
extern "C" uint64_t ns_nsmffn_size(const ns_nsmffn *f) { return f ? f->size : 0; }

extern "C" int ns_nsmffn_lookup(const ns_nsmffn *f, uint64_t source_offset, uint64_t *offset, int *reordered) {
    if (!f || !offset || !reordered) {
        set_error("ns_nsmffn_lookup: null argument");
        return NS_ERR_ARG;
    }
    const auto it = f->entries.find(source_offset);
    if (it == f->entries.end()) {
        set_error("tensor missing from Metal FFN file: source offset " + std::to_string(source_offset));
        return NS_ERR_ARG;
    }
    *offset = it->second.offset;          // MetalFfnFile::offset (metal_ffn.cpp:300-305)
    *reordered = it->second.kind != NS_FFN_NONE;  // MetalFfnFile::reordered (metal_ffn.cpp:307-311)
    return NS_OK;
}
