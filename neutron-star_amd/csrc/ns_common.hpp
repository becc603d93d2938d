// ns_common.hpp -- block formats and weight layouts shared by host and device code.
//
// Q4_K / Q6_K super-blocks hold 256 weights (include/neutron/native/gguf.hpp:13,
// src/native/gguf.cpp:65-69 of the reference: 144 and 210 bytes).
//
// Three byte layouts of a [rows][cols] quantised tensor (nb = cols/256 blocks/row):
//   ROW_MAJOR  GGUF order: block (r, b) at index r*nb + b.
//   NSMFFN     the reference's .nsmffn order (src/native/metal_ffn.cpp:135-149):
//              64-row slabs, [slab][kblock][row%64] whole blocks.
//   CDNA4      this build's lossless re-tile of NSMFFN for wave64 access.  The
//              64 blocks of one (slab, kblock) keep their NSMFFN byte range, but
//              inside it the block is cut into 16-byte chunks and chunk c of row
//              r%64 is stored at (c*64 + r%64)*16, so that one wave64 load
//              instruction (one 16-byte chunk per lane, lane = row) reads 1 KiB
//              of contiguous memory.  Q4_K: 9 chunks (chunk 0 = d, dmin,
//              scales[12]; chunks 1..8 = qs).  Q6_K: 13 chunks (0..7 ql,
//              8..11 qh, 12 scales) followed by the 64 fp16 d values (2 bytes
//              per row at 13*1024 + 2*(r%64)).
#pragma once
#include <cstdint>

namespace ns {

enum Type : int { Q4_K = 12, Q6_K = 14 };
enum Layout : int { ROW_MAJOR = 0, NSMFFN = 1, CDNA4 = 2 };
enum Acc : int { ACC_FP32 = 0, ACC_FP16 = 1 };

constexpr uint32_t kQK = 256;       // weights per super-block
constexpr uint32_t kRowTile = 64;   // .nsmffn slab height (metal_ffn.cpp:21)
constexpr uint32_t kQ4Bytes = 144;
constexpr uint32_t kQ6Bytes = 210;
constexpr uint32_t kQ4Chunks = 9;
constexpr uint32_t kQ6Chunks = 13;

__host__ __device__ constexpr uint32_t block_bytes(int type) {
    return type == Q4_K ? kQ4Bytes : kQ6Bytes;
}

// Index (in blocks) of block (row, kb) for ROW_MAJOR and NSMFFN.
__host__ __device__ inline uint64_t block_index(int layout, uint64_t row, uint64_t kb, uint64_t nb) {
    return layout == ROW_MAJOR ? row * nb + kb : ((row / kRowTile) * nb + kb) * kRowTile + row % kRowTile;
}

// Byte offset of the (slab, kb) region shared by NSMFFN and CDNA4.
__host__ __device__ inline uint64_t region_offset(int type, uint64_t slab, uint64_t kb, uint64_t nb) {
    return (slab * nb + kb) * kRowTile * block_bytes(type);
}

// Byte offset of byte `j` of block (row, kb) in any layout.
__host__ __device__ inline uint64_t byte_offset(int type, int layout, uint64_t row, uint64_t kb,
                                                uint64_t nb, uint32_t j) {
    if (layout != CDNA4) return block_index(layout, row, kb, nb) * block_bytes(type) + j;
    const uint64_t base = region_offset(type, row / kRowTile, kb, nb);
    const uint32_t r = static_cast<uint32_t>(row % kRowTile);
    const uint32_t nchunk = type == Q4_K ? kQ4Chunks : kQ6Chunks;
    const uint32_t c = j / 16;
    if (c < nchunk) return base + (uint64_t(c) * kRowTile + r) * 16 + (j % 16);
    return base + uint64_t(nchunk) * kRowTile * 16 + r * 2 + (j - nchunk * 16);  // Q6_K d
}

}  // namespace ns
