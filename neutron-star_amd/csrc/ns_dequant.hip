// ns_dequant.hip -- bit-exact dequantisation check hook and the device-side
// layout converter.
//
// ns_dequant() exposes the exact per-element arithmetic the GEMM tiles use
// (ns_quant.hpp) so it can be compared with the reference's quant.cpp values
// bit for bit: fp32 = quant.cpp's value, fp16 = its round-to-nearest-even.
#include "ns_internal.hpp"
#include "ns_quant.hpp"

namespace ns {
namespace {

__device__ __forceinline__ uint32_t rd8(const uint8_t *w, int type, int layout, uint32_t row, uint32_t kb,
                                        uint32_t nb, uint32_t j) {
    return w[byte_offset(type, layout, row, kb, nb, j)];
}
__device__ __forceinline__ uint32_t rd16(const uint8_t *w, int type, int layout, uint32_t row, uint32_t kb,
                                         uint32_t nb, uint32_t j) {
    return rd8(w, type, layout, row, kb, nb, j) | (rd8(w, type, layout, row, kb, nb, j + 1) << 8);
}
__device__ __forceinline__ uint32_t rd32(const uint8_t *w, int type, int layout, uint32_t row, uint32_t kb,
                                         uint32_t nb, uint32_t j) {
    return rd16(w, type, layout, row, kb, nb, j) | (rd16(w, type, layout, row, kb, nb, j + 2) << 16);
}

// The 32 values of group g (0..7) of super-block kb of `row`, as quant.cpp computes them.
__device__ void group_values(const uint8_t *__restrict__ w, int type, int layout, uint32_t row, uint32_t kb,
                             uint32_t nb, uint32_t g, float (&v)[32]) {
    if (type == Q4_K) {
        const uint32_t hdr = rd32(w, type, layout, row, kb, nb, 0);
        const Q4Scales s = q4_scales(rd32(w, type, layout, row, kb, nb, 4), rd32(w, type, layout, row, kb, nb, 8),
                                     rd32(w, type, layout, row, kb, nb, 12));
        const float D1 = lo_half(hdr) * float(q4_sc(s, g)), M1 = hi_half(hdr) * float(q4_m(s, g));
        for (int l = 0; l < 32; ++l) {
            const uint32_t qb = rd8(w, type, layout, row, kb, nb, 16 + (g / 2) * 32 + l);
            v[l] = q4_value(D1, M1, (g & 1) ? qb >> 4 : qb & 15);
        }
    } else {
        // group g of 32 = half h, quarter q: ql byte lo[l] / lo[l+32], qh byte hi[l]
        const uint32_t h = g / 4, q = g % 4;
        const float d = lo_half(rd16(w, type, layout, row, kb, nb, 208));
        for (int l = 0; l < 32; ++l) {
            const uint32_t a = rd8(w, type, layout, row, kb, nb, h * 64 + l);
            const uint32_t b = rd8(w, type, layout, row, kb, nb, h * 64 + 32 + l);
            const uint32_t hb = rd8(w, type, layout, row, kb, nb, 128 + h * 32 + l);
            const Q6Quarters qq = q6_quarters(a, b, hb);
            const uint32_t vv = q == 0 ? qq.v0 : q == 1 ? qq.v1 : q == 2 ? qq.v2 : qq.v3;
            const int8_t sc = int8_t(rd8(w, type, layout, row, kb, nb, 192 + h * 8 + l / 16 + 2 * q));
            v[l] = q6_value(d * float(sc), vv & 0xffu);
        }
    }
}

// One thread per (row, 32-element group of one super-block).
__global__ void dequant_kernel(const uint8_t *__restrict__ w, int type, int layout, uint32_t cols,
                               uint32_t row0, uint32_t nrows, float *__restrict__ out32,
                               uint16_t *__restrict__ out16) {
    const uint32_t groups = cols / 32;
    const uint64_t idx = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= uint64_t(nrows) * groups) return;
    const uint32_t rr = uint32_t(idx / groups), gi = uint32_t(idx % groups);
    float v[32];
    group_values(w, type, layout, row0 + rr, gi / 8, cols / kQK, gi % 8, v);
    const size_t o = size_t(rr) * cols + size_t(gi) * 32;
    for (int l = 0; l < 32; ++l) {
        if (out32) out32[o + l] = v[l];
        if (out16) out16[o + l] = __builtin_bit_cast(uint16_t, _Float16(v[l]));
    }
}

// Embedding lookup (gemma_q6k_embedding, metal:503-505): out[t][i] = scale * value(ids[t], i),
// one thread per (token, 32-element group).  An id outside [0, rows) writes NaN.
__global__ void embedding_kernel(const uint8_t *__restrict__ w, int type, int layout, uint32_t cols, uint32_t rows,
                                 const int32_t *__restrict__ ids, uint32_t batch, float scale,
                                 float *__restrict__ out) {
    const uint32_t groups = cols / 32;
    const uint64_t idx = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= uint64_t(batch) * groups) return;
    const uint32_t t = uint32_t(idx / groups), gi = uint32_t(idx % groups);
    const int32_t id = ids[t];
    float *o = out + size_t(t) * cols + size_t(gi) * 32;
    if (id < 0 || uint32_t(id) >= rows) {
        for (int l = 0; l < 32; ++l) o[l] = __builtin_nanf("");
        return;
    }
    float v[32];
    group_values(w, type, layout, uint32_t(id), gi / 8, cols / kQK, gi % 8, v);
    for (int l = 0; l < 32; ++l) o[l] = scale * v[l];
}

// One thread per (row, super-block): moves the block's 2-byte units.
__global__ void retile_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int type,
                              int from, int to, uint32_t rows, uint32_t nb) {
    const uint64_t idx = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= uint64_t(rows) * nb) return;
    const uint32_t row = uint32_t(idx / nb), kb = uint32_t(idx % nb);
    const uint32_t bs = block_bytes(type);
    for (uint32_t j = 0; j < bs; j += 2)
        *reinterpret_cast<uint16_t *>(dst + byte_offset(type, to, row, kb, nb, j)) =
            *reinterpret_cast<const uint16_t *>(src + byte_offset(type, from, row, kb, nb, j));
}

}  // namespace

hipError_t launch_dequant(int type, int layout, const uint8_t *w, uint32_t cols, uint32_t rows,
                          uint32_t row0, uint32_t nrows, float *out_f32, uint16_t *out_f16,
                          hipStream_t stream) {
    (void)rows;
    const uint64_t n = uint64_t(nrows) * (cols / 32);
    if (!n) return hipSuccess;
    dequant_kernel<<<dim3(uint32_t((n + 255) / 256)), dim3(256), 0, stream>>>(w, type, layout, cols, row0, nrows,
                                                                              out_f32, out_f16);
    return hipGetLastError();
}

hipError_t launch_embedding(int type, int layout, const uint8_t *w, uint32_t cols, uint32_t rows, const int32_t *ids,
                            uint32_t batch, float scale, float *out, hipStream_t stream) {
    const uint64_t n = uint64_t(batch) * (cols / 32);
    if (!n) return hipSuccess;
    embedding_kernel<<<dim3(uint32_t((n + 255) / 256)), dim3(256), 0, stream>>>(w, type, layout, cols, rows, ids, batch,
                                                                                scale, out);
    return hipGetLastError();
}

hipError_t launch_retile(int type, const uint8_t *src, uint8_t *dst, uint32_t cols, uint32_t rows,
                         int from_layout, int to_layout, hipStream_t stream) {
    const uint32_t nb = cols / kQK;
    const uint64_t n = uint64_t(rows) * nb;
    if (!n) return hipSuccess;
    retile_kernel<<<dim3(uint32_t((n + 255) / 256)), dim3(256), 0, stream>>>(src, dst, type, from_layout,
                                                                            to_layout, rows, nb);
    return hipGetLastError();
}

}  // namespace ns
