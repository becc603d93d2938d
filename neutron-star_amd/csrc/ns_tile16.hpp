// ns_tile16.hpp -- the fp16 weight tiles of the prefill GEMM's FP16 mode.
//
// The reference's FP16-accumulation kernels (metal/gemma4.metal:379-383,
// :391-395, :486-490) multiply fp16 tiles of the dequantised weights,
//   Q4_K: half(d*sc*q - dmin*m)   (q4_dequant_32_pair_thread, metal:229-232)
//   Q6_K: half(d*sc*(v - 32))     (q6_dequant_16_thread, metal:415-419)
// with fp16 x and write a half output tile (metal:394, :489).  This build's FP16
// mode takes the same tile values with one change of scale: every weight row r
// carries a power of two c_r, chosen from its largest block factor, so that the
// tile is formed by one packed fp16 FMA straight from the quant bits:
//
//   M_r  = max over the row's super-blocks of max(|d|, |dmin|)  (Q6_K: |d|)
//   c_r  = 2^(-15 - E_r), E_r = ceil(log2 M_r)  (Q6_K: E_r = floor(log2 M_r) + 1, the
//          power of two strictly above M_r; c_r = 1 when M_r = 0)
//   A    = RNE16(d * sc * 2^24 * c_r)    (Q4_K: |A| <= 63 * 2^9; Q6_K, int8 sc down to -128:
//          |A| <= 2^16 * M_r / 2^E_r <= 65504, the fp16 maximum.  With ceil, a row whose
//          largest d is a power of two and whose block has sc = -128, as llama.cpp's
//          quantiser gives every Q6_K block, would put A at -2^16, past fp16's range)
//   B    = RNE16(-dmin * m * c_r)        (Q6_K: RNE16(-32 * d * sc * c_r))
//   F    = RNE16(q * 2^-24 * A + B)      (one rounding: the packed FMA is fused)
//
// q * 2^-24 is the quant itself read as an fp16 subnormal (a mask of the
// packed nibbles / 6-bit values, no conversion).  Then F ~= c_r * w to fp16
// precision, and the GEMM accumulates sum_k F * x in fp32 (CDNA4's MFMA has no
// fp16 accumulator), multiplies by 1/c_r (exact) and rounds the result once to
// fp16 precision (11 significant bits, fp32 exponent range: BASELINE's
// synthetic down outputs reach 1.7e5, past fp16's 65504).  The oracle
// (oracle/ns_oracle.c, nso_f16_tile_*) restates these formulas.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "ns_quant.hpp"

namespace ns {

// Row scale: returns c * 2^24 (the A factor's scale) and 1/c (the output's).
// M is the largest |factor| of the row in fp32 (every fp16 is an fp32 normal);
// above (Q6_K rows) takes the power of two strictly above M instead of ceil(log2 M).
__device__ __forceinline__ void row_scale(float M, float &c24, float &inv_c, bool above) {
    const uint32_t b = __builtin_bit_cast(uint32_t, M);
    const int e = int(b >> 23) - 127 + ((above || (b & 0x7FFFFFu) != 0u) ? 1 : 0);  // E_r
    const bool pos = M > 0.f;
    c24 = pos ? __builtin_bit_cast(float, uint32_t(127 + 9 - e) << 23) : 16777216.0f;
    inv_c = pos ? __builtin_bit_cast(float, uint32_t(127 + 15 + e) << 23) : 1.0f;
}

__device__ __forceinline__ half2_t splat(_Float16 v) { return half2_t{v, v}; }

// One qs dword (elements l..l+3 of groups 2p (low nibbles) and 2p+1 (high)):
// lo[0..1] = F of l..l+3 in group 2p, hi[0..1] the same in group 2p+1.
__device__ __forceinline__ void q4_f16x8(uint32_t w, half2_t Alo, half2_t Blo, half2_t Ahi, half2_t Bhi,
                                         uint32_t (&lo)[2], uint32_t (&hi)[2]) {
    const uint32_t p = __builtin_amdgcn_perm(w, w, 0x03010200u);  // bytes [b0, b2, b1, b3]
    auto f = [](uint32_t q, half2_t A, half2_t B) {
        return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(half2_t, q), A, B));
    };
    lo[0] = f(p & 0x000F000Fu, Alo, Blo);
    lo[1] = f((p >> 8) & 0x000F000Fu, Alo, Blo);
    hi[0] = f((p >> 4) & 0x000F000Fu, Ahi, Bhi);
    hi[1] = f((p >> 12) & 0x000F000Fu, Ahi, Bhi);
}

// Four 6-bit Q6_K values, one per byte of v (elements l..l+3): F of l..l+3.
__device__ __forceinline__ void q6_f16x4(uint32_t v, half2_t A, half2_t B, uint32_t (&out)[2]) {
    auto f = [](uint32_t q, half2_t a, half2_t b) {
        return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(half2_t, q), a, b));
    };
    out[0] = f(__builtin_amdgcn_perm(0u, v, 0x0C010C00u), A, B);  // [b0, 0, b1, 0]
    out[1] = f(__builtin_amdgcn_perm(0u, v, 0x0C030C02u), A, B);  // [b2, 0, b3, 0]
}

}  // namespace ns
