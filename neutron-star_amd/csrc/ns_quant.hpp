// ns_quant.hpp -- device-side Q4_K / Q6_K arithmetic shared by every kernel.
//
// Element values follow the reference's src/native/quant.cpp:
//   Q4_K (quant.cpp:9-12): w = d*sc*q - dmin*m.  d*sc and dmin*m are exact in
//     fp32 (11+6 bits), so fmaf(d*sc, q, -dmin*m) is the single rounding of the
//     exact value -- the same fp32 value quant.cpp produces, whatever the
//     compiler's contraction choice.
//   Q6_K (quant.cpp:13-18): w = d*sc*(v-32) needs <= 11+6+6 = 23 bits: exact.
// fp16 tiles hold RNE(fp32 value), as half(d*q - dm) does in metal/gemma4.metal:231.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace ns {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float lo_half(uint32_t w) { return float(__builtin_bit_cast(half2_t, w).x); }
__device__ __forceinline__ float hi_half(uint32_t w) { return float(__builtin_bit_cast(half2_t, w).y); }
__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xffu; }

// Q4_K 6-bit scales and mins.  S0, S1, S2 are scales[0..3], [4..7], [8..11]
// (little-endian dwords).  Returns packed bytes sc[0..3], sc[4..7], m[0..3], m[4..7]
// with the unpack of quant.cpp:11 applied four groups at a time:
//   g < 4:  sc = s[g] & 63,                     m = s[g+4] & 63
//   g >= 4: sc = (s[g+4] & 15) | (s[g-4]>>6)<<4, m = (s[g+4]>>4) | (s[g]>>6)<<4
struct Q4Scales {
    uint32_t sc03, sc47, m03, m47;
};
__device__ __forceinline__ Q4Scales q4_scales(uint32_t S0, uint32_t S1, uint32_t S2) {
    Q4Scales s;
    s.sc03 = S0 & 0x3F3F3F3Fu;
    s.m03 = S1 & 0x3F3F3F3Fu;
    s.sc47 = (S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u);
    s.m47 = ((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
    return s;
}
__device__ __forceinline__ uint32_t q4_sc(const Q4Scales &s, int g) {
    return byte_of(g < 4 ? s.sc03 : s.sc47, g & 3);
}
__device__ __forceinline__ uint32_t q4_m(const Q4Scales &s, int g) {
    return byte_of(g < 4 ? s.m03 : s.m47, g & 3);
}

// fp32 value of one Q4_K weight given D1 = d*sc and M1 = dmin*m (both exact).
// The empty asm keeps the fp32 rounding: without it the compiler may fuse the
// FMA with a following fp16 conversion (v_fma_mixlo_f16), rounding the exact
// value once to fp16 instead of fp32-then-fp16 as the reference does.
__device__ __forceinline__ float q4_value(float D1, float M1, uint32_t q) {
    float v = __builtin_fmaf(D1, float(q), -M1);
    asm volatile("" : "+v"(v));
    return v;
}
// fp32 value of one Q6_K weight given D1 = d*sc (exact) and the 6-bit v.
__device__ __forceinline__ float q6_value(float D1, uint32_t v) { return D1 * float(int(v) - 32); }

// Q6_K: the four 6-bit values of quarters 0..3 for four consecutive l, one byte
// each, from the ql dwords at l (a) and l+32 (b) and the qh dword at l (quant.cpp:16).
struct Q6Quarters {
    uint32_t v0, v1, v2, v3;
};
__device__ __forceinline__ Q6Quarters q6_quarters(uint32_t a, uint32_t b, uint32_t h) {
    Q6Quarters q;
    q.v0 = (a & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
    q.v1 = (b & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
    q.v2 = ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
    q.v3 = ((b >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
    return q;
}

// GeGLU (metal/gemma4.metal:78): 0.5*g*(1 + tanh(z)), z = 0.7978845608028654*g*(1 + 0.044715*g*g).
// Evaluated through the identity 0.5*(1 + tanh(z)) = 1/(1 + exp(-2z)) as g / (1 + 2^(-2z*log2(e))):
// one exp2 and one reciprocal, no cancellation for negative g, and exact limits (g for
// large g, -0 for very negative g).  Within a few fp32 ulps of the tanh form.
__device__ __forceinline__ float gelu_tanh(float g) {
    const float z = 0.7978845608028654f * g * (1.0f + 0.044715f * g * g);
    return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z * -2.8853900817779268f));
}

}  // namespace ns
