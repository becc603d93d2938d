// ns_gemv.hip -- decode (batch 1) dequant-fused GEMV for gfx950.
//
// Replaces gemma_q4k_mv_fast[_metal], gemma_q6k_mv_fast[_metal] and
// gemma_q4k_gate_up_geglu_mv2[_metal] (metal/gemma4.metal:55-124, selected by
// matmul batch==1 at metal_engine.mm:272 and gate_up_geglu_decode at mm:290).
//
// Work decomposition (wave64, lane = weight row):
//   * the work is the flattened sequence of (64-row slab, super-block) units;
//     each workgroup takes an equal contiguous run of units and splits it
//     evenly over its waves.  The grid (plan_gemv, plan_one_unit) is one slab
//     per 4-wave workgroup for the streaming lm-head, one workgroup (or k) per
//     slab for the one-unit-per-wave instance, else the resident workgroups;
//   * every lane streams its own row's blocks: in the CDNA4 layout each of the
//     9 (Q4_K) or 13 (Q6_K) 16-byte chunk loads of a wave is one contiguous
//     1 KiB transaction; the streaming instance prefetches the next unit into a
//     second register buffer while one is computed;
//   * x is wave-uniform (every lane needs the same 256 values of a block) and
//     is read with scalar loads; per-group sums of x are built across lanes;
//   * a wave writes the slabs it covers whole; slabs cut between waves meet in
//     LDS in wave order, and slabs cut between workgroups are finished by the
//     last workgroup to arrive, which adds the parts in workgroup order, so
//     results are deterministic.
//
// Per super-block the Q4_K dot is factorised as in the reference's
// q4k_mv_block_fast (metal:73):  sum_k w_k x_k = d * sum_g sc_g (sum_l q x)
//   - dmin * sum_g m_g (sum_l x).  The 4-bit q are widened without a convert:
// masking a dword with 0x000F000F leaves two fp16 subnormals q*2^-24 (and
// 0x00F000F0 gives q*2^-20 for the high nibble), which the fp32 FMA reads
// exactly; the 2^24 / 2^20 factors are folded into the group scale.
#include "ns_internal.hpp"
#include "ns_quant.hpp"
#include "ns_rms.hpp"

namespace ns {
namespace {

constexpr uint32_t kWgWaves = 4;   // waves per workgroup of the flattened split

// Largest workgroup (in waves) a kernel instance supports.  Without the
// prefetch buffer every instance fits in 128 VGPRs, 4 waves per SIMD.  The
// streaming (PF) Q4_K and Q6_K instances hold two unit buffers in up to 256
// VGPRs (two waves per SIMD) and run 4-wave workgroups; the PF gate/up pair
// (~190 VGPRs) fits 2 waves per SIMD.
constexpr uint32_t max_wg_waves(int type, bool pair, bool pf) {
    (void)type;
    return !pf ? 16 : pair ? 8 : 4;
}

// ---- block loads --------------------------------------------------------

template <int LAYOUT>
__device__ __forceinline__ void q4_load(const uint8_t *__restrict__ w, uint32_t lane, uint32_t row,
                                        uint32_t slab, uint32_t b, uint32_t nb, u32x4 (&c)[kQ4Chunks]) {
    if constexpr (LAYOUT == CDNA4) {
        const u32x4 *base = reinterpret_cast<const u32x4 *>(w + region_offset(Q4_K, slab, b, nb)) + lane;
#pragma unroll
        for (int i = 0; i < int(kQ4Chunks); ++i) c[i] = __builtin_nontemporal_load(base + i * 64);
    } else {
        const u32x4 *blk = reinterpret_cast<const u32x4 *>(w + block_index(LAYOUT, row, b, nb) * kQ4Bytes);
#pragma unroll
        for (int i = 0; i < int(kQ4Chunks); ++i) c[i] = __builtin_nontemporal_load(blk + i);
    }
}

// Q6_K: c[0..12] = block bytes 0..207 in 16-byte chunks, dbits = fp16 d.
template <int LAYOUT>
__device__ __forceinline__ void q6_load(const uint8_t *__restrict__ w, uint32_t lane, uint32_t row,
                                        uint32_t slab, uint32_t b, uint32_t nb, u32x4 (&c)[kQ6Chunks],
                                        uint32_t &dbits) {
    if constexpr (LAYOUT == CDNA4) {
        const uint8_t *base = w + region_offset(Q6_K, slab, b, nb);
        const u32x4 *p = reinterpret_cast<const u32x4 *>(base) + lane;
#pragma unroll
        for (int i = 0; i < int(kQ6Chunks); ++i) c[i] = __builtin_nontemporal_load(p + i * 64);
        dbits = reinterpret_cast<const uint16_t *>(base + kQ6Chunks * 1024)[lane];
    } else {
        // 210-byte blocks are only 2-byte aligned: assemble dwords from halves.
        const uint16_t *h = reinterpret_cast<const uint16_t *>(w + block_index(LAYOUT, row, b, nb) * kQ6Bytes);
#pragma unroll
        for (int i = 0; i < int(kQ6Chunks); ++i) {
            const uint16_t *s = h + 8 * i;
            c[i] = u32x4{s[0] | (uint32_t(s[1]) << 16), s[2] | (uint32_t(s[3]) << 16),
                         s[4] | (uint32_t(s[5]) << 16), s[6] | (uint32_t(s[7]) << 16)};
        }
        dbits = h[104];
    }
}

// ---- per-block dots -----------------------------------------------------

__device__ __forceinline__ uint32_t comp(const u32x4 &v, int i) { return v[i]; }

// N matrices that share x (1, or 2 for gate/up).  xb: the block's 256 x values
// (wave-uniform); xs[g]: sum of x over group g (32 values).  Interleaving the
// matrices per chunk lets both reuse each scalar-loaded x value at once.
template <int N>
__device__ __forceinline__ void q4_dot(const u32x4 (&c)[N][kQ4Chunks], const float *__restrict__ xb,
                                       const float (&xs)[8], float (&res)[N]) {
    float A[N][8];
#pragma unroll
    for (int n = 0; n < N; ++n)
#pragma unroll
        for (int g = 0; g < 8; ++g) A[n][g] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int p = j >> 1, l0 = 16 * (j & 1);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float *xl = xb + 64 * p + l0 + 4 * t;  // group 2p
            const float *xh = xl + 32;                   // group 2p+1
#pragma unroll
            for (int n = 0; n < N; ++n) {
                const uint32_t wv = comp(c[n][1 + j], t), w8 = wv >> 8;
                const uint32_t lo0 = wv & 0x000F000Fu, hi0 = wv & 0x00F000F0u;
                const uint32_t lo1 = w8 & 0x000F000Fu, hi1 = w8 & 0x00F000F0u;
                float a = A[n][2 * p], h = A[n][2 * p + 1];
                a = __builtin_fmaf(lo_half(lo0), xl[0], a);
                a = __builtin_fmaf(lo_half(lo1), xl[1], a);
                a = __builtin_fmaf(hi_half(lo0), xl[2], a);
                a = __builtin_fmaf(hi_half(lo1), xl[3], a);
                h = __builtin_fmaf(lo_half(hi0), xh[0], h);
                h = __builtin_fmaf(lo_half(hi1), xh[1], h);
                h = __builtin_fmaf(hi_half(hi0), xh[2], h);
                h = __builtin_fmaf(hi_half(hi1), xh[3], h);
                A[n][2 * p] = a;
                A[n][2 * p + 1] = h;
            }
        }
    }
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const float d = lo_half(c[n][0].x), dmin = hi_half(c[n][0].x);
        const Q4Scales s = q4_scales(c[n][0].y, c[n][0].z, c[n][0].w);
        float sq = 0.f, sm = 0.f;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            // low nibbles carry 2^-24, high nibbles 2^-20 (see file comment)
            const float f = (g & 1) ? 1048576.0f : 16777216.0f;
            sq = __builtin_fmaf(float(q4_sc(s, g)) * f, A[n][g], sq);
            sm = __builtin_fmaf(float(q4_m(s, g)), xs[g], sm);
        }
        res[n] = d * sq - dmin * sm;
    }
}

// Q6_K (quant.cpp:13-18): element (half h, quarter q, l) of a super-block is
// v = nibble of ql[64h + 32(q&1) + l] (low for q < 2) | ((qh[32h + l] >> 2q) & 3) << 4
// and uses scale 8h + 2q + l/16; sum (v-32) x = sum v x - 32 sum x over each
// 16-wide scale group.  The 6-bit v are assembled directly as fp16 subnormals
// (as for Q4_K): for the even bytes of a dword, (ql & 0x000F000F) | (qh<<4 &
// 0x00300030) is v * 2^-24 in both halves (quarter 0), and (ql & 0x00F000F0) |
// (qh<<4 & 0x03000300) is v * 2^-20 (quarter 2); quarters 1 and 3 take qh<<2
// and the ql dword at l+32; the odd bytes repeat this on the operands shifted
// right by 8.  22 integer operations then feed 16 mixed-precision FMAs.
__device__ __forceinline__ float q6_dot(const u32x4 (&c)[kQ6Chunks], uint32_t dbits,
                                        const float *__restrict__ xb, const float (&xs)[16]) {
    const float d = lo_half(dbits);
    float A[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) A[i] = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t a = comp(c[4 * h + t], u), b = comp(c[4 * h + 2 + t], u);
                const uint32_t hq = comp(c[8 + 2 * h + t], u);
                const float *x0 = xb + 128 * h + 16 * t + 4 * u;
#pragma unroll
                for (int odd = 0; odd < 2; ++odd) {
                    const uint32_t aa = odd ? a >> 8 : a, bb = odd ? b >> 8 : b;
                    const uint32_t h4 = odd ? hq >> 4 : hq << 4, h2 = odd ? hq >> 6 : hq << 2;
                    const uint32_t e0 = (aa & 0x000F000Fu) | (h4 & 0x00300030u);
                    const uint32_t e2 = (aa & 0x00F000F0u) | (h4 & 0x03000300u);
                    const uint32_t e1 = (bb & 0x000F000Fu) | (h2 & 0x00300030u);
                    const uint32_t e3 = (bb & 0x00F000F0u) | (h2 & 0x03000300u);
                    const float *xo = x0 + odd;  // elements l+odd (lo half) and l+odd+2 (hi half)
                    float &g0 = A[8 * h + 0 + t], &g1 = A[8 * h + 2 + t], &g2 = A[8 * h + 4 + t], &g3 = A[8 * h + 6 + t];
                    g0 = __builtin_fmaf(lo_half(e0), xo[0], g0);
                    g0 = __builtin_fmaf(hi_half(e0), xo[2], g0);
                    g1 = __builtin_fmaf(lo_half(e1), xo[32], g1);
                    g1 = __builtin_fmaf(hi_half(e1), xo[34], g1);
                    g2 = __builtin_fmaf(lo_half(e2), xo[64], g2);
                    g2 = __builtin_fmaf(hi_half(e2), xo[66], g2);
                    g3 = __builtin_fmaf(lo_half(e3), xo[96], g3);
                    g3 = __builtin_fmaf(hi_half(e3), xo[98], g3);
                }
            }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        // group i = 8h + 2q + t: quarters 0, 1 carry 2^-24, quarters 2, 3 carry 2^-20
        const float f = ((i >> 1) & 3) >= 2 ? 1048576.0f : 16777216.0f;
        const float sc = float(int8_t(byte_of(comp(c[12], i >> 2), i & 3)));
        s = __builtin_fmaf(sc, __builtin_fmaf(A[i], f, -32.0f * xs[i]), s);
    }
    return d * s;
}

// q6_dot in two halves, for a caller that holds the block before x is known.  q6_merge6
// forms the 256 six-bit values, one per byte, in 64 dwords: m[4*((2h + t)*4 + u) + j] holds
// quarter j of (h, t, u) for l = 4u .. 4u+3 (byte k = element l + k, the bytes whose two
// 2-bit-and-nibble halves q6_dot assembles as e_j).  q6_dot_merged then takes each e_j as
// one byte permute (bytes odd and 2 + odd to the two fp16 halves: v * 2^-24) and issues
// q6_dot's FMAs in q6_dot's order.  Quarters 2 and 3 carry 2^-24 here instead of 2^-20: every
// product and partial sum of their groups is the same value times 2^-4, which the final factor
// 2^24 (instead of 2^20) undoes exactly, so the result equals q6_dot's bit for bit.
__device__ __forceinline__ uint32_t q6_merge6(uint32_t ql, uint32_t qh, int j) {
    const uint32_t lo = (j >= 2 ? ql >> 4 : ql) & 0x0F0F0F0Fu;
    const uint32_t hb = j == 0 ? (qh << 4) : j == 1 ? (qh << 2) : j == 2 ? qh : (qh >> 2);
    return lo | (hb & 0x30303030u);
}

__device__ __forceinline__ void q6_merge_block(const u32x4 (&c)[kQ6Chunks], uint32_t (&m)[64]) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t a = comp(c[4 * h + t], u), b = comp(c[4 * h + 2 + t], u);
                const uint32_t hq = comp(c[8 + 2 * h + t], u);
                uint32_t *mm = m + 4 * ((2 * h + t) * 4 + u);
                mm[0] = q6_merge6(a, hq, 0);
                mm[1] = q6_merge6(b, hq, 1);
                mm[2] = q6_merge6(a, hq, 2);
                mm[3] = q6_merge6(b, hq, 3);
            }
}

__device__ __forceinline__ float q6_dot_merged(const uint32_t (&m)[64], const u32x4 &scales, uint32_t dbits,
                                               const float *__restrict__ xb, const float (&xs)[16]) {
    float s = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        // half h's eight groups (i = 8h .. 8h+7) are finished before half h+1 starts: s adds
        // the groups in q6_dot's order, and only eight accumulators are live
        float A[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) A[i] = 0.f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                // the x reads of one (t, u) step are not hoisted above the previous step: the
                // 256 broadcast values would otherwise fill the register budget
                __builtin_amdgcn_sched_barrier(0);
                const uint32_t *mm = m + 4 * ((2 * h + t) * 4 + u);
                const float *x0 = xb + 128 * h + 16 * t + 4 * u;
#pragma unroll
                for (int odd = 0; odd < 2; ++odd) {
                    // bytes odd and 2 + odd into the low bytes of the two halves, zero above
                    const uint32_t sel = odd ? 0x0C030C01u : 0x0C020C00u;
                    const uint32_t e0 = __builtin_amdgcn_perm(0u, mm[0], sel);
                    const uint32_t e1 = __builtin_amdgcn_perm(0u, mm[1], sel);
                    const uint32_t e2 = __builtin_amdgcn_perm(0u, mm[2], sel);
                    const uint32_t e3 = __builtin_amdgcn_perm(0u, mm[3], sel);
                    const float *xo = x0 + odd;
                    float &g0 = A[0 + t], &g1 = A[2 + t], &g2 = A[4 + t], &g3 = A[6 + t];
                    g0 = __builtin_fmaf(lo_half(e0), xo[0], g0);
                    g0 = __builtin_fmaf(hi_half(e0), xo[2], g0);
                    g1 = __builtin_fmaf(lo_half(e1), xo[32], g1);
                    g1 = __builtin_fmaf(hi_half(e1), xo[34], g1);
                    g2 = __builtin_fmaf(lo_half(e2), xo[64], g2);
                    g2 = __builtin_fmaf(hi_half(e2), xo[66], g2);
                    g3 = __builtin_fmaf(lo_half(e3), xo[96], g3);
                    g3 = __builtin_fmaf(hi_half(e3), xo[98], g3);
                }
            }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int i = 8 * h + k;
            const float sc = float(int8_t(byte_of(comp(scales, i >> 2), i & 3)));
            s = __builtin_fmaf(sc, __builtin_fmaf(A[k], 16777216.0f, -32.0f * xs[i]), s);
        }
    }
    return lo_half(dbits) * s;
}

// ---- several tokens (the batch 2-4 regime) -------------------------------------
//
// The block is unpacked once and multiplies NT token vectors.  Per token the FMA
// order is that of q4_dot / q6_dot.  x is fp32 or fp16 (XH); an fp16 x value
// feeds the mixed-precision FMA directly, as the weight does.
template <bool XH>
__device__ __forceinline__ float xval(const void *__restrict__ xb, uint32_t i) {
    if constexpr (XH) return float(reinterpret_cast<const _Float16 *>(xb)[i]);
    else return reinterpret_cast<const float *>(xb)[i];
}

template <int N, int NT, bool XH>
__device__ __forceinline__ void q4_dot_mt(const u32x4 (&c)[N][kQ4Chunks], const void *const (&xb)[NT],
                                          const float (&xs)[NT][8], float (&res)[NT][N]) {
    float A[NT][N][8];
#pragma unroll
    for (int k = 0; k < NT; ++k)
#pragma unroll
        for (int n = 0; n < N; ++n)
#pragma unroll
            for (int g = 0; g < 8; ++g) A[k][n][g] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int p = j >> 1, l0 = 16 * (j & 1);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t il = 64 * p + l0 + 4 * t, ih = il + 32;  // groups 2p, 2p+1
#pragma unroll
            for (int n = 0; n < N; ++n) {
                const uint32_t wv = comp(c[n][1 + j], t), w8 = wv >> 8;
                const uint32_t lo0 = wv & 0x000F000Fu, hi0 = wv & 0x00F000F0u;
                const uint32_t lo1 = w8 & 0x000F000Fu, hi1 = w8 & 0x00F000F0u;
#pragma unroll
                for (int k = 0; k < NT; ++k) {
                    float a = A[k][n][2 * p], h = A[k][n][2 * p + 1];
                    a = __builtin_fmaf(lo_half(lo0), xval<XH>(xb[k], il + 0), a);
                    a = __builtin_fmaf(lo_half(lo1), xval<XH>(xb[k], il + 1), a);
                    a = __builtin_fmaf(hi_half(lo0), xval<XH>(xb[k], il + 2), a);
                    a = __builtin_fmaf(hi_half(lo1), xval<XH>(xb[k], il + 3), a);
                    h = __builtin_fmaf(lo_half(hi0), xval<XH>(xb[k], ih + 0), h);
                    h = __builtin_fmaf(lo_half(hi1), xval<XH>(xb[k], ih + 1), h);
                    h = __builtin_fmaf(hi_half(hi0), xval<XH>(xb[k], ih + 2), h);
                    h = __builtin_fmaf(hi_half(hi1), xval<XH>(xb[k], ih + 3), h);
                    A[k][n][2 * p] = a;
                    A[k][n][2 * p + 1] = h;
                }
            }
        }
    }
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const float d = lo_half(c[n][0].x), dmin = hi_half(c[n][0].x);
        const Q4Scales s = q4_scales(c[n][0].y, c[n][0].z, c[n][0].w);
#pragma unroll
        for (int k = 0; k < NT; ++k) {
            float sq = 0.f, sm = 0.f;
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                const float f = (g & 1) ? 1048576.0f : 16777216.0f;
                sq = __builtin_fmaf(float(q4_sc(s, g)) * f, A[k][n][g], sq);
                sm = __builtin_fmaf(float(q4_m(s, g)), xs[k][g], sm);
            }
            res[k][n] = d * sq - dmin * sm;
        }
    }
}

template <int NT, bool XH>
__device__ __forceinline__ void q6_dot_mt(const u32x4 (&c)[kQ6Chunks], uint32_t dbits, const void *const (&xb)[NT],
                                          const float (&xs)[NT][16], float (&res)[NT]) {
    const float d = lo_half(dbits);
    float A[NT][16];
#pragma unroll
    for (int k = 0; k < NT; ++k)
#pragma unroll
        for (int i = 0; i < 16; ++i) A[k][i] = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t a = comp(c[4 * h + t], u), b = comp(c[4 * h + 2 + t], u);
                const uint32_t hq = comp(c[8 + 2 * h + t], u);
                const uint32_t i0 = 128 * h + 16 * t + 4 * u;
#pragma unroll
                for (int odd = 0; odd < 2; ++odd) {
                    const uint32_t aa = odd ? a >> 8 : a, bb = odd ? b >> 8 : b;
                    const uint32_t h4 = odd ? hq >> 4 : hq << 4, h2 = odd ? hq >> 6 : hq << 2;
                    const uint32_t e0 = (aa & 0x000F000Fu) | (h4 & 0x00300030u);
                    const uint32_t e2 = (aa & 0x00F000F0u) | (h4 & 0x03000300u);
                    const uint32_t e1 = (bb & 0x000F000Fu) | (h2 & 0x00300030u);
                    const uint32_t e3 = (bb & 0x00F000F0u) | (h2 & 0x03000300u);
                    const uint32_t io = i0 + odd;  // elements l+odd (lo half) and l+odd+2 (hi half)
#pragma unroll
                    for (int k = 0; k < NT; ++k) {
                        float &g0 = A[k][8 * h + 0 + t], &g1 = A[k][8 * h + 2 + t], &g2 = A[k][8 * h + 4 + t],
                              &g3 = A[k][8 * h + 6 + t];
                        g0 = __builtin_fmaf(lo_half(e0), xval<XH>(xb[k], io + 0), g0);
                        g0 = __builtin_fmaf(hi_half(e0), xval<XH>(xb[k], io + 2), g0);
                        g1 = __builtin_fmaf(lo_half(e1), xval<XH>(xb[k], io + 32), g1);
                        g1 = __builtin_fmaf(hi_half(e1), xval<XH>(xb[k], io + 34), g1);
                        g2 = __builtin_fmaf(lo_half(e2), xval<XH>(xb[k], io + 64), g2);
                        g2 = __builtin_fmaf(hi_half(e2), xval<XH>(xb[k], io + 66), g2);
                        g3 = __builtin_fmaf(lo_half(e3), xval<XH>(xb[k], io + 96), g3);
                        g3 = __builtin_fmaf(hi_half(e3), xval<XH>(xb[k], io + 98), g3);
                    }
                }
            }
#pragma unroll
    for (int k = 0; k < NT; ++k) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float f = ((i >> 1) & 3) >= 2 ? 1048576.0f : 16777216.0f;
            const float sc = float(int8_t(byte_of(comp(c[12], i >> 2), i & 3)));
            s = __builtin_fmaf(sc, __builtin_fmaf(A[k][i], f, -32.0f * xs[k][i]), s);
        }
        res[k] = d * s;
    }
}

// group_sums for fp32 or fp16 x (each lane adds 4 values in fp32).
template <int GROUP, bool XH>
__device__ __forceinline__ void group_sums_x(const void *__restrict__ xb, uint32_t lane, float *xs) {
    float s;
    if constexpr (XH) {
        typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
        const half4_t v = reinterpret_cast<const half4_t *>(xb)[lane];
        s = (float(v.x) + float(v.y)) + (float(v.z) + float(v.w));
    } else {
        const float4 v = reinterpret_cast<const float4 *>(xb)[lane];
        s = (v.x + v.y) + (v.z + v.w);
    }
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    if constexpr (GROUP == 32) s += __shfl_xor(s, 4);
#pragma unroll
    for (int g = 0; g < 256 / GROUP; ++g)
        xs[g] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s), g * (GROUP / 4)));
}

// Lane exchange by DPP (no address registers, no LDS): 0xB1 and 0x4E are quad_perm [1,0,3,2]
// and [2,3,0,1] (lane ^ 1, lane ^ 2), 0x141 row_half_mirror (lane i of 8 takes lane 7 - i).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sums of x over the block's groups of 32 (Q4_K, 8 values) or 16 (Q6_K, 16
// values), returned wave-uniform.  Each lane adds 4 values; the groups are
// completed with cross-lane exchanges and read back with readlane.  After the
// two quad steps every lane of a quad holds the quad's sum, so the mirrored lane
// of the other quad (lane 7 - i) holds the value lane i ^ 4 holds.
template <int GROUP>
__device__ __forceinline__ void group_sums_of(const float4 &v, float *xs) {
    float s = (v.x + v.y) + (v.z + v.w);
    s += dpp_f<0xB1>(s);
    s += dpp_f<0x4E>(s);
    if constexpr (GROUP == 32) s += dpp_f<0x141>(s);
#pragma unroll
    for (int g = 0; g < 256 / GROUP; ++g)
        xs[g] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s), g * (GROUP / 4)));
}

template <int GROUP>
__device__ __forceinline__ void group_sums(const float *__restrict__ xb, uint32_t lane, float *xs) {
    group_sums_of<GROUP>(reinterpret_cast<const float4 *>(xb)[lane], xs);
}

// A streaming loop loads the lane's float4 of x for the group sums together with
// the unit's weights.  Vector memory operations complete in order, so a load of x
// issued after the next unit's prefetch would make the current unit wait for
// the whole prefetch.  (The dot products read x with scalar loads, which are
// counted apart from vector memory operations.)
__device__ __forceinline__ float4 x_lane(const float *__restrict__ x, uint32_t b, uint32_t lane) {
    return reinterpret_cast<const float4 *>(x + size_t(b) * kQK)[lane];
}

// Flattened work: unit i = (slab i / nb, super-block i % nb), i < U = nslabs * nb.
// Workgroup g of G takes units [first(g), first(g+1)) with first(g) = g*q +
// min(g, r), q = U / G, r = U % G, and splits them evenly over its waves, so
// every wave streams the same amount of weights.  With G = nslabs every
// workgroup owns one whole slab and no slab is cut between workgroups.  A wave writes the
// slabs it covers whole.  Parts of slabs cut between waves meet in LDS (wave
// order); a slab cut between workgroups is finished by the last of its
// workgroups to arrive, which adds the workgroup parts in workgroup order.
// Results therefore do not depend on timing.
struct Split {
    uint32_t q, r;
    __device__ __forceinline__ uint32_t first(uint32_t g) const { return g * q + __builtin_elementwise_min(g, r); }
    // the workgroup whose range holds unit i
    __device__ __forceinline__ uint32_t owner(uint32_t i) const {
        const uint32_t big = r * (q + 1);
        return i < big ? i / (q + 1) : r + (i - big) / q;
    }
};

// NormPrologue (ns_internal.hpp) into xn[0..cols) by the whole workgroup (the
// XL 1 form).  Rows of at most one float4 per thread (the 3,840-wide input over
// the 15 waves of a whole-slab workgroup) are held in registers: norm_load issues
// their loads before the kernel requests its first weights, and norm_finish then
// waits for those loads only.  Longer rows take a looped form in norm_finish.
// Every workgroup computes the same values in the same order.
__device__ __forceinline__ bool norm_in_regs(uint32_t cols) { return cols / 4 <= blockDim.x; }

__device__ __forceinline__ void norm_load(RmsRow<1> &rr, const NormPrologue &np, uint32_t cols) {
    if (norm_in_regs(cols))
        rms_row_load<1>(rr, reinterpret_cast<const float4 *>(np.x), reinterpret_cast<const float4 *>(np.wb), nullptr,
                        nullptr, nullptr, cols / 4);
}

__device__ void norm_finish(RmsRow<1> &rr, const NormPrologue &np, uint32_t cols, float *xn, float *part,
                            uint32_t nw) {
    const uint32_t nt = blockDim.x, tid = threadIdx.x;
    if (norm_in_regs(cols)) {
        float4 *xn4 = reinterpret_cast<float4 *>(xn);
        rms_row_finish<1>(rr, false, false, false, cols / 4, np.eps, part,
                          [&](uint32_t j, const float4 &v) { xn4[j] = v; }, [](uint32_t, const float4 &) {});
    } else {
        float s = 0.f;
        for (uint32_t k = tid; k < cols; k += nt) s = __builtin_fmaf(np.x[k], np.x[k], s);
        const float r = rms_factor(wg_sum(s, part, nw), cols, np.eps);
        for (uint32_t k = tid; k < cols; k += nt) xn[k] = (np.x[k] * r) * np.wb[k];
    }
    __syncthreads();
}

// PF: the next unit's weights are loaded while one is computed (the streaming
// regime, many units per wave).  Without PF a wave loads and computes one unit
// at a time; that instance needs fewer registers, so a CU holds twice the waves
// of the gate/up pair, and a grid with one unit per wave issues every load at
// launch.
// XL (the NormPrologue forms; dynamic LDS of cols floats; the dot products
// read x from LDS):
//   1: every workgroup first builds the whole normalised vector (ns::rms_row or
//      a loop); the weights of each wave's first unit are requested before the
//      prologue's arithmetic, so its reads overlap their latency;
//   2: on a whole-slab grid of one super-block per wave (W = nb):
//      the waves of a workgroup together cover x exactly once, so each wave
//      forms only its own block x*w in LDS and its own sum of squares, with no
//      barrier; r = 1/sqrt(mean(x^2) + eps) multiplies the finished dot
//      products in the final combine (W.((x*r)*w) = r * W.(x*w) to rounding).
//      A workgroup barrier at the start would hold every wave until the last
//      one of its workgroup had been dispatched and had its row.
template <int TYPE, int LAYOUT, bool PAIR, bool PF, int XL>
__global__ __launch_bounds__(max_wg_waves(TYPE, PAIR, PF) * 64, PF && !PAIR ? 2 : 1) void gemv_kernel(
    const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, const float *__restrict__ xg,
    float *__restrict__ out, uint32_t rows, uint32_t nb, uint32_t nslabs, float *__restrict__ partial,
    uint32_t *__restrict__ counters, const NormPrologue np) {
    constexpr uint32_t kPlanes = PAIR ? 2 : 1;
    constexpr uint32_t kMaxW = max_wg_waves(TYPE, PAIR, PF);
    __shared__ float lds_part[kMaxW][2][kPlanes][64];
    __shared__ uint32_t lds_slab[kMaxW][2];
    __shared__ float lds_sum[kMaxW];
    extern __shared__ __attribute__((aligned(16))) float lds_x[];
    const uint32_t nw = blockDim.x >> 6;  // waves in this workgroup (<= kMaxW)
    const float *__restrict__ x = XL ? lds_x : xg;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t G = gridDim.x, g = blockIdx.x, U = nslabs * nb;
    const Split sp{U / G, U % G};
    const uint32_t wg0 = sp.first(g), wg1 = sp.first(g + 1), n = wg1 - wg0;
    const uint32_t i0 = wg0 + wave * n / nw, i1 = wg0 + (wave + 1) * n / nw;

    RmsRow<1> rr;
    float4 xv{}, wv{};
    float xsq = 0.f;  // XL 2: this wave's sum of squares of its block of x
    if constexpr (XL == 1) norm_load(rr, np, nb * kQK);
    if constexpr (XL == 2) {
        const uint32_t blk = i0 % nb;
        xv = reinterpret_cast<const float4 *>(np.x)[blk * (kQK / 4) + lane];
        wv = reinterpret_cast<const float4 *>(np.wb)[blk * (kQK / 4) + lane];
    }
    auto prologue = [&]() {
        if constexpr (XL == 1) norm_finish(rr, np, nb * kQK, lds_x, lds_sum, nw);
        if constexpr (XL == 2) {
            const uint32_t blk = i0 % nb;
            reinterpret_cast<float4 *>(lds_x)[blk * (kQK / 4) + lane] =
                float4{xv.x * wv.x, xv.y * wv.y, xv.z * wv.z, xv.w * wv.w};
            float sq = sumsq4(xv, 0.f);
            for (int m = 32; m >= 1; m >>= 1) sq += __shfl_xor(sq, m);
            xsq = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, sq)));
            if (lane == 0) lds_sum[wave] = xsq;
        }
    };
    // XL 2: the factor r applied to finished sums (ts: the sum of squares of all of x)
    auto rms_scale = [&](float ts) { return rms_factor(ts, nb * kQK, np.eps); };

    if (lane < 2) lds_slab[wave][lane] = ~0u;
    float acc0 = 0.f, acc1 = 0.f;
    uint32_t slab = i0 / nb, b = i0 - slab * nb, seg_b0 = b, segi = 0;

    // Segment (slab, blocks seg_b0..b) done: write it if whole, else park it in LDS.
    auto step_done = [&](uint32_t i) {
        if (b == nb - 1 || i + 1 == i1) {
            if (seg_b0 == 0 && b == nb - 1) {
                const uint32_t row = slab * kRowTile + lane;
                if (XL == 2) {  // one wave covers the whole row (nb == 1)
                    const float r = rms_scale(xsq);
                    acc0 *= r;
                    acc1 *= r;
                }
                if (row < rows) {
                    if constexpr (PAIR) out[row] = gelu_tanh(acc0) * acc1;
                    else out[row] = acc0;
                }
            } else {
                lds_part[wave][segi][0][lane] = acc0;
                if constexpr (PAIR) lds_part[wave][segi][kPlanes - 1][lane] = acc1;
                if (lane == 0) lds_slab[wave][segi] = slab;
                segi = 1;
            }
            acc0 = 0.f;
            acc1 = 0.f;
            seg_b0 = 0;
        }
    };
    // Rows past `rows` (ROW_MAJOR tails only) load the last row instead; their results are dropped.
    auto lrow = [&](uint32_t s) { return __builtin_elementwise_min(s * kRowTile + lane, rows - 1); };
    auto advance = [&](uint32_t &s, uint32_t &bb) {
        if (++bb == nb) {
            bb = 0;
            ++s;
        }
    };

    // Each branch requests the first unit's weights, runs the prologue (all
    // threads of the workgroup: it has barriers), then walks the wave's units.
    if constexpr (PF && XL == 0 && !PAIR) {
        // The streaming loop.  Two unit buffers alternate (A, B), so a prefetch
        // lands in the registers its compute reads (a loop-carried buffer is
        // copied at the end of each iteration, and the copy waits for the
        // prefetch), and no load is issued under a condition that later merges:
        // each compute then waits for its own unit's loads only.  x's float4 for
        // the group sums travels with the weights (vector memory operations
        // complete in order; a load of x issued after the prefetch would make
        // the compute wait for the whole prefetch).  (The gate/up pair keeps the
        // loop below: two pair buffers do not fit 256 VGPRs without spills.)
        constexpr int N = PAIR ? 2 : 1;
        struct Buf {
            u32x4 c[N][TYPE == Q4_K ? kQ4Chunks : kQ6Chunks];
            uint32_t d;
            float4 xv;
        };
        auto load = [&](Buf &f, uint32_t s, uint32_t bb) {
            if constexpr (TYPE == Q4_K) {
                q4_load<LAYOUT>(w0, lane, lrow(s), s, bb, nb, f.c[0]);
                if constexpr (PAIR) q4_load<LAYOUT>(w1, lane, lrow(s), s, bb, nb, f.c[N - 1]);
            } else {
                q6_load<LAYOUT>(w0, lane, lrow(s), s, bb, nb, f.c[0], f.d);
            }
            f.xv = x_lane(x, bb, lane);
        };
        // unit i (at slab, b) from buffer f
        auto unit = [&](const Buf &f, uint32_t i) {
            const float *xb = x + size_t(b) * kQK;
            if constexpr (TYPE == Q4_K) {
                float xs[8], r[N];
                group_sums_of<32>(f.xv, xs);
                q4_dot<N>(f.c, xb, xs, r);
                acc0 += r[0];
                if constexpr (PAIR) acc1 += r[N - 1];
            } else {
                float xs[16];
                group_sums_of<16>(f.xv, xs);
                acc0 += q6_dot(f.c[0], f.d, xb, xs);
            }
            step_done(i);
        };
        if (i0 < i1) {
            Buf A, B;
            load(A, slab, b);
            uint32_t i = i0;
            while (true) {
                if (i + 1 == i1) {
                    unit(A, i);
                    break;
                }
                uint32_t ns_ = slab, nbk = b;
                advance(ns_, nbk);
                load(B, ns_, nbk);
                __builtin_amdgcn_sched_barrier(0);
                unit(A, i);
                slab = ns_;
                b = nbk;
                if (++i + 1 == i1) {
                    unit(B, i);
                    break;
                }
                ns_ = slab;
                nbk = b;
                advance(ns_, nbk);
                load(A, ns_, nbk);
                __builtin_amdgcn_sched_barrier(0);
                unit(B, i);
                slab = ns_;
                b = nbk;
                ++i;
            }
        }
    } else if constexpr (TYPE == Q4_K) {
        constexpr int N = PAIR ? 2 : 1;
        const uint8_t *wm[2] = {w0, w1};
        // xv: the lane's float4 of x, loaded with the weights (PF from global memory)
        auto compute = [&](const u32x4(&cc)[N][kQ4Chunks], const float4 &xv) {
            const float *xb = x + size_t(b) * kQK;
            float xs[8], r[N];
            if constexpr (PF && !XL) group_sums_of<32>(xv, xs);
            else group_sums<32>(xb, lane, xs);
            q4_dot<N>(cc, xb, xs, r);
            acc0 += r[0];
            if constexpr (PAIR) acc1 += r[N - 1];
        };
        u32x4 c[N][kQ4Chunks];
        float4 xc{};
        if constexpr (XL) {
            // Unconditional (a wave without units loads the last unit and drops it), so
            // the wait for the prologue's row counts these loads as still outstanding.
            const uint32_t iu = i0 < U ? i0 : U - 1, su = iu / nb, bu = iu - su * nb;
#pragma unroll
            for (int m = 0; m < N; ++m) q4_load<LAYOUT>(wm[m], lane, lrow(su), su, bu, nb, c[m]);
        } else if constexpr (PF) {
            if (i0 < i1) {
#pragma unroll
                for (int m = 0; m < N; ++m) q4_load<LAYOUT>(wm[m], lane, lrow(slab), slab, b, nb, c[m]);
                xc = x_lane(x, b, lane);
            }
        }
        prologue();
        if constexpr (PF) {
            for (uint32_t i = i0; i < i1; ++i) {
                uint32_t ns_ = slab, nbk = b;
                advance(ns_, nbk);
                u32x4 nx[N][kQ4Chunks];
                float4 xn{};
                if (i + 1 < i1) {
#pragma unroll
                    for (int m = 0; m < N; ++m) q4_load<LAYOUT>(wm[m], lane, lrow(ns_), ns_, nbk, nb, nx[m]);
                    if constexpr (!XL) xn = x_lane(x, nbk, lane);
                }
                compute(c, xc);
                step_done(i);
                slab = ns_;
                b = nbk;
#pragma unroll
                for (int m = 0; m < N; ++m)
#pragma unroll
                    for (int k = 0; k < int(kQ4Chunks); ++k) c[m][k] = nx[m][k];
                xc = xn;
            }
        } else if constexpr (XL == 2) {
            compute(c, xc);  // exactly one unit per wave (W = nb, one slab per workgroup)
            step_done(i0);
        } else {
            for (uint32_t i = i0; i < i1; ++i) {
                if (!XL || i != i0)
#pragma unroll
                    for (int m = 0; m < N; ++m) q4_load<LAYOUT>(wm[m], lane, lrow(slab), slab, b, nb, c[m]);
                compute(c, xc);
                step_done(i);
                advance(slab, b);
            }
        }
    } else {
        auto compute = [&](const u32x4(&cc)[kQ6Chunks], uint32_t dd, const float4 &xv) {
            const float *xb = x + size_t(b) * kQK;
            float xs[16];
            if constexpr (PF && !XL) group_sums_of<16>(xv, xs);
            else group_sums<16>(xb, lane, xs);
            acc0 += q6_dot(cc, dd, xb, xs);
        };
        u32x4 c0[kQ6Chunks];
        uint32_t d0 = 0;
        float4 xc{};
        if ((PF || XL) && i0 < i1) {
            q6_load<LAYOUT>(w0, lane, lrow(slab), slab, b, nb, c0, d0);
            if constexpr (PF && !XL) xc = x_lane(x, b, lane);
        }
        prologue();
        if constexpr (PF) {
            for (uint32_t i = i0; i < i1; ++i) {
                uint32_t ns_ = slab, nbk = b;
                advance(ns_, nbk);
                u32x4 n0[kQ6Chunks];
                uint32_t dn = 0;
                float4 xn{};
                if (i + 1 < i1) {
                    q6_load<LAYOUT>(w0, lane, lrow(ns_), ns_, nbk, nb, n0, dn);
                    if constexpr (!XL) xn = x_lane(x, nbk, lane);
                }
                compute(c0, d0, xc);
                step_done(i);
                slab = ns_;
                b = nbk;
#pragma unroll
                for (int k = 0; k < int(kQ6Chunks); ++k) c0[k] = n0[k];
                d0 = dn;
                xc = xn;
            }
        } else {
            for (uint32_t i = i0; i < i1; ++i) {
                if (!XL || i != i0) q6_load<LAYOUT>(w0, lane, lrow(slab), slab, b, nb, c0, d0);
                compute(c0, d0, xc);
                step_done(i);
                advance(slab, b);
            }
        }
    }
    if (n == 0) return;
    const uint32_t s_lo = wg0 / nb, s_hi = (wg1 - 1) / nb;
    // Slabs parked in LDS: at most the workgroup's first and last slab (cut
    // between workgroups) and slabs cut only between its own waves.
    __syncthreads();
    for (uint32_t s = s_lo + wave; s <= s_hi; s += nw) {
        float r0 = 0.f, r1 = 0.f;
        bool any = false;
        for (uint32_t v = 0; v < nw; ++v)
#pragma unroll
            for (uint32_t k = 0; k < 2; ++k)
                if (lds_slab[v][k] == s) {
                    r0 += lds_part[v][k][0][lane];
                    if constexpr (PAIR) r1 += lds_part[v][k][kPlanes - 1][lane];
                    any = true;
                }
        if (!any) continue;  // whole slab, already written
        const uint32_t row = s * kRowTile + lane;
        const bool cut = s * nb < wg0 || (s + 1) * nb > wg1;
        if (cut) {
            // Device-coherent (agent-scope) atomic stores and loads only: the
            // parts bypass the XCD-private L2, so no L2-wide fence is needed.
            // The wait makes the part stores complete before the arrival is
            // counted; the last arrival reads the parts after its atomic returned.
            const uint32_t slot = s == s_lo ? 0u : 1u;
            float *dst = partial + (size_t(g) * 2 + slot) * (kPlanes * 64);
            __hip_atomic_store(&dst[lane], r0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if constexpr (PAIR) __hip_atomic_store(&dst[64 + lane], r1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            const uint32_t gf = sp.owner(s * nb), gl = sp.owner(s * nb + nb - 1);
            uint32_t prev = 0;
            if (lane == 0) prev = __hip_atomic_fetch_add(&counters[s], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            prev = __builtin_amdgcn_readfirstlane(__shfl(prev, 0));
            if (prev != gl - gf) continue;
            r0 = 0.f;
            r1 = 0.f;
            // Parts of workgroups gf..gl, loaded 16 at a time (one round trip for the
            // 15 workgroups of a down-projection slab cut 15 ways) and added in order.
            for (uint32_t h0 = gf; h0 <= gl; h0 += 16) {
                float v0[16], v1[16];
#pragma unroll
                for (uint32_t j = 0; j < 16; ++j) {
                    const uint32_t h = __builtin_elementwise_min(h0 + j, gl);
                    // workgroup h's part of slab s is its first slot unless h began in an earlier slab
                    const uint32_t si = sp.first(h) < s * nb ? 1u : 0u;
                    const float *p = partial + (size_t(h) * 2 + si) * (kPlanes * 64);
                    v0[j] = __hip_atomic_load(&p[lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    v1[j] = PAIR ? __hip_atomic_load(&p[64 + lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
                }
#pragma unroll
                for (uint32_t j = 0; j < 16; ++j)
                    if (h0 + j <= gl) {
                        r0 += v0[j];
                        r1 += v1[j];
                    }
            }
            if (lane == 0) __hip_atomic_store(&counters[s], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if constexpr (XL == 2) {  // whole-slab grid: the workgroup's waves cover all of x
            float ts = 0.f;
            for (uint32_t v = 0; v < nw; ++v) ts += lds_sum[v];
            const float r = rms_scale(ts);
            r0 *= r;
            r1 *= r;
        }
        if (row < rows) {
            if constexpr (PAIR) out[row] = gelu_tanh(r0) * r1;
            else out[row] = r0;
        }
    }
}

// NT tokens: out[t][r] for t < batch (x[t] at x + t*cols; tokens past batch
// repeat the last one and are not written).  PAIR with OUTH writes fp16 h
// (gemma_q4k_gate_up_geglu_mm_f16, metal:102-107); plain writes fp32
// (gemma_q4k/q6k_mm_fast[_f16], metal:125-177).  Same work split as gemv_kernel.
constexpr uint32_t max_wg_waves_mt(int type, bool pair, int nt) { return (type == Q4_K && !pair && nt <= 2) ? 12 : 8; }

template <int TYPE, int LAYOUT, bool PAIR, int NT, bool XH, bool OUTH>
__global__ __launch_bounds__(max_wg_waves_mt(TYPE, PAIR, NT) * 64) void gemv_mt_kernel(
    const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, const void *__restrict__ x, uint32_t batch,
    void *__restrict__ out, uint32_t rows, uint32_t nb, uint32_t nslabs, float *__restrict__ partial,
    uint32_t *__restrict__ counters) {
    constexpr uint32_t kP = (PAIR ? 2 : 1) * NT;  // values per row: plane-major (gate 0..NT-1, up 0..NT-1)
    constexpr uint32_t kMaxW = max_wg_waves_mt(TYPE, PAIR, NT);
    constexpr uint32_t kXBytes = XH ? 2 : 4;
    // The next unit's weights are loaded while one is computed, except for the
    // four-token gate/up pair, whose accumulators leave no registers for them.
    constexpr bool kPrefetch = !(PAIR && NT == 4);
    __shared__ float lds_part[kMaxW][2][kP][64];
    __shared__ uint32_t lds_slab[kMaxW][2];
    const uint32_t nw = blockDim.x >> 6;
    const uint32_t cols = nb * kQK;

    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t G = gridDim.x, g = blockIdx.x, U = nslabs * nb;
    const Split sp{U / G, U % G};
    const uint32_t wg0 = sp.first(g), wg1 = sp.first(g + 1), n = wg1 - wg0;
    const uint32_t i0 = wg0 + wave * n / nw, i1 = wg0 + (wave + 1) * n / nw;
    const uint8_t *xtok[NT];
#pragma unroll
    for (int k = 0; k < NT; ++k)
        xtok[k] = static_cast<const uint8_t *>(x) + size_t(__builtin_elementwise_min(uint32_t(k), batch - 1)) * cols * kXBytes;

    if (lane < 2) lds_slab[wave][lane] = ~0u;
    float acc[kP];
#pragma unroll
    for (int k = 0; k < int(kP); ++k) acc[k] = 0.f;
    uint32_t slab = i0 / nb, b = i0 - slab * nb, seg_b0 = b, segi = 0;

    auto store_out = [&](uint32_t row, const float (&v)[kP]) {
#pragma unroll
        for (int k = 0; k < NT; ++k) {
            if (uint32_t(k) >= batch) break;
            if constexpr (PAIR) {
                const float hv = gelu_tanh(v[k]) * v[NT + k];
                if constexpr (OUTH) static_cast<_Float16 *>(out)[size_t(k) * rows + row] = _Float16(hv);
                else static_cast<float *>(out)[size_t(k) * rows + row] = hv;
            } else {
                static_cast<float *>(out)[size_t(k) * rows + row] = v[k];
            }
        }
    };
    auto step_done = [&](uint32_t i) {
        if (b == nb - 1 || i + 1 == i1) {
            if (seg_b0 == 0 && b == nb - 1) {
                const uint32_t row = slab * kRowTile + lane;
                if (row < rows) store_out(row, acc);
            } else {
#pragma unroll
                for (int k = 0; k < int(kP); ++k) lds_part[wave][segi][k][lane] = acc[k];
                if (lane == 0) lds_slab[wave][segi] = slab;
                segi = 1;
            }
#pragma unroll
            for (int k = 0; k < int(kP); ++k) acc[k] = 0.f;
            seg_b0 = 0;
        }
    };
    auto lrow = [&](uint32_t s) { return __builtin_elementwise_min(s * kRowTile + lane, rows - 1); };
    auto advance = [&](uint32_t &s, uint32_t &bb) {
        if (++bb == nb) {
            bb = 0;
            ++s;
        }
    };

    if (i0 < i1) {
        if constexpr (TYPE == Q4_K) {
            constexpr int N = PAIR ? 2 : 1;
            const uint8_t *wm[2] = {w0, w1};
            u32x4 c[N][kQ4Chunks];
            if constexpr (kPrefetch)
#pragma unroll
                for (int m = 0; m < N; ++m) q4_load<LAYOUT>(wm[m], lane, lrow(slab), slab, b, nb, c[m]);
            for (uint32_t i = i0; i < i1; ++i) {
                uint32_t ns_ = slab, nbk = b;
                advance(ns_, nbk);
                u32x4 nx[N][kQ4Chunks];
                if constexpr (kPrefetch) {
                    if (i + 1 < i1)
#pragma unroll
                        for (int m = 0; m < N; ++m) q4_load<LAYOUT>(wm[m], lane, lrow(ns_), ns_, nbk, nb, nx[m]);
                } else {
#pragma unroll
                    for (int m = 0; m < N; ++m) q4_load<LAYOUT>(wm[m], lane, lrow(slab), slab, b, nb, c[m]);
                }
                const void *xb[NT];
                float xs[NT][8], r[NT][N];
#pragma unroll
                for (int k = 0; k < NT; ++k) {
                    xb[k] = xtok[k] + size_t(b) * kQK * kXBytes;
                    group_sums_x<32, XH>(xb[k], lane, xs[k]);
                }
                q4_dot_mt<N, NT, XH>(c, xb, xs, r);
#pragma unroll
                for (int k = 0; k < NT; ++k) {
                    acc[k] += r[k][0];
                    if constexpr (PAIR) acc[NT + k] += r[k][N - 1];
                }
                step_done(i);
                slab = ns_;
                b = nbk;
                if constexpr (kPrefetch)
#pragma unroll
                    for (int m = 0; m < N; ++m)
#pragma unroll
                        for (int q = 0; q < int(kQ4Chunks); ++q) c[m][q] = nx[m][q];
            }
        } else {
            u32x4 c0[kQ6Chunks];
            uint32_t d0 = 0;
            q6_load<LAYOUT>(w0, lane, lrow(slab), slab, b, nb, c0, d0);
            for (uint32_t i = i0; i < i1; ++i) {
                uint32_t ns_ = slab, nbk = b;
                advance(ns_, nbk);
                u32x4 n0[kQ6Chunks];
                uint32_t dn = 0;
                if (i + 1 < i1) q6_load<LAYOUT>(w0, lane, lrow(ns_), ns_, nbk, nb, n0, dn);
                const void *xb[NT];
                float xs[NT][16], r[NT];
#pragma unroll
                for (int k = 0; k < NT; ++k) {
                    xb[k] = xtok[k] + size_t(b) * kQK * kXBytes;
                    group_sums_x<16, XH>(xb[k], lane, xs[k]);
                }
                q6_dot_mt<NT, XH>(c0, d0, xb, xs, r);
#pragma unroll
                for (int k = 0; k < NT; ++k) acc[k] += r[k];
                step_done(i);
                slab = ns_;
                b = nbk;
#pragma unroll
                for (int q = 0; q < int(kQ6Chunks); ++q) c0[q] = n0[q];
                d0 = dn;
            }
        }
    }
    if (n == 0) return;
    const uint32_t s_lo = wg0 / nb, s_hi = (wg1 - 1) / nb;
    __syncthreads();
    for (uint32_t s = s_lo + wave; s <= s_hi; s += nw) {
        float r[kP];
#pragma unroll
        for (int k = 0; k < int(kP); ++k) r[k] = 0.f;
        bool any = false;
        for (uint32_t v = 0; v < nw; ++v)
#pragma unroll
            for (uint32_t q = 0; q < 2; ++q)
                if (lds_slab[v][q] == s) {
#pragma unroll
                    for (int k = 0; k < int(kP); ++k) r[k] += lds_part[v][q][k][lane];
                    any = true;
                }
        if (!any) continue;  // whole slab, already written
        const uint32_t row = s * kRowTile + lane;
        const bool cut = s * nb < wg0 || (s + 1) * nb > wg1;
        if (cut) {
            // hand-off between workgroups as in gemv_kernel, kP values per row
            const uint32_t slot = s == s_lo ? 0u : 1u;
            float *dst = partial + (size_t(g) * 2 + slot) * (kP * 64);
#pragma unroll
            for (int k = 0; k < int(kP); ++k)
                __hip_atomic_store(&dst[k * 64 + lane], r[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            const uint32_t gf = sp.owner(s * nb), gl = sp.owner(s * nb + nb - 1);
            uint32_t prev = 0;
            if (lane == 0) prev = __hip_atomic_fetch_add(&counters[s], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            prev = __builtin_amdgcn_readfirstlane(__shfl(prev, 0));
            if (prev != gl - gf) continue;
#pragma unroll
            for (int k = 0; k < int(kP); ++k) r[k] = 0.f;
            // parts of workgroups gf..gl, 4 at a time (kP values each), added in order
            for (uint32_t h0 = gf; h0 <= gl; h0 += 4) {
                float v[4][kP];
#pragma unroll
                for (uint32_t j = 0; j < 4; ++j) {
                    const uint32_t h = __builtin_elementwise_min(h0 + j, gl);
                    const uint32_t si = sp.first(h) < s * nb ? 1u : 0u;
                    const float *pp = partial + (size_t(h) * 2 + si) * (kP * 64);
#pragma unroll
                    for (int k = 0; k < int(kP); ++k)
                        v[j][k] = __hip_atomic_load(&pp[k * 64 + lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
#pragma unroll
                for (uint32_t j = 0; j < 4; ++j)
                    if (h0 + j <= gl)
#pragma unroll
                        for (int k = 0; k < int(kP); ++k) r[k] += v[j][k];
            }
            if (lane == 0) __hip_atomic_store(&counters[s], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (row < rows) store_out(row, r);
    }
}

template <int TYPE, int LAYOUT, bool PAIR, bool PF>
constexpr auto kernel_of() {
    return &gemv_kernel<TYPE, LAYOUT, PAIR, PF, 0>;
}

// Resident waves per CU of one kernel instance, and the CU count, per device.
struct DeviceShape {
    int cus = 0;
};
DeviceShape device_shape() {
    static DeviceShape cache[64];
    int dev = 0;
    (void)hipGetDevice(&dev);
    DeviceShape &d = cache[dev & 63];
    if (d.cus == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
        d.cus = cus;
    }
    return d;
}

template <int TYPE, int LAYOUT, bool PAIR, bool PF>
int waves_per_cu() {
    static int cache[64] = {};
    int dev = 0;
    (void)hipGetDevice(&dev);
    int &w = cache[dev & 63];
    if (w == 0) {
        int wgs = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&wgs, kernel_of<TYPE, LAYOUT, PAIR, PF>(), kWgWaves * 64, 0) !=
                hipSuccess || wgs <= 0)
            wgs = 2;
        w = wgs * kWgWaves;
    }
    return w;
}

struct GemvPlan {
    uint32_t nslabs, G, W;  // G workgroups of W waves
};

// G: as many workgroups as the device holds at once (never more than there
// are units).  With slab_per_wg (the batch-1 streaming Q4_K/Q6_K instance) and
// at least two slabs per resident workgroup, one workgroup per slab instead:
// its 4 waves split the slab's super-blocks and meet in LDS, nothing crosses
// workgroups, and the dispatcher gives a CU its next slab as one finishes, so
// CUs that stream faster take more slabs.  Measured on MI355X, 262,144-row
// lm-head (4096 slabs, 2048 resident waves): one slab per workgroup 122.9 us;
// one slab per wave (4096 waves) 125.1 us; the resident grid (two slabs per
// wave) 127.2 us; 12288 waves (slabs cut between workgroups) 130.6 us.
// Tuning::gemv_waves sets the flattened grid's wave count instead.
GemvPlan plan_gemv(uint32_t cols, uint32_t rows, int resident_waves, uint32_t max_waves, uint32_t cus,
                   bool slab_per_wg, const Tuning &t) {
    GemvPlan p;
    const uint32_t nb = cols / kQK;
    p.nslabs = (rows + kRowTile - 1) / kRowTile;
    const uint32_t U = p.nslabs * nb;
    uint32_t cap = uint32_t(resident_waves > 0 ? resident_waves : 2048);
    const int forced = t.gemv_waves;
    if (forced > 0) cap = uint32_t(forced);
    if (slab_per_wg && forced <= 0 && p.nslabs >= 2 * ((cap + kWgWaves - 1) / kWgWaves)) {
        p.W = kWgWaves < nb ? kWgWaves : nb;
        p.G = p.nslabs;
        return p;
    }
    // About one slab per CU (the 15360-row gate/up projections: 240 slabs): one
    // workgroup per slab, as many waves as the CU holds -- nothing crosses
    // workgroups.  Otherwise the flattened split over resident 4-wave workgroups.
    const bool whole = t.gemv_whole != 0 && 4 * p.nslabs >= 3 * cus && p.nslabs <= 2 * cus;
    if (whole) {
        p.W = max_waves < nb ? max_waves : nb;
        p.G = p.nslabs;
        return p;
    }
    p.W = kWgWaves;
    p.G = (cap + kWgWaves - 1) / kWgWaves;
    if (p.G > U) p.G = U;
    return p;
}

template <int TYPE, bool PAIR, bool PF>
int resident_waves(int layout) {
    const int cus = device_shape().cus;
    if (layout == CDNA4) return cus * waves_per_cu<TYPE, CDNA4, PAIR, PF>();
    if (layout == NSMFFN) return cus * waves_per_cu<TYPE, NSMFFN, PAIR, PF>();
    return cus * waves_per_cu<TYPE, ROW_MAJOR, PAIR, PF>();
}

// One unit per wave (the instance without PF): whole slabs per workgroup when a
// slab has at most 16 super-blocks per row, a CU holds that many waves of the
// instance (cu_waves) and the slabs fit one workgroup per CU; k = nb/16 (rounded
// up) workgroups per slab when nb splits evenly and those fit one per CU (the
// 3840 x 15360 down projection: 14.5 -> 14.2 us on MI355X against 15 workgroups
// of 4 waves per slab); else the flattened split over 4-wave workgroups.
GemvPlan plan_one_unit(uint32_t cols, uint32_t rows, uint32_t cus, uint32_t cu_waves, const Tuning &t) {
    GemvPlan p;
    const uint32_t nb = cols / kQK;
    p.nslabs = (rows + kRowTile - 1) / kRowTile;
    const uint32_t k = (nb + 15) / 16;  // workgroups per slab
    if (nb <= 16 && nb <= cu_waves && p.nslabs <= cus) {
        p.W = nb;
        p.G = p.nslabs;
    } else if (t.gemv_qslab != 0 && nb % k == 0 && nb / k <= cu_waves && p.nslabs * k <= cus) {
        // k workgroups of nb/k waves per slab (the 60-block down projection: 4 x 15):
        // 4 parts cross workgroups instead of 15
        p.W = nb / k;
        p.G = p.nslabs * k;
    } else {
        p.W = kWgWaves;
        p.G = (p.nslabs * nb + kWgWaves - 1) / kWgWaves;
    }
    return p;
}

struct GemvChoice {
    GemvPlan plan;
    bool pf;
};

// The prefetching instance streams many units per wave (the lm-head: 61,440
// units).  When the device keeps a wave resident for every unit of the
// instance without the prefetch buffer (the gate/up pair and the down
// projection: 3,600 units), that instance runs with one unit per wave: every
// load is issued at launch and each wave computes as soon as its own unit
// arrives.  Tuning::gemv_pf = 0 / 1 forces either instance.
template <int TYPE, bool PAIR>
GemvChoice choose_gemv(int layout, uint32_t cols, uint32_t rows, const Tuning &t) {
    const uint32_t cus = uint32_t(device_shape().cus);
    const uint32_t nb = cols / kQK, units = ((rows + kRowTile - 1) / kRowTile) * nb;
    const int force = t.gemv_pf;
    const bool one = force == 0 || (force < 0 && int(units) <= resident_waves<TYPE, PAIR, false>(layout));
    if (one) return {plan_one_unit(cols, rows, cus, uint32_t(resident_waves<TYPE, PAIR, false>(layout)) / cus, t), false};
    return {plan_gemv(cols, rows, resident_waves<TYPE, PAIR, true>(layout), max_wg_waves(TYPE, PAIR, true), cus,
                      !PAIR, t),
            true};
}

GemvChoice choose_gemv_for(int type, int layout, bool pair, uint32_t cols, uint32_t rows, const Tuning &t) {
    if (pair) return choose_gemv<Q4_K, true>(layout, cols, rows, t);
    if (type == Q4_K) return choose_gemv<Q4_K, false>(layout, cols, rows, t);
    return choose_gemv<Q6_K, false>(layout, cols, rows, t);
}

template <int TYPE, int LAYOUT, bool PAIR, bool PF>
void launch_layout(const GemvPlan &p, const uint8_t *w, const uint8_t *up, const float *x, float *out, uint32_t cols,
                   uint32_t rows, const Workspace &ws, hipStream_t stream, const NormPrologue *np) {
    const uint32_t nb = cols / kQK;
    const dim3 grid(p.G), block(p.W * 64);
    if constexpr (PAIR) {
        if (np) {
            const size_t lds = size_t(cols) * sizeof(float);
            if constexpr (!PF) {
                // the barrier-free form: one super-block per wave, whole slabs
                if (p.W == nb && p.G == p.nslabs) {
                    gemv_kernel<TYPE, LAYOUT, PAIR, PF, 2><<<grid, block, lds, stream>>>(
                        w, up, x, out, rows, nb, p.nslabs, ws.partial, ws.counters, *np);
                    return;
                }
            }
            gemv_kernel<TYPE, LAYOUT, PAIR, PF, 1><<<grid, block, lds, stream>>>(w, up, x, out, rows, nb, p.nslabs,
                                                                                ws.partial, ws.counters, *np);
            return;
        }
    }
    gemv_kernel<TYPE, LAYOUT, PAIR, PF, 0><<<grid, block, 0, stream>>>(w, up, x, out, rows, nb, p.nslabs,
                                                                      ws.partial, ws.counters, NormPrologue{});
}

template <int TYPE, bool PAIR, bool PF>
void launch_instance(int layout, const GemvPlan &p, const uint8_t *w, const uint8_t *up, const float *x, float *out,
                     uint32_t cols, uint32_t rows, const Workspace &ws, hipStream_t stream, const NormPrologue *np) {
    if (layout == CDNA4) launch_layout<TYPE, CDNA4, PAIR, PF>(p, w, up, x, out, cols, rows, ws, stream, np);
    else if (layout == NSMFFN) launch_layout<TYPE, NSMFFN, PAIR, PF>(p, w, up, x, out, cols, rows, ws, stream, np);
    else launch_layout<TYPE, ROW_MAJOR, PAIR, PF>(p, w, up, x, out, cols, rows, ws, stream, np);
}

template <int TYPE, bool PAIR>
hipError_t launch_typed(int layout, const uint8_t *w, const uint8_t *up, const float *x, float *out,
                        uint32_t cols, uint32_t rows, const Workspace &ws, hipStream_t stream,
                        const NormPrologue *np) {
    const GemvChoice c = choose_gemv<TYPE, PAIR>(layout, cols, rows, ws.tune);
    if (c.pf) launch_instance<TYPE, PAIR, true>(layout, c.plan, w, up, x, out, cols, rows, ws, stream, np);
    else launch_instance<TYPE, PAIR, false>(layout, c.plan, w, up, x, out, cols, rows, ws, stream, np);
    return hipGetLastError();
}

// ---- batch 2-4: one instance per (type, layout, pair, NT, fp16 x) -------------
template <int TYPE, int LAYOUT, bool PAIR, int NT, bool XH>
struct Mt {
    static constexpr auto kernel() { return &gemv_mt_kernel<TYPE, LAYOUT, PAIR, NT, XH, PAIR>; }
    static GemvPlan plan(uint32_t cols, uint32_t rows, const Tuning &t) {
        static int cache[64] = {};  // resident waves per CU, per device
        int dev = 0;
        (void)hipGetDevice(&dev);
        int &w = cache[dev & 63];
        if (w == 0) {
            int wgs = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&wgs, kernel(), kWgWaves * 64, 0) != hipSuccess || wgs <= 0)
                wgs = 2;
            w = wgs * kWgWaves;
        }
        const uint32_t cus = uint32_t(device_shape().cus);
        return plan_gemv(cols, rows, w * int(cus), max_wg_waves_mt(TYPE, PAIR, NT), cus, false, t);
    }
};

template <int TYPE, bool PAIR, int NT, bool XH, class Fn>
auto mt_by_layout(int layout, Fn &&fn) {
    if (layout == CDNA4) return fn(Mt<TYPE, CDNA4, PAIR, NT, XH>{});
    if (layout == NSMFFN) return fn(Mt<TYPE, NSMFFN, PAIR, NT, XH>{});
    return fn(Mt<TYPE, ROW_MAJOR, PAIR, NT, XH>{});
}
template <int TYPE, bool PAIR, bool XH, class Fn>
auto mt_by_nt(uint32_t nt, int layout, Fn &&fn) {
    if constexpr (XH)
        return nt == 2 ? mt_by_layout<TYPE, PAIR, 2, XH>(layout, fn) : mt_by_layout<TYPE, PAIR, 4, XH>(layout, fn);
    else
        return mt_by_layout<TYPE, PAIR, 4, XH>(layout, fn);
}
// The gate/up pair takes fp16 x and writes fp16 h (the reference's only small-batch pair kernel).
template <class Fn>
auto dispatch_mt(int type, int layout, bool pair, uint32_t nt, bool xh, Fn &&fn) {
    if (pair) return mt_by_nt<Q4_K, true, true>(nt, layout, fn);
    if (type == Q4_K) return xh ? mt_by_nt<Q4_K, false, true>(nt, layout, fn) : mt_by_nt<Q4_K, false, false>(nt, layout, fn);
    return xh ? mt_by_nt<Q6_K, false, true>(nt, layout, fn) : mt_by_nt<Q6_K, false, false>(nt, layout, fn);
}

// Tokens per kernel instance.  fp32 x takes the four-token instance for every
// batch: two tokens of fp32 x do not fit the scalar registers the instance keeps
// x in, and the spilled instance is slower than the four-token one (MI355X).
uint32_t mt_tokens(uint32_t batch, bool xh) { return xh && batch <= 2 ? 2u : 4u; }

// ---- the decode FFN block in one launch (mm:571-573), CDNA4 layout -----------------
//
// gate/up + GeGLU writes h, the down projection reads it.  As two launches the down
// projection's weights, which do not depend on h, start streaming only after the last
// gate/up workgroup has drained, and each launch pays its own ramp and tail.  Here one grid
// of NG = F/64 workgroups of W = D/256 waves does both; workgroup g:
//   1. gate/up slab g, one super-block per wave (the whole-slab grid of the decode GEMV:
//      the pair's dot products, optionally with the RMSNorm of x folded in, the waves' parts
//      added in LDS in wave order); wave 0 stores h = gelu(g)*u into the caller's h and, as
//      tagged 64-bit words (value and the launch's tag, see below), into the context's
//      tagged copy;
//   2. as soon as its gate/up weights are consumed, each wave requests its down weights: the
//      down projection's (slab g % DS, column part kq = g / DS, DS = D/64 = 4W), one
//      super-block per wave, so the down weights stream while other workgroups still finish
//      their gate/up slabs;
//   3. each wave reads its 256 values of h (from the DS gate/up slabs of part kq, workgroups
//      kq*DS .. kq*DS + DS-1) as tagged words and re-reads until every tag is current, then
//      forms its part of the down projection; wave 0 stores the workgroup's part as tagged
//      words, and the slab's reducer, the workgroup of part kq = 0, re-reads the other KQ-1
//      parts until they are current and adds them in part order (the order of the decode
//      GEMV's k-workgroups-per-slab plan).
// The tag is the launch's epoch * 64 + 1.  The epoch is a context-owned counter that the
// launch's last slab advances (the multi-layer launch below advances the same counter), so
// words left by an earlier launch carry no current tag; with the tags no counter has to be
// acknowledged, counted and polled before h moves on (28.4 -> 26.7 us per block at the
// model's shape).
// NG = DS * KQ always (F/64 = (D/64) * (F/D)), so every workgroup has exactly one task of
// each kind.  The wait in 3 needs the workgroups it waits on to run: the host launches this
// kernel only when the whole grid fits on the device at once (NG <= CUs x resident
// workgroups per CU), so every workgroup is dispatched whatever else runs on the device:
// work of other kernels ends without waiting on this one and frees its CUs.  The wait is also
// bounded: a wave whose spin limit runs out records it in status and goes on, so every wave
// exits, and the slabs finished after that are written as NaN (the limit is seconds long).
// The last slab to finish clears the counters for the next launch.  Per row and part
// the arithmetic and its order are those of gemv_kernel's whole-slab gate/up and its
// k-workgroups-per-slab down, the plans the two launches take at the model's shape (3840 x
// 15360), so there the results are the same bit for bit.
constexpr uint32_t kBlockMaxW = 16;
constexpr uint32_t kCtrStride = 32;  // one counter per 128-byte line

// A value and its tag as one 64-bit word, stored and loaded at agent scope.
__device__ __forceinline__ void store_tagged(uint64_t *p, float v, uint32_t tag) {
    __hip_atomic_store(p, uint64_t(__builtin_bit_cast(uint32_t, v)) | (uint64_t(tag) << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_tagged(const uint64_t *p) {
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float tagged_value(uint64_t w) { return __builtin_bit_cast(float, uint32_t(w)); }
__device__ __forceinline__ uint32_t tagged_tag(uint64_t w) { return uint32_t(w >> 32); }

// A slab's reducer: the KQ column parts of this lane's output row ([KQ][64] tagged words at
// parts), added in part order from 0, with its own part `own` taken from `mine`; the others
// are read 16 at a time and re-read until their tags are `tag` (bounded by spin_limit polls;
// once status is set nothing waits, and a wait that runs out sets status and records `bit`).
// The order of the sum is that of the last-arriver hand-off it replaces, so the result is the
// same bit for bit.
__device__ __forceinline__ float reduce_tagged_parts(const uint64_t *parts, uint32_t KQ, uint32_t own, float mine,
                                                     uint32_t lane, uint32_t tag, uint32_t spin_limit,
                                                     uint32_t *status, uint32_t *err, uint32_t bit) {
    float sum = 0.f;
    for (uint32_t q0 = 0; q0 < KQ; q0 += 16) {
        uint64_t v[16];
#pragma unroll
        for (uint32_t j = 0; j < 16; ++j) v[j] = load_tagged(parts + __builtin_elementwise_min(q0 + j, KQ - 1) * 64 + lane);
        for (uint32_t it = 0;;) {
            bool ok = true;
#pragma unroll
            for (uint32_t j = 0; j < 16; ++j)
                if (q0 + j < KQ && q0 + j != own) ok = ok && tagged_tag(v[j]) == tag;
            if (__all(ok)) break;
            if (__builtin_amdgcn_readfirstlane(__hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) break;
            __builtin_amdgcn_s_sleep(1);
            if (++it >= spin_limit) {
                if (lane == 0) {
                    __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    record_wait_timeout(err, bit);
                }
                break;
            }
#pragma unroll
            for (uint32_t j = 0; j < 16; ++j)
                v[j] = load_tagged(parts + __builtin_elementwise_min(q0 + j, KQ - 1) * 64 + lane);
        }
#pragma unroll
        for (uint32_t j = 0; j < 16; ++j)
            if (q0 + j < KQ) sum += q0 + j == own ? mine : tagged_value(v[j]);
    }
    return sum;
}

// signal fences keep the compiler from moving memory operations across the barrier; the
// barrier itself does not wait for this wave's global loads in flight
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// 4 waves per SIMD (at most 128 VGPRs) is the occupancy the grid is sized for; without the
// bound the compiler trades the loads in flight for registers
template <int DTYPE, bool NORM>
__global__ __launch_bounds__(kBlockMaxW * 64) __attribute__((amdgpu_waves_per_eu(4, 4))) void block_decode_kernel(
    const uint8_t *__restrict__ wg, const uint8_t *__restrict__ wu, const uint8_t *__restrict__ wd,
    const float *__restrict__ x, const float *__restrict__ normw, float eps, float *__restrict__ h,
    float *__restrict__ y, uint32_t D, uint32_t F, uint32_t *__restrict__ ctr, uint32_t spin_limit,
    uint32_t *__restrict__ err, uint32_t *__restrict__ epoch, uint64_t *__restrict__ htag, uint64_t *__restrict__ ptag) {
    __shared__ __attribute__((aligned(16))) float lds_x[kBlockMaxW * kQK];
    __shared__ float lds_part[kBlockMaxW][2][64];
    __shared__ float lds_sum[kBlockMaxW];
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nbg = D / kQK, nbd = F / kQK, KQ = nbd / nbg, DS = D / kRowTile, W = nbg;
    const uint32_t g = blockIdx.x, kq = g / DS, dslab = g - kq * DS;
    // ctr: slabs_done, status
    uint32_t *slabs_done = ctr, *status = ctr + 1;
    float *xw = lds_x + wave * kQK;  // this wave's 256 inputs
    // the launch's tag: every wave reads the epoch before the last slab can advance it
    const uint32_t E = __builtin_amdgcn_readfirstlane(__hip_atomic_load(epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const uint32_t tg = E * 64u + 1u;

    // ---- 1. gate/up slab g, super-block `wave` ----
    {
        u32x4 c[2][kQ4Chunks];
        const float4 xv = reinterpret_cast<const float4 *>(x + size_t(wave) * kQK)[lane];
        float4 wv{1.f, 1.f, 1.f, 1.f};
        if constexpr (NORM) wv = reinterpret_cast<const float4 *>(normw + size_t(wave) * kQK)[lane];
        q4_load<CDNA4>(wg, lane, 0, g, wave, nbg, c[0]);
        q4_load<CDNA4>(wu, lane, 0, g, wave, nbg, c[1]);
        const float4 xin = NORM ? float4{xv.x * wv.x, xv.y * wv.y, xv.z * wv.z, xv.w * wv.w} : xv;
        reinterpret_cast<float4 *>(xw)[lane] = xin;
        if constexpr (NORM) {
            float sq = sumsq4(xv, 0.f);
            for (int m = 32; m >= 1; m >>= 1) sq += __shfl_xor(sq, m);
            if (lane == 0) lds_sum[wave] = sq;
        }
        float xs[8], r[2];
        group_sums_of<32>(xin, xs);
        q4_dot<2>(c, xw, xs, r);
        lds_part[wave][0][lane] = r[0];
        lds_part[wave][1][lane] = r[1];
    }
    // ---- 2. this wave's down weights: slab dslab, part kq, super-block kq*W + wave ----
    // (wave 0 requests them after its arrival below: the arrival waits for all of wave 0's
    // memory operations to complete)
    const uint32_t b = kq * nbg + wave;
    u32x4 c[DTYPE == Q4_K ? kQ4Chunks : kQ6Chunks];
    uint32_t dbits = 0;
    const auto load_down = [&] {
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if constexpr (DTYPE == Q4_K) {
            q4_load<CDNA4>(wd, lane, 0, dslab, b, nbd, c);
        } else {
            // the 13 chunks only: d is read with h (a register less across the wait)
            const u32x4 *p = reinterpret_cast<const u32x4 *>(wd + region_offset(Q6_K, dslab, b, nbd)) + lane;
#pragma unroll
            for (int i = 0; i < int(kQ6Chunks); ++i) c[i] = __builtin_nontemporal_load(p + i * 64);
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    };
    // Q6_K: the six-bit values are merged while the wave waits for h (q6_merge_block), so only
    // the byte permutes and the FMAs of q6_dot remain once h is complete
    uint32_t m6[64];
    const auto merge_down = [&] {
        if constexpr (DTYPE == Q6_K) q6_merge_block(c, m6);
    };
    if (wave != 0) load_down();
    lds_barrier();
    if (wave != 0) merge_down();
    if (wave == 0) {
        float gs = 0.f, us = 0.f;
        for (uint32_t v = 0; v < W; ++v) {
            gs += lds_part[v][0][lane];
            us += lds_part[v][1][lane];
        }
        if constexpr (NORM) {
            float ts = 0.f;
            for (uint32_t v = 0; v < W; ++v) ts += lds_sum[v];
            const float rs = rms_factor(ts, D, eps);
            gs *= rs;
            us *= rs;
        }
        const float hv = gelu_tanh(gs) * us;
        store_tagged(&htag[g * kRowTile + lane], hv, tg);
        h[g * kRowTile + lane] = hv;  // the caller's h
        load_down();
        merge_down();
    }
    // wave 0's reads of lds_part end before any wave writes it again below
    lds_barrier();
    if constexpr (DTYPE == Q6_K)
        dbits = reinterpret_cast<const uint16_t *>(wd + region_offset(Q6_K, dslab, b, nbd) + kQ6Chunks * 1024)[lane];
    // ---- 3. this wave's 256 values of h, re-read until all carry the launch's tag (bounded;
    // once status is set no wave waits) ----
    const uint64_t *hbase = htag + size_t(b) * kQK;  // wave-uniform: the loads take a scalar base
    uint32_t hl = 4 * lane;
    asm volatile("" : "+v"(hl));
    uint64_t hr[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) hr[k] = load_tagged(hbase + hl + k);
    for (uint32_t it = 0;;) {
        const bool ok = tagged_tag(hr[0]) == tg && tagged_tag(hr[1]) == tg && tagged_tag(hr[2]) == tg &&
                        tagged_tag(hr[3]) == tg;
        if (__all(ok)) break;
        if (__builtin_amdgcn_readfirstlane(__hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) break;
        __builtin_amdgcn_s_sleep(1);
        if (++it >= spin_limit) {
            if (lane == 0) {
                __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                record_wait_timeout(err, kWaitBlock);
            }
            break;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) hr[k] = load_tagged(hbase + hl + k);
    }
    // the Q6_K scale bytes are extracted after the wait, not held through it
    if constexpr (DTYPE == Q6_K) asm volatile("" : "+v"(c[12]));
    const float4 hv{tagged_value(hr[0]), tagged_value(hr[1]), tagged_value(hr[2]), tagged_value(hr[3])};
    // lane-derived LDS addresses are formed again here from an opaque copy of the lane: kept
    // from the start, they would be live across the wait (spilled at four waves per SIMD)
    uint32_t lane_b = lane;
    if constexpr (DTYPE == Q6_K) asm volatile("" : "+v"(lane_b));
    reinterpret_cast<float4 *>(xw)[lane_b] = hv;
    float acc;
    if constexpr (DTYPE == Q4_K) {
        const u32x4(&cc)[1][kQ4Chunks] = reinterpret_cast<const u32x4(&)[1][kQ4Chunks]>(c);
        float xs[8], r[1];
        group_sums_of<32>(hv, xs);
        q4_dot<1>(cc, xw, xs, r);
        acc = r[0];
    } else {
        float xs[16];
        group_sums_of<16>(hv, xs);
        acc = q6_dot_merged(m6, c[12], dbits, xw, xs);
    }
    lds_part[wave][0][lane_b] = acc;
    __syncthreads();
    if (wave == 0) {
        float r0 = 0.f;
        for (uint32_t v = 0; v < W; ++v) r0 += lds_part[v][0][lane];
        store_tagged(&ptag[(size_t(dslab) * KQ + kq) * 64 + lane], r0, tg);
        if (kq == 0) {
            // the slab's reducer: its KQ column parts added in part order
            const float sum = reduce_tagged_parts(ptag + size_t(dslab) * KQ * 64, KQ, 0, r0, lane, tg, spin_limit,
                                                  status, err, kWaitBlock);
            // a part that stopped waiting read h too early: the slab is not a result
            const bool late = __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
            y[dslab * kRowTile + lane] = late ? __builtin_nanf("") : sum;
            if (lane == 0) {
                // every workgroup's part has been read once the last slab is done: nothing reads
                // status or the epoch any more in this launch
                const uint32_t done = __hip_atomic_fetch_add(slabs_done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (done == DS - 1) {
                    __hip_atomic_store(slabs_done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(status, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(epoch, E + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
    }
}

// ---- the decode FFN blocks of consecutive layers in one launch ---------------------------
//
// The block above, looped over the layers of a stack inside one grid: x_{l+1} = y_l, with the
// RMSNorm of x_l (weight normw[l]) folded into layer l's gate/up dot products.  Between two
// launches of the block, the next layer's weights start streaming only after the last
// workgroup has drained, and each launch pays its own ramp.  Here no launch ends between
// layers, and the weights of the next layer stream while this one finishes.
//
// Workgroup g of NG = F/64 has W = D/256 compute waves (one gate/up super-block and one down
// super-block each, the block's split) and one control wave (wave W) that combines the waves'
// parts and hands them to other workgroups.
//
// Hand-off by tagged values.  Every value of h and of the intermediate y is stored together
// with a tag, the launch's epoch * 64 + layer + 1, as one 64-bit agent-scope store; a reader
// loads the 64-bit words and re-reads until every tag is the one it needs.  So no counter has
// to be acknowledged, counted and polled before data moves on: a reader's first loads are
// issued right after the weight loads it needs anyway, complete in order behind them, and
// find the values there in the common case.  The epoch lives in a buffer of its own that the
// launch's last workgroup advances, so a word left by an earlier launch (or zeroed at
// allocation: tag 0, the epoch starts at 1) never carries a current tag, also across graph
// replays.  y's column parts are tagged words too: each slab's reducer (the workgroup of
// part 0) re-reads the others until they are current and adds them in part order.
//
// Per layer l, four workgroup barriers:
//   B5  (l > 0) the control wave has handed off layer l-1: the compute waves request layer
//       l's up weights (the gate weights came into LDS by DMA during layer l-1's down phase,
//       see below), then read x_l = y_{l-1} (tags of layer l-1) and form the gate/up parts;
//   B2  the parts are in LDS and every compute wave has requested its down weights; the
//       control wave combines them (wave order) and stores h tagged;
//   B3  the control wave's reads of the parts are done; the compute waves read their 256
//       values of h (tags of layer l), request the next layer's gate weights into LDS and form
//       their down parts;
//   B4  the down parts are in LDS: the control wave stores the workgroup's part tagged; in the
//       slab's reducer (kq = 0) it then adds the KQ parts in part order into y_l (tagged; the
//       caller's y, plainly, after the last layer); then B5.
// The gate DMA and the up loads stay out of the control wave's way: the DMA is requested
// after the compute waves' h loads and streams during the down dot products; the up loads
// wait for B5, since requested at B4 the loads sat ahead of the control wave's part store in
// the CU's memory pipeline (its acknowledgement took ~8 us).
//
// Buffers are reused across layers safely: layer l+1 writes h and the column parts only after
// reading x_{l+1}, which is complete only after every workgroup has formed its layer-l down
// part (so has read h_l), and y_{l+1}'s slab s only after every workgroup has passed layer
// l+1's gate/up (its KQ parts each read h of DS slabs, together all NG workgroups), so after
// every read of y_l.  Per row the arithmetic and its order are the block's, so the outputs
// equal L launches of the block (and so the two-launch form) bit for bit.
//
// Progress: as the block, the host launches it only when the whole grid is resident at once.
// Every read of tagged values is bounded: a compute wave whose bound runs out sets status and
// records kWaitStack in err; from then on no wave waits (each wait also watches status), and
// every workgroup still does all its steps and exits.  A y slab finished with status set is
// NaN, and every slab of the last layer is finished after the timed-out wave's workgroup has
// counted its last part, so the whole result is NaN.
constexpr uint32_t kStackMaxLayers = 64;

template <int T>
struct DTag {
    static constexpr int value = T;
};

struct StackLayers {
    const uint8_t *wg[kStackMaxLayers];
    const uint8_t *wu[kStackMaxLayers];
    const uint8_t *wd[kStackMaxLayers];
    const float *normw[kStackMaxLayers];
    uint64_t q6_down;  // bit l: layer l's down projection is Q6_K (else Q4_K)
};

template <bool NORM>
__global__ __launch_bounds__(kBlockMaxW * 64) __attribute__((amdgpu_waves_per_eu(4, 4))) void stack_decode_kernel(
    const StackLayers layers, uint32_t L, const float *x0, float eps, float *__restrict__ h, float *y, uint32_t D,
    uint32_t F, uint32_t *__restrict__ ctr, uint32_t *__restrict__ epoch, uint64_t *__restrict__ htag,
    uint64_t *__restrict__ ytag, uint64_t *__restrict__ ptag, uint32_t spin_limit, uint32_t *__restrict__ err) {
    // each compute wave's gate super-block of the next layer, DMA'd from HBM (9 KiB a wave)
    __shared__ __attribute__((aligned(16))) u32x4 lds_gate[kBlockMaxW - 1][kQ4Chunks][64];
    __shared__ __attribute__((aligned(16))) float lds_x[(kBlockMaxW - 1) * kQK];
    __shared__ float lds_part[kBlockMaxW - 1][2][64];
    __shared__ float lds_sum[kBlockMaxW - 1];
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nbg = D / kQK, nbd = F / kQK, KQ = nbd / nbg, DS = D / kRowTile, W = nbg, NG = DS * KQ;
    const uint32_t g = blockIdx.x, kq = g / DS, dslab = g - kq * DS;
    // ctr: status, exits
    uint32_t *status = ctr, *exits = ctr + 1;
    // the launch's epoch: read by every wave before any workgroup can have exited (the last one
    // out advances it)
    const uint32_t E = __builtin_amdgcn_readfirstlane(__hip_atomic_load(epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const auto tag_of = [&](uint32_t l) { return E * 64u + l + 1u; };
    const auto acknowledged = [] {
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    };

    // The two roles run loops of their own with the same barrier sequence (a barrier counts
    // waves, wherever in the program they reach it), so no value of one role is live in the
    // other's code: one shared loop made the compiler spill the compute waves' merged Q6_K
    // bits around the control code.
    if (wave == W) {
        // ---- the control wave ----
        // Its stores and arrivals share the CU's memory pipeline with the compute waves' weight
        // loads; at a higher issue priority they are not held behind loads that were merely
        // ready to issue at the same time.
        __builtin_amdgcn_s_setprio(3);
        for (uint32_t l = 0; l < L; ++l) {
            const uint32_t t = tag_of(l);
            const bool last = l + 1 == L;
            lds_barrier();  // B2: the gate/up parts, wave order
            float gs = 0.f, us = 0.f;
            for (uint32_t v = 0; v < W; ++v) {
                gs += lds_part[v][0][lane];
                us += lds_part[v][1][lane];
            }
            if constexpr (NORM) {
                float ts = 0.f;
                for (uint32_t v = 0; v < W; ++v) ts += lds_sum[v];
                const float rs = rms_factor(ts, D, eps);
                gs *= rs;
                us *= rs;
            }
            const float hv = gelu_tanh(gs) * us;
            store_tagged(&htag[g * kRowTile + lane], hv, t);
            if (last) h[g * kRowTile + lane] = hv;  // the caller's h: the last layer's
            lds_barrier();  // B3: the parts have been read
            lds_barrier();  // B4: the down parts, wave order
            float r0 = 0.f;
            for (uint32_t v = 0; v < W; ++v) r0 += lds_part[v][0][lane];
            store_tagged(&ptag[(size_t(dslab) * KQ + kq) * 64 + lane], r0, t);
            if (kq == 0) {
                // the slab's reducer: its KQ column parts added in part order
                const float sum = reduce_tagged_parts(ptag + size_t(dslab) * KQ * 64, KQ, 0, r0, lane, t, spin_limit,
                                                      status, err, kWaitStack);
                const bool bad = __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
                const float yv = bad ? __builtin_nanf("") : sum;
                if (last) y[dslab * kRowTile + lane] = yv;
                else store_tagged(&ytag[dslab * kRowTile + lane], yv, t);
            }
            if (!last) lds_barrier();  // B5: the hand-off is done; the next layer's loads may go
        }
        // the last workgroup out clears the counters and advances the epoch for the next launch
        // (nothing reads them any more in this one); this wave's stores and increments are
        // performed before its exit is counted, so none can land after the clear
        acknowledged();
        if (lane == 0) {
            const uint32_t done = __hip_atomic_fetch_add(exits, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (done == NG - 1) {
                __hip_atomic_store(status, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(epoch, E + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(exits, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        return;
    }

    // ---- a compute wave: gate/up super-block `wave` of slab g, down super-block kq*W + wave ----
    float *xw = lds_x + wave * kQK;  // this wave's 256 inputs
    const uint32_t b = kq * nbg + wave;
    // Lane-derived addresses are formed again at each use from an opaque copy of the lane:
    // hoisted out of the layer loop they would stay live through every layer.
    const auto opaque_lane = [&] {
        uint32_t v = lane;
        asm volatile("" : "+v"(v));
        return v;
    };
    u32x4 cg[2][kQ4Chunks];
    const auto load_up = [&](uint32_t l) {
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        q4_load<CDNA4>(layers.wu[l], opaque_lane(), 0, g, wave, nbg, cg[1]);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    };
    // Layer l's gate super-block into this wave's LDS slot by DMA: instruction i writes chunk
    // i of the 64 rows, lane L's 16 bytes at lds_gate[wave][i][L], the bytes q4_load would put
    // in lane L's register.  Lane L later reads back only what it wrote itself.
    const auto dma_gate = [&](uint32_t l) {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(layers.wg[l]), 0, int(F * nbg * kQ4Bytes), 0x00020000);
        const uint32_t base = uint32_t(region_offset(Q4_K, g, wave, nbg));
        const uint32_t vo = opaque_lane() * 16;
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
        for (int i = 0; i < int(kQ4Chunks); ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)&lds_gate[wave][i][0],
                                                     16, vo, base + uint32_t(i) * 1024, 0, 0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    };
    // Re-reads this lane's 4 tagged words at p until the whole wave holds tag `want` (bounded;
    // see Progress above).  v holds a first read already issued.
    const auto settle = [&](const uint64_t *p, uint64_t (&v)[4], uint32_t want) {
        uint32_t it = 0;
        for (;;) {
            const bool ok = tagged_tag(v[0]) == want && tagged_tag(v[1]) == want && tagged_tag(v[2]) == want &&
                            tagged_tag(v[3]) == want;
            if (__all(ok)) return;
            if (__builtin_amdgcn_readfirstlane(__hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)))
                return;  // a wait elsewhere ran out: no more waiting
            __builtin_amdgcn_s_sleep(1);
            if (++it >= spin_limit) {
                if (lane == 0) {
                    __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    record_wait_timeout(err, kWaitStack);
                }
                return;
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] = load_tagged(p + k);
        }
    };
    // One layer, per down type: the type branch encloses the whole layer, so that no value
    // crosses from one layer to the next.  Register-held weights requested at the end of the
    // previous iteration would be live across the loop's back edge, and the compiler spilled
    // them: the up weights are requested first in the layer instead.
    const auto layer = [&](uint32_t l, auto tag) {
        constexpr bool q6 = decltype(tag)::value == Q6_K;
        const uint8_t *wd = layers.wd[l];
        const uint32_t t = tag_of(l);
        if (l > 0) lds_barrier();  // B5: this workgroup's hand-off of layer l-1 is done
        load_up(l);
        u32x4 c[q6 ? kQ6Chunks : kQ4Chunks];
        uint32_t m6[q6 ? 64 : 1];
        uint32_t dbits = 0;
        {
            // ---- gate/up slab g, super-block `wave` (the block's step 1) ----
            const uint32_t lane = opaque_lane();
            float4 xv;
            if (l == 0) {
                xv = reinterpret_cast<const float4 *>(x0 + size_t(wave) * kQK)[lane];
            } else {
                // x_l = y_{l-1}: its tagged words, read behind the up weights
                const uint64_t *xp = ytag + size_t(wave) * kQK + 4 * lane;
                uint64_t xr[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) xr[k] = load_tagged(xp + k);
                settle(xp, xr, t - 1u);
                xv = float4{tagged_value(xr[0]), tagged_value(xr[1]), tagged_value(xr[2]), tagged_value(xr[3])};
            }
            float4 wv{1.f, 1.f, 1.f, 1.f};
            if constexpr (NORM) wv = reinterpret_cast<const float4 *>(layers.normw[l] + size_t(wave) * kQK)[lane];
            const float4 xin = NORM ? float4{xv.x * wv.x, xv.y * wv.y, xv.z * wv.z, xv.w * wv.w} : xv;
            reinterpret_cast<float4 *>(xw)[lane] = xin;
            if constexpr (NORM) {
                float sq = sumsq4(xv, 0.f);
                for (int m = 32; m >= 1; m >>= 1) sq += __shfl_xor(sq, m);
                if (lane == 0) lds_sum[wave] = sq;
            }
            float xs[8], r[2];
            group_sums_of<32>(xin, xs);
            // the gate chunks DMA'd into LDS are there once this wave's earlier memory operations
            // are done (the up weights and x, issued after the DMA, are needed now anyway)
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
            for (int i = 0; i < int(kQ4Chunks); ++i) cg[0][i] = lds_gate[wave][i][lane];
            q4_dot<2>(cg, xw, xs, r);
            lds_part[wave][0][lane] = r[0];
            lds_part[wave][1][lane] = r[1];
            // ---- this wave's down weights: slab dslab, part kq, super-block kq*W + wave ----
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            const uint32_t ld = opaque_lane();
            if constexpr (q6) {
                const uint8_t *base = wd + region_offset(Q6_K, dslab, b, nbd);
                const u32x4 *p = reinterpret_cast<const u32x4 *>(base) + ld;
#pragma unroll
                for (int i = 0; i < int(kQ6Chunks); ++i) c[i] = __builtin_nontemporal_load(p + i * 64);
                dbits = reinterpret_cast<const uint16_t *>(base + kQ6Chunks * 1024)[ld];
            } else {
                q4_load<CDNA4>(wd, ld, 0, dslab, b, nbd, c);
            }
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
        }
        lds_barrier();  // B2
        // the down weights enter the merge only after the barrier: the compiler would otherwise
        // move the merge (pure arithmetic) above it, and the wave would wait there for its data
#pragma unroll
        for (int i = 0; i < int(q6 ? kQ6Chunks : kQ4Chunks); ++i) asm volatile("" : "+v"(c[i]));
        if constexpr (q6) asm volatile("" : "+v"(dbits));
        if constexpr (q6) q6_merge_block(c, m6);  // the six-bit values, while h is being completed
        lds_barrier();  // B3
        {
            // ---- this wave's down part over h's column part kq ----
            const uint32_t lane = opaque_lane();
            const uint64_t *hp = htag + size_t(b) * kQK + 4 * lane;
            // The first read of h's tagged words and the next layer's gate DMA in one block,
            // which waits for the h loads only: the DMA streams while this layer's down dot
            // products run.  The compiler does not see the DMA instructions; had it issued them,
            // its first LDS access after them (the h values stored below) would wait for all of
            // them, as it cannot tell that they write other LDS.  Vector memory operations
            // complete in order, so operations the compiler does not count only make its own
            // later waits stricter; the gate slot is read after an explicit wait for everything.
            // After the last layer the same block runs with a buffer range of 0: the DMA reads are
            // out of range, which reads no memory and writes zeros to the slot.
            u32x4 h0, h1;
            {
                const bool next = l + 1 < L;
                const uint64_t gb = reinterpret_cast<uint64_t>(layers.wg[next ? l + 1 : l]);
                // buffer resource: base address, stride 0, the range in bytes, the format word
                const u32x4 rs{uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(gb))),
                               uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(gb >> 32) & 0xFFFFu)),
                               uint32_t(__builtin_amdgcn_readfirstlane(next ? F * nbg * kQ4Bytes : 0u)), 0x00020000u};
                const uint32_t so = __builtin_amdgcn_readfirstlane(uint32_t(region_offset(Q4_K, g, wave, nbg)));
                const uint32_t lds = __builtin_amdgcn_readfirstlane(
                    uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) u32x4 *)&lds_gate[wave][0][0])));
                const uint32_t vo = lane * 16;
                uint32_t st;
#define NS_GATE_DMA "s_nop 0\n\tbuffer_load_dwordx4 %[vo], %[rs], %[st] offen lds\n\t"
#define NS_GATE_NEXT "s_add_u32 m0, m0, 0x400\n\ts_add_u32 %[st], %[st], 0x400\n\t"
                asm volatile("global_load_dwordx4 %[h0], %[ha], off sc1\n\t"
                             "global_load_dwordx4 %[h1], %[ha], off offset:16 sc1\n\t"
                             "s_mov_b32 m0, %[lds]\n\t"
                             "s_mov_b32 %[st], %[so]\n\t" NS_GATE_DMA NS_GATE_NEXT NS_GATE_DMA NS_GATE_NEXT NS_GATE_DMA
                                 NS_GATE_NEXT NS_GATE_DMA NS_GATE_NEXT NS_GATE_DMA NS_GATE_NEXT NS_GATE_DMA NS_GATE_NEXT
                                     NS_GATE_DMA NS_GATE_NEXT NS_GATE_DMA NS_GATE_NEXT NS_GATE_DMA
                             "s_waitcnt vmcnt(9)"
                             : [h0] "=&v"(h0), [h1] "=&v"(h1), [st] "=&s"(st)
                             : [ha] "v"(hp), [rs] "s"(rs), [so] "s"(so), [lds] "s"(lds), [vo] "v"(vo)
                             : "memory", "m0", "scc");
#undef NS_GATE_DMA
#undef NS_GATE_NEXT
            }
            // lanes go through by-value arguments: clang's __builtin_bit_cast applied to a lane of
            // an ext-vector reads lane 0 whatever the lane
            const auto word = [](uint32_t lo, uint32_t hi) { return uint64_t(lo) | (uint64_t(hi) << 32); };
            uint64_t hr[4] = {word(h0.x, h0.y), word(h0.z, h0.w), word(h1.x, h1.y), word(h1.z, h1.w)};
            settle(hp, hr, t);
            const float4 hv{tagged_value(hr[0]), tagged_value(hr[1]), tagged_value(hr[2]), tagged_value(hr[3])};
            uint32_t lane_b = lane;
            asm volatile("" : "+v"(lane_b));
            reinterpret_cast<float4 *>(xw)[lane_b] = hv;
            float acc;
            if constexpr (q6) {
                float xs[16];
                group_sums_of<16>(hv, xs);
                acc = q6_dot_merged(m6, c[12], dbits, xw, xs);
            } else {
                const u32x4(&cc)[1][kQ4Chunks] = reinterpret_cast<const u32x4(&)[1][kQ4Chunks]>(c);
                float xs[8], r[1];
                group_sums_of<32>(hv, xs);
                q4_dot<1>(cc, xw, xs, r);
                acc = r[0];
            }
            lds_part[wave][0][lane_b] = acc;
        }
        lds_barrier();  // B4
    };
    dma_gate(0);
    for (uint32_t l = 0; l < L; ++l) {
        if ((layers.q6_down >> l) & 1u) layer(l, DTag<Q6_K>{});
        else layer(l, DTag<Q4_K>{});
    }
}
}  // namespace

void gemv_workspace_need(int type, int layout, uint32_t cols, uint32_t rows, bool pair, const Tuning &t,
                         size_t *partial_floats, size_t *counters) {
    const GemvPlan p = choose_gemv_for(type, layout, pair, cols, rows, t).plan;
    *partial_floats = size_t(p.G) * 2 * 64 * (pair ? 2 : 1);
    *counters = p.nslabs;
}

hipError_t launch_gemv(int type, int layout, const uint8_t *w, const uint8_t *up, const float *x,
                       float *out, uint32_t cols, uint32_t rows, const Workspace &ws, hipStream_t stream,
                       const NormPrologue *np) {
    if (up) return launch_typed<Q4_K, true>(layout, w, up, x, out, cols, rows, ws, stream, np);
    if (np) return hipErrorInvalidValue;  // the prologue exists for the gate/up pair only
    if (type == Q4_K) return launch_typed<Q4_K, false>(layout, w, nullptr, x, out, cols, rows, ws, stream, nullptr);
    return launch_typed<Q6_K, false>(layout, w, nullptr, x, out, cols, rows, ws, stream, nullptr);
}

void gemv_mt_workspace_need(int type, int layout, uint32_t cols, uint32_t rows, bool pair, uint32_t batch, bool xh,
                            const Tuning &t, size_t *partial_floats, size_t *counters) {
    if (gemv_mfma_eligible(layout, pair, xh, batch, t)) return gemv_mfma_workspace_need(cols, rows, pair, t, partial_floats, counters);
    const uint32_t nt = mt_tokens(batch, xh);
    const GemvPlan p = dispatch_mt(type, layout, pair, nt, xh, [&](auto m) { return decltype(m)::plan(cols, rows, t); });
    *partial_floats = size_t(p.G) * 2 * 64 * (pair ? 2 : 1) * nt;
    *counters = p.nslabs;
}

hipError_t launch_gemv_mt(int type, int layout, const uint8_t *w, const uint8_t *up, const void *x, bool xh,
                          uint32_t batch, void *out, uint32_t cols, uint32_t rows, const Workspace &ws,
                          hipStream_t stream) {
    const bool pair = up != nullptr;
    if (gemv_mfma_eligible(layout, pair, xh, batch, ws.tune))
        return launch_gemv_mfma(type, w, up, x, xh, batch, out, cols, rows, ws, stream);
    return dispatch_mt(type, layout, pair, mt_tokens(batch, xh), xh, [&](auto m) {
        using M = decltype(m);
        const GemvPlan p = M::plan(cols, rows, ws.tune);
        M::kernel()<<<dim3(p.G), dim3(p.W * 64), 0, stream>>>(w, up, x, batch, out, rows, cols / kQK, p.nslabs,
                                                               ws.partial, ws.counters);
        return hipGetLastError();
    });
}


template <int DTYPE, bool NORM>
constexpr auto block_kernel_of() {
    return &block_decode_kernel<DTYPE, NORM>;
}

// Workgroups of nbg waves of one instance that a CU holds at once, per device.
template <int DTYPE, bool NORM>
int block_wgs_per_cu(uint32_t nbg) {
    static int cache[64][kBlockMaxW + 1] = {};
    int dev = 0;
    (void)hipGetDevice(&dev);
    int &w = cache[dev & 63][nbg];
    if (w == 0) {
        int wgs = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&wgs, block_kernel_of<DTYPE, NORM>(), int(nbg) * 64, 0) !=
                hipSuccess || wgs <= 0)
            wgs = -1;  // unknown: never taken as room
        w = wgs;
    }
    return w;
}

bool block_decode_supported(int layout, int down_type, bool norm, uint32_t cols, uint32_t ffn) {
    const uint32_t nbg = cols / kQK, nbd = ffn / kQK;
    if (!(layout == CDNA4 && cols % kQK == 0 && ffn % kQK == 0 && nbg >= 1 && nbg <= kBlockMaxW && nbd % nbg == 0))
        return false;
    // the whole grid (ffn/64 workgroups) must fit on the device at once
    const int per_cu = down_type == Q4_K ? (norm ? block_wgs_per_cu<Q4_K, true>(nbg) : block_wgs_per_cu<Q4_K, false>(nbg))
                                         : (norm ? block_wgs_per_cu<Q6_K, true>(nbg) : block_wgs_per_cu<Q6_K, false>(nbg));
    return per_cu > 0 && uint64_t(ffn / kRowTile) <= uint64_t(per_cu) * uint64_t(device_shape().cus);
}

void block_decode_workspace_need(uint32_t cols, uint32_t ffn, size_t *partial_floats, size_t *counters) {
    (void)cols;
    (void)ffn;
    *partial_floats = 0;     // the column parts are tagged words in the context's buffers
    *counters = kCtrStride;  // slabs_done, status
}

hipError_t launch_block_decode(int down_type, const uint8_t *wg, const uint8_t *wu, const uint8_t *wd, const float *x,
                               const float *normw, float eps, float *h, float *y, uint32_t cols, uint32_t ffn,
                               const Workspace &ws, const StackBuffers &sb, hipStream_t stream) {
    if (!block_decode_supported(CDNA4, down_type, normw != nullptr, cols, ffn)) return hipErrorInvalidValue;
    size_t pf = 0, nc = 0;
    block_decode_workspace_need(cols, ffn, &pf, &nc);
    if (ws.counter_count < nc || !sb.epoch || sb.ffn < ffn) return hipErrorInvalidValue;
    // 2^22 polls, each an L2 round trip plus s_sleep 1: seconds
    const uint32_t spin = ws.tune.block_spin > 0 ? uint32_t(ws.tune.block_spin) : 1u << 22;
    const dim3 g(ffn / kRowTile), blk((cols / kQK) * 64);
    const auto args = [&](auto kernel) {
        kernel<<<g, blk, 0, stream>>>(wg, wu, wd, x, normw, eps, h, y, cols, ffn, ws.counters, spin, ws.err, sb.epoch,
                                      sb.htag, sb.ptag);
    };
    if (down_type == Q4_K) {
        if (normw) args(block_kernel_of<Q4_K, true>());
        else args(block_kernel_of<Q4_K, false>());
    } else {
        if (normw) args(block_kernel_of<Q6_K, true>());
        else args(block_kernel_of<Q6_K, false>());
    }
    return hipGetLastError();
}

// ---- the multi-layer decode launch --------------------------------------------------------

// Workgroups of W compute waves + 1 control wave that a CU holds at once, per device.
template <bool NORM>
int stack_wgs_per_cu(uint32_t nbg) {
    static int cache[64][kBlockMaxW + 1] = {};
    int dev = 0;
    (void)hipGetDevice(&dev);
    int &w = cache[dev & 63][nbg];
    if (w == 0) {
        int wgs = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&wgs, &stack_decode_kernel<NORM>, int(nbg + 1) * 64, 0) !=
                hipSuccess || wgs <= 0)
            wgs = -1;  // unknown: never taken as room
        w = wgs;
    }
    return w;
}

bool stack_decode_supported(int layout, bool norm, uint32_t cols, uint32_t ffn) {
    const uint32_t nbg = cols / kQK, nbd = ffn / kQK;
    if (!(layout == CDNA4 && cols % kQK == 0 && ffn % kQK == 0 && nbg >= 1 && nbg < kBlockMaxW && nbd % nbg == 0))
        return false;
    // the whole grid (ffn/64 workgroups) must fit on the device at once
    const int per_cu = norm ? stack_wgs_per_cu<true>(nbg) : stack_wgs_per_cu<false>(nbg);
    return per_cu > 0 && uint64_t(ffn / kRowTile) <= uint64_t(per_cu) * uint64_t(device_shape().cus);
}

void stack_decode_workspace_need(uint32_t cols, uint32_t ffn, size_t *partial_floats, size_t *counters) {
    (void)cols;
    (void)ffn;
    *partial_floats = 0;     // the column parts are tagged words in the context's buffers
    *counters = kCtrStride;  // status, exits
}

hipError_t launch_stack_decode(uint32_t n_layers, const uint8_t *const *wg, const uint8_t *const *wu,
                               const uint8_t *const *wd, const int *down_types, const float *x,
                               const float *const *normw, float eps, float *h, float *y, uint32_t cols, uint32_t ffn,
                               const Workspace &ws, const StackBuffers &sb, hipStream_t stream) {
    const bool norm = normw != nullptr;
    if (n_layers == 0 || !stack_decode_supported(CDNA4, norm, cols, ffn)) return hipErrorInvalidValue;
    size_t pf = 0, nc = 0;
    stack_decode_workspace_need(cols, ffn, &pf, &nc);
    if (ws.counter_count < nc || !sb.epoch || sb.cols < cols || sb.ffn < ffn) return hipErrorInvalidValue;
    // 2^22 polls, each an L2 round trip plus s_sleep 1: seconds
    const uint32_t spin = ws.tune.block_spin > 0 ? uint32_t(ws.tune.block_spin) : 1u << 22;
    const dim3 g(ffn / kRowTile), blk((cols / kQK + 1) * 64);
    // chunks of at most kStackMaxLayers layers (the table is a kernel argument); each chunk
    // continues from the previous one's y in place
    for (uint32_t l0 = 0; l0 < n_layers; l0 += kStackMaxLayers) {
        const uint32_t L = n_layers - l0 < kStackMaxLayers ? n_layers - l0 : kStackMaxLayers;
        StackLayers t{};
        for (uint32_t l = 0; l < L; ++l) {
            t.wg[l] = wg[l0 + l];
            t.wu[l] = wu[l0 + l];
            t.wd[l] = wd[l0 + l];
            t.normw[l] = norm ? normw[l0 + l] : nullptr;
            if (down_types[l0 + l] == Q6_K) t.q6_down |= uint64_t(1) << l;
        }
        const float *xin = l0 == 0 ? x : y;
        const auto run = [&](auto kernel) {
            kernel<<<g, blk, 0, stream>>>(t, L, xin, eps, h, y, cols, ffn, ws.counters, sb.epoch, sb.htag, sb.ytag,
                                          sb.ptag, spin, ws.err);
        };
        if (norm) run(&stack_decode_kernel<true>);
        else run(&stack_decode_kernel<false>);
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace ns
