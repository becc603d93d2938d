// ns_gemv_mfma.hip -- batch 1-4 (the MTP-verification regime of metal:102-177, mm:273, mm:282)
// on the matrix cores, for the CDNA4 layout.
//
// The small-batch VALU kernel (gemv_mt_kernel) repeats one FMA per weight per token, which
// makes it VALU-bound at four tokens.  Here the tokens are the rows of an MFMA tile and the
// weights its columns: the weight side is unpacked once into fp16 B fragments that are exact
// integers, and the matrix core does the per-token products.
//
//   v_mfma_f32_16x16x32_f16: A[i][k] (token rows) and B[k][n] (16 weight rows) hold 8 halves
//   per lane, lane = row + 16 * (k / 8); the 16x16 result D[i][n] sits in lane n + 16*(i/4),
//   slot i % 4 (the 16x16x16 form, measured on MI355X, has the same result layout).
//
// Exact fp16 fragments (every product and every fp16 value below is exact):
//   Q6_K  B = v - 32 (|B| <= 32): one MFMA covers two 16-element scale groups, group a in
//         k 0-15 and group b in k 16-31.  The A rows of group a are zero in k 16-31 and those of
//         group b zero in k 0-15, so D's rows separate the groups, and each lane scales its
//         group's D by d*sc (exact in fp32) into the fp32 accumulator.
//   Q4_K  B = sc*q (<= 945): sc folds into the fragment, so the eight 32-element groups of a
//         super-block accumulate in one MFMA chain S, and the min term M = sum_g m_g * xs_g
//         (xs = the group sums of x) is one 16x16x16 MFMA.  acc += d*S - dmin*M.
// fp32 tokens are split into fp16 hi + lo rows (22 significant bits; the product error is
// ~2^-22 relative) after an exact per-token power-of-two scale that keeps |x| < 2^15; fp16
// tokens enter as they are.  x of a workgroup's column range is staged once in LDS.
//
// Work split: a wave takes one 64-row slab (four 16-row MFMA tiles) of one matrix over a
// contiguous run of super-blocks.  A workgroup holds S slabs x M matrices (the gate/up pair:
// M = 2) x P column parts and stages x for its column part KP; parts meet in LDS in wave
// order, and column parts of different workgroups (KP > 1) by the deterministic hand-off of
// the decode GEMV: agent-scope atomic stores of the parts, an arrival counter per slab, and
// the last workgroup to arrive adds the KP parts in order.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "ns_common.hpp"
#include "ns_internal.hpp"
#include "ns_quant.hpp"

namespace ns {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

constexpr int NT = 4;                  // token rows (batch <= 4)
constexpr int kMaxSb = 15;             // super-blocks of x one workgroup stages (3840 columns)
constexpr int kMaxNk = kMaxSb * 256;
constexpr int kStripe = kMaxNk + 8;    // halves per LDS stripe: +16 B so stripes start on different banks
constexpr int kMaxWaves = 8;
constexpr int kStage = 16;             // x quads per thread in the staging round

__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, int(bytes), 0x00020000);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, int(voff), int(soff), 0);
}
__device__ __forceinline__ u32x2 bload8(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, int(voff), int(soff), 0);
}
__device__ __forceinline__ uint32_t bload2(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, int(voff), int(soff), 0);
}

// Lane exchanges inside a row of 16 lanes by DPP (no LDS round trip): dpp_ctrl 0xB1 and 0x4E
// are quad_perm [1,0,3,2] and [2,3,0,1] (lane ^ 1, lane ^ 2), 0x141 row_half_mirror (lane i of
// an 8-lane half takes lane 7 - i), 0x140 row_mirror (lane i of the row takes lane 15 - i).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Sum over 8 consecutive lanes, in every lane of them: a + a^1, then + (^2), then the other
// quad's sum (the values a butterfly with lane ^ 4 would add, in the same order).
__device__ __forceinline__ float sum8(float s) {
    s += dpp<0xB1>(s);
    s += dpp<0x4E>(s);
    return s + dpp<0x141>(s);
}
// Largest value of the wave (every lane's value >= 0), wave-uniform.
__device__ __forceinline__ float wave_max(float m) {
    m = __builtin_fmaxf(m, dpp<0xB1>(m));
    m = __builtin_fmaxf(m, dpp<0x4E>(m));
    m = __builtin_fmaxf(m, dpp<0x141>(m));
    m = __builtin_fmaxf(m, dpp<0x140>(m));
    const auto rl = [&](int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m), l)); };
    return __builtin_fmaxf(__builtin_fmaxf(rl(0), rl(16)), __builtin_fmaxf(rl(32), rl(48)));
}

// Four bytes (values < 1024) -> four exact fp16 values byte - bias, in element order.
// (0x6400 | b) is the fp16 1024 + b; one packed add removes 1024 + bias.
__device__ __forceinline__ void bytes_to_f16(uint32_t v, half2_t bias, uint32_t &lo, uint32_t &hi) {
    const uint32_t e01 = __builtin_amdgcn_perm(0x64646464u, v, 0x04010400u);  // [b0, 0x64, b1, 0x64]
    const uint32_t e23 = __builtin_amdgcn_perm(0x64646464u, v, 0x04030402u);  // [b2, 0x64, b3, 0x64]
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, e01) + bias);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, e23) + bias);
}

// Q6_K: the 6-bit values of quarter j (0..3) for four consecutive l, one per byte, from the
// ql dword (low nibbles for j < 2, high for j >= 2) and the qh dword (bits 2j..2j+1).
__device__ __forceinline__ uint32_t q6_merge(uint32_t ql, uint32_t qh, int j) {
    const uint32_t lo = (j >= 2 ? ql >> 4 : ql) & 0x0F0F0F0Fu;
    const uint32_t hb = j == 0 ? (qh << 4) : j == 1 ? (qh << 2) : j == 2 ? qh : (qh >> 2);
    return lo | (hb & 0x30303030u);
}

// Q4_K: one qs dword = elements e..e+3 of groups 2j (low nibbles) and 2j+1 (high nibbles).
// Returns sc_lo*q (low) and sc_hi*q (high) as exact fp16, element order: (0x6400 | q) is
// 1024 + q, and fma(1024 + q, sc, -1024*sc) = sc*q exactly.
// mask (an SGPR) and c (a VGPR) come in as opaque registers so that (v & mask) | c is one
// v_and_or_b32: with both as literals the compiler emits an AND and an OR (a VOP3 instruction
// takes no literal on this architecture).
__device__ __forceinline__ void q4_scaled(uint32_t w, half2_t slo, half2_t mlo, half2_t shi, half2_t mhi,
                                          uint32_t mask, uint32_t c, uint32_t (&lo)[2], uint32_t (&hi)[2]) {
    const uint32_t p = __builtin_amdgcn_perm(w, w, 0x03010200u);  // bytes [b0, b2, b1, b3]
    auto f = [](uint32_t q, half2_t s, half2_t m) {
        return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(half2_t, q), s, m));
    };
    lo[0] = f((p & mask) | c, slo, mlo);
    lo[1] = f(((p >> 8) & mask) | c, slo, mlo);
    hi[0] = f(((p >> 4) & mask) | c, shi, mhi);
    hi[1] = f(((p >> 12) & mask) | c, shi, mhi);
}

struct Q6Raw {
    u32x2 ql[4][4];  // [tile][2h + (j&1)]: 8 bytes of the ql chunk
    u32x2 qh[4][2];  // [tile][h]
    u32x4 sc[4];     // the row's 16 scales
    uint32_t d[4];   // the row's d (low half)
};
struct Q4Raw {
    u32x2 qs[4][4];  // [tile][j]
    u32x4 hdr[4];    // d, dmin, scales[12]
};

template <int TYPE>
using RawOf = typename std::conditional<TYPE == Q6_K, Q6Raw, Q4Raw>::type;

struct Plan {
    uint32_t S, M, P, KP;
};

template <int TYPE, bool PAIR, bool XH>
__global__ __launch_bounds__(kMaxWaves * 64) void gemv_mfma_kernel(
    const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, const void *__restrict__ x, uint32_t batch,
    void *__restrict__ out, uint32_t rows, uint32_t nb, Plan pl, float *__restrict__ partial,
    uint32_t *__restrict__ counters) {
    constexpr bool Q6 = TYPE == Q6_K;
    constexpr uint32_t BB = Q6 ? kQ6Bytes : kQ4Bytes;
    constexpr int kPlanes = XH ? 1 : 2;            // hi (+ lo) stripes per token
    constexpr int kZero = kPlanes * NT;            // the zero stripe
    constexpr int M = PAIR ? 2 : 1;
    __shared__ __attribute__((aligned(16))) _Float16 xl[(kZero + 1) * kStripe];
    __shared__ __attribute__((aligned(16))) _Float16 xsl[kMaxSb][2][NT][8];  // Q4_K group sums (hi, lo)
    __shared__ float wmax[kMaxWaves][NT];
    __shared__ float xsc[kMaxSb][NT];  // Q4_K, fp16 x: 2^(e+5) of each super-block's group sums

    const uint32_t tid = threadIdx.x, lane = tid & 63, nw = blockDim.x >> 6;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t slabs = rows / kRowTile, cols = nb * kQK;
    const uint32_t g = blockIdx.x, kp = g % pl.KP, sg = g / pl.KP;
    const uint32_t sb_lo = kp * nb / pl.KP, sb_hi = (kp + 1) * nb / pl.KP, nsb = sb_hi - sb_lo;
    const uint32_t nk = nsb * kQK, k0 = sb_lo * kQK;
    // this wave: slab, matrix and column part
    const uint32_t ws = wave / (M * pl.P), wm = (wave / pl.P) % M, wp = wave % pl.P;
    const uint32_t slab = sg * pl.S + ws;
    const bool active = slab < slabs;
    const uint32_t wsb0 = sb_lo + wp * nsb / pl.P, wsb1 = sb_lo + (wp + 1) * nsb / pl.P;

    const uint32_t wbytes = rows * nb * BB;
    const rsrc_t wsrc = make_rsrc(PAIR && wm == 1 ? w1 : w0, wbytes);
    const uint32_t n = lane & 15, o = lane >> 4;
    // lane part of the weight offsets: 8 bytes at chunk (o >> 1) of row n, half (o & 1)
    const uint32_t vq = ((o >> 1) * kRowTile + n) * 16 + 8 * (o & 1);
    const uint32_t vrow = n * 16;  // 16-byte piece of row n in a chunk
    auto region = [&](uint32_t sb) {
        const uint32_t s = __builtin_elementwise_min(slab, slabs - 1);
        return uint32_t(region_offset(TYPE, s, sb, nb));
    };
    auto load = [&](uint32_t sb, RawOf<TYPE> &r) {
        const uint32_t base = __builtin_amdgcn_readfirstlane(region(sb));
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t tb = base + 256 * t;  // rows 16t.. of the slab
            if constexpr (Q6) {
#pragma unroll
                for (int c = 0; c < 4; ++c) r.ql[t][c] = bload8(wsrc, vq, tb + (2 * c) * 1024);
#pragma unroll
                for (int h = 0; h < 2; ++h) r.qh[t][h] = bload8(wsrc, vq, tb + (8 + 2 * h) * 1024);
                r.sc[t] = bload16(wsrc, vrow, tb + 12 * 1024);
                r.d[t] = bload2(wsrc, 2 * n, base + 13 * 1024 + 2 * 16 * t);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) r.qs[t][j] = bload8(wsrc, vq, tb + (1 + 2 * j) * 1024);
                r.hdr[t] = bload16(wsrc, vrow, tb);
            }
        }
    };

    // ---- prologue: the first super-block's weights in flight, then x staged in LDS -------
    RawOf<TYPE> ra, rb;

    // Per-token powers of two, from the largest |x| of the workgroup's columns (2^E <= max < 2^(E+1)):
    //  - fp32 tokens enter the MFMA as x * 2^-e, e = E - 14, so the largest is in [2^14, 2^15): the
    //    fp16 hi part cannot overflow, and tiny tokens keep their bits out of fp16's subnormals;
    //  - the Q4_K group sums enter as xs * 2^-(e+5) (|xs| <= 32 * max|x|); for fp16 tokens e comes
    //    from the super-block's own largest |x| (the min term of each super-block is scaled
    //    back on its own).
    // Both are exact; the results are scaled back by the inverse powers.
    float oscale[NT], minfac[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) oscale[t] = minfac[t] = 1.f;
    // e + 128 of every token, one byte each: a lane picks its token's with one bit-field
    // extract (selecting from a register array by a lane-varying index would put the array in
    // scratch, and the scratch load's wait would also wait for the weights in flight)
    uint32_t epack = 128u * 0x01010101u;
    auto p2 = [](int k) { return __builtin_bit_cast(float, uint32_t(127 + k) << 23); };
    auto e_of = [&](uint32_t t) { return int(__builtin_amdgcn_ubfe(epack, 8 * (t & 3), 8)) - 128; };
    const uint32_t nq = nk / 4;  // 4-column quads per token
    // One round of loads: quad i = r * blockDim + tid (token i / nq) for r < kStage; the plan
    // gives every workgroup enough threads (64 * waves * kStage >= NT * nq).  All loads are in
    // flight before the first use.
    // The loads are unconditional (token and quad clamped into the tensor, then masked), and x's
    // are issued before the first super-block's weights: x comes from L2 and the staging below
    // then waits for x only, while the weights are still in flight.
    float4_t xv[kStage];
    {
        using XT = typename std::conditional<XH, half4_t, float4_t>::type;
        XT raw[kStage];
#pragma unroll
        for (int r = 0; r < kStage; ++r) {
            const uint32_t i = r * blockDim.x + tid, t = i / nq;
            const uint32_t tc = __builtin_elementwise_min(t, batch - 1), qc = t < batch ? i - t * nq : 0u;
            raw[r] = *reinterpret_cast<const XT *>(static_cast<const uint8_t *>(x) +
                                                   (size_t(tc) * cols + k0 + 4 * qc) * (XH ? 2 : 4));
        }
        // unconditional (a wave past the last slab re-reads the last one): a branch around
        // the loads would make the staging wait for them at the merge
        load(__builtin_elementwise_min(wsb0, nb - 1), ra);
        __builtin_amdgcn_sched_barrier(0);  // the weights stay ahead of the staging work
#pragma unroll
        for (int r = 0; r < kStage; ++r) {
            const uint32_t t = (r * blockDim.x + tid) / nq;
            float4_t v;
            if constexpr (XH) v = float4_t{float(raw[r].x), float(raw[r].y), float(raw[r].z), float(raw[r].w)};
            else v = raw[r];
            xv[r] = t < batch ? v : float4_t{0.f, 0.f, 0.f, 0.f};
        }
    }
    // fp32 tokens: one power of two per token for the workgroup's columns (the A rows carry it
    // into every super-block).  fp16 tokens only scale the Q4_K group sums, per super-block, in
    // the store loop below: no workgroup-wide maximum, no barrier.
    if constexpr (!XH) {
        float mx[NT] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < kStage; ++r) {
            const uint32_t t = (r * blockDim.x + tid) / nq;
            const float4_t v = xv[r];
            const float m = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
                                            __builtin_fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w)));
#pragma unroll
            for (int u = 0; u < NT; ++u)
                if (uint32_t(u) == t) mx[u] = __builtin_fmaxf(mx[u], m);
        }
#pragma unroll
        for (int u = 0; u < NT; ++u) {
            mx[u] = wave_max(mx[u]);
            if (lane == 0) wmax[wave][u] = mx[u];
        }
        // a bare barrier: __syncthreads() would also wait for the first super-block's weights
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        epack = 0;
#pragma unroll
        for (int u = 0; u < NT; ++u) {
            float m = 0.f;
            for (uint32_t v = 0; v < nw; ++v) m = __builtin_fmaxf(m, wmax[v][u]);
            const int E = int((__builtin_bit_cast(uint32_t, m) >> 23) & 0xFF) - 127;  // floor(log2 m), normal m
            const int e = m >= 1.17549435e-38f && E < 128 ? __builtin_elementwise_max(E - 14, -100) : 0;
            oscale[u] = p2(e);
            minfac[u] = 32.f;
            epack |= uint32_t(e + 128) << (8 * u);
        }
    }
#pragma unroll
    for (int r = 0; r < kStage; ++r) {
        // every thread stores (quads past the last token into the unread tail of the zero
        // stripe): a store under a condition would let the compiler sink x's load under it
        const uint32_t i = r * blockDim.x + tid, t = i / nq, q = i - t * nq;
        const uint32_t dst_hi = t < NT ? t * kStripe + 4 * q : kZero * kStripe + kMaxNk;
        const uint32_t dst_lo = t < NT ? (NT + t) * kStripe + 4 * q : kZero * kStripe + kMaxNk + 4;
        uint32_t hi01, hi23, lo01 = 0, lo23 = 0;
        if constexpr (XH) {
            const float4_t v = xv[r];  // fp16 values, exact in fp32
            hi01 = __builtin_bit_cast(uint32_t, half2_t{_Float16(v.x), _Float16(v.y)});
            hi23 = __builtin_bit_cast(uint32_t, half2_t{_Float16(v.z), _Float16(v.w)});
        } else {
            const float4_t v = xv[r] * p2(-e_of(t));
            const half2_t h01{_Float16(v.x), _Float16(v.y)}, h23{_Float16(v.z), _Float16(v.w)};
            const half2_t l01{_Float16(v.x - float(h01.x)), _Float16(v.y - float(h01.y))};
            const half2_t l23{_Float16(v.z - float(h23.x)), _Float16(v.w - float(h23.y))};
            hi01 = __builtin_bit_cast(uint32_t, h01);
            hi23 = __builtin_bit_cast(uint32_t, h23);
            lo01 = __builtin_bit_cast(uint32_t, l01);
            lo23 = __builtin_bit_cast(uint32_t, l23);
        }
        *reinterpret_cast<u32x2 *>(&xl[dst_hi]) = u32x2{hi01, hi23};
        if constexpr (!XH) *reinterpret_cast<u32x2 *>(&xl[dst_lo]) = u32x2{lo01, lo23};
        if constexpr (!Q6) {
            // group sum of 32 columns = 8 quads held by 8 consecutive lanes (nq and blockDim are
            // multiples of 8): a fixed butterfly, times 2^-(e+5), split into fp16 hi + lo
            float s = (xv[r].x + xv[r].y) + (xv[r].z + xv[r].w);
            s = sum8(s);
            int eg = e_of(t);
            if constexpr (XH) {
                // the wave's 64 quads are one super-block of one token (nq is a multiple of 64):
                // its largest |x| sets the group sums' power of two
                const float4_t v = xv[r];
                const float m = wave_max(__builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
                                                         __builtin_fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w))));
                const int E = int((__builtin_bit_cast(uint32_t, m) >> 23) & 0xFF) - 127;
                eg = m >= 1.17549435e-38f && E < 128 ? __builtin_elementwise_max(E - 14, -100) : 0;
                if (lane == 0 && t < NT) xsc[q >> 6][t] = p2(eg + 5);
            }
            s *= p2(-(eg + 5));
            if ((q & 7) == 0 && t < NT) {
                const uint32_t gi = q >> 3;
                const _Float16 h = _Float16(s);
                xsl[gi >> 3][0][t][gi & 7] = h;
                xsl[gi >> 3][1][t][gi & 7] = _Float16(s - float(h));
            }
        }
    }
    for (uint32_t i = tid; i < nq; i += blockDim.x) *reinterpret_cast<u32x2 *>(&xl[kZero * kStripe + 4 * i]) = u32x2{0u, 0u};
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);

    // ---- A operands: this lane's LDS stripe (or the zero stripe) -------------------------------
    //   Q6_K fp32 x: row i = 8*group + 4*plane + token;  Q6_K fp16 x: row i = 4*group + token;
    //   Q4_K fp32 x: row i = 4*plane + token;  Q4_K fp16 x: row i = token.
    uint32_t stripe = kZero;
    {
        const uint32_t i = n;
        uint32_t t = i & 3, plane = 0, grp = 0;
        bool valid;
        if constexpr (Q6 && !XH) {
            grp = i >> 3;
            plane = (i >> 2) & 1;
            valid = (o >> 1) == grp;
        } else if constexpr (Q6) {
            grp = i >> 2;
            valid = i < 8 && (o >> 1) == grp;
        } else if constexpr (!XH) {
            plane = i >> 2;
            valid = i < 8;
        } else {
            valid = i < 4;
        }
        if (valid && t < batch) stripe = plane * NT + t;
    }
    const _Float16 *abase = &xl[stripe * kStripe + 8 * o];
    // Q4_K min term A: row i = token, k = 4*o + slot: groups 4*(o&1).. of plane o >> 1
    const bool xs_valid = n < 4 && n < batch;
    // Q6_K: the scale group of this lane's D rows (a: 0, b: 1)
    const uint32_t glane8 = 8 * (XH ? ((lane >> 4) & 1) : (lane >> 5));

    float4_t acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
    const half2_t bias6{_Float16(-1056.0f), _Float16(-1056.0f)}, bias4{_Float16(-1024.0f), _Float16(-1024.0f)};

    uint32_t nib_mask, f16_1024;
    asm volatile("s_mov_b32 %0, 0x000F000F" : "=s"(nib_mask));
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(f16_1024));
    auto compute = [&](const RawOf<TYPE> &r, uint32_t sb) {
        const _Float16 *ab = abase + (sb - sb_lo) * kQK;
        if constexpr (Q6) {
            float dv[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) dv[t] = lo_half(r.d[t]);
#pragma unroll
            for (int p = 0; p < 8; ++p) {
                const half8_t a = *reinterpret_cast<const half8_t *>(ab + 32 * p);
                const int h = p >> 2, j = p & 3;
                // the four tiles' fragments, then their MFMAs, then the scaling: a result is read
                // four MFMAs after it was issued, not right behind it
                float4_t dd[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const u32x2 ql = r.ql[t][2 * h + (j & 1)], qh = r.qh[t][h];
                    uint32_t b[4];
                    bytes_to_f16(q6_merge(ql.x, qh.x, j), bias6, b[0], b[1]);
                    bytes_to_f16(q6_merge(ql.y, qh.y, j), bias6, b[2], b[3]);
                    dd[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        a, __builtin_bit_cast(half8_t, u32x4{b[0], b[1], b[2], b[3]}), float4_t{0.f, 0.f, 0.f, 0.f},
                        0, 0, 0);
                }
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int sc = __builtin_amdgcn_sbfe(r.sc[t][p >> 1], 16 * (p & 1) + glane8, 8);
                    const float ds = dv[t] * float(sc);
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_fmaf(ds, dd[t][v], acc[t][v]);
                }
            }
        } else {
            Q4Scales s4[4];
            float4_t S[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                s4[t] = q4_scales(r.hdr[t].y, r.hdr[t].z, r.hdr[t].w);
                S[t] = float4_t{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const half8_t alo = *reinterpret_cast<const half8_t *>(ab + 64 * j);
                const half8_t ahi = *reinterpret_cast<const half8_t *>(ab + 64 * j + 32);
                u32x4 blo[4], bhi[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const _Float16 sl = _Float16(float(q4_sc(s4[t], 2 * j))), sh = _Float16(float(q4_sc(s4[t], 2 * j + 1)));
                    const half2_t slo{sl, sl}, shi{sh, sh};
                    const half2_t mlo = slo * half2_t{_Float16(-1024.0f), _Float16(-1024.0f)};
                    const half2_t mhi = shi * half2_t{_Float16(-1024.0f), _Float16(-1024.0f)};
                    uint32_t l0[2], h0[2], l1[2], h1[2];
                    q4_scaled(r.qs[t][j].x, slo, mlo, shi, mhi, nib_mask, f16_1024, l0, h0);
                    q4_scaled(r.qs[t][j].y, slo, mlo, shi, mhi, nib_mask, f16_1024, l1, h1);
                    blo[t] = u32x4{l0[0], l0[1], l1[0], l1[1]};
                    bhi[t] = u32x4{h0[0], h0[1], h1[0], h1[1]};
                }
                // the chain of each tile's S takes its two MFMAs four MFMAs apart
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    S[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, __builtin_bit_cast(half8_t, blo[t]), S[t], 0, 0, 0);
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    S[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, __builtin_bit_cast(half8_t, bhi[t]), S[t], 0, 0, 0);
            }
            const uint32_t si = sb - sb_lo;
            float mf[NT];
#pragma unroll
            for (int v = 0; v < NT; ++v) mf[v] = XH ? xsc[si][v] : minfac[v];
            u32x2 am = *reinterpret_cast<const u32x2 *>(&xsl[si][o >> 1][n & 3][4 * (o & 1)]);
            if (!xs_valid) am = u32x2{0u, 0u};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t mw = (o & 1) ? s4[t].m47 : s4[t].m03;
                uint32_t m0, m1;
                bytes_to_f16(mw, bias4, m0, m1);
                const float4_t mn = __builtin_amdgcn_mfma_f32_16x16x16f16(
                    __builtin_bit_cast(half4_t, am), __builtin_bit_cast(half4_t, u32x2{m0, m1}),
                    float4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                const float d = lo_half(r.hdr[t].x), dmin = hi_half(r.hdr[t].x);
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    acc[t][v] = __builtin_fmaf(d, S[t][v], __builtin_fmaf(-dmin * mf[v], mn[v], acc[t][v]));
            }
        }
    };

    // ---- main loop: compute one super-block while the next one's weights load ---------------
    // Two buffers alternate.  The first iteration is peeled: its prefetch is unconditional
    // (clamped into the tensor; a wave with one super-block drops it) and pinned by a signal
    // fence, so it leaves right after the staging barrier.  Entering the loop with the
    // prologue's buffer instead made the compiler copy that buffer into the loop's registers,
    // which waited for its loads before the first prefetch could issue.  Inside the loop the end
    // test comes before each prefetch, so every prefetch is consumed on every path: a load that a
    // path leaves unused is sunk by the compiler past the compute into the path that uses it,
    // which serialises load and compute.  The scheduling barrier keeps the prefetch ahead of the
    // compute.  Every wave runs it (one past the last slab on the clamped last slab, its results
    // dropped), and every wave has at least one super-block (the plan keeps P <= nsb).
    {
        uint32_t sb = wsb0;
        const bool more = sb + 1 != wsb1;
        load(__builtin_elementwise_min(sb + 1, nb - 1), rb);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_sched_barrier(0);
        compute(ra, sb);
        ++sb;
        while (more) {
            if (sb + 1 == wsb1) {
                compute(rb, sb);
                break;
            }
            load(sb + 1, ra);
            __builtin_amdgcn_sched_barrier(0);
            compute(rb, sb);
            ++sb;
            if (sb + 1 == wsb1) {
                compute(ra, sb);
                break;
            }
            load(sb + 1, rb);
            __builtin_amdgcn_sched_barrier(0);
            compute(ra, sb);
            ++sb;
        }
    }

    // ---- combine: the four D quarters (planes, groups) of each row, then the token scale -------
    float tot[4][4];  // [tile][token] for row 16*tile + n
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            float s = acc[t][v];
            s += __shfl_xor(s, 16);
            s += __shfl_xor(s, 32);
            tot[t][v] = s * oscale[v];
        }
    // lane l takes row l of the slab (tile l >> 4)
    float mine[NT];
#pragma unroll
    for (int v = 0; v < NT; ++v) {
        const uint32_t t = lane >> 4;
        mine[v] = t == 0 ? tot[0][v] : t == 1 ? tot[1][v] : t == 2 ? tot[2][v] : tot[3][v];
    }
    const uint32_t row = slab * kRowTile + lane;
    auto store_out = [&](const float (&gv)[NT], const float (&uv)[NT]) {
#pragma unroll
        for (int v = 0; v < NT; ++v) {
            if (uint32_t(v) >= batch) break;
            if constexpr (PAIR)
                static_cast<_Float16 *>(out)[size_t(v) * rows + row] = _Float16(gelu_tanh(gv[v]) * uv[v]);
            else
                static_cast<float *>(out)[size_t(v) * rows + row] = gv[v];
        }
    };
    if (pl.P == 1 && M == 1 && pl.KP == 1) {
        if (active) store_out(mine, mine);
        return;
    }

    // parts of this workgroup meet in LDS (the x stripes are free once every wave is past its loop)
    float *part = reinterpret_cast<float *>(xl);  // [wave][token][64]
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
    for (int v = 0; v < NT; ++v) part[(wave * NT + v) * 64 + lane] = mine[v];
    __syncthreads();
    if (!active || wm != 0 || wp != 0) return;
    float r[M][NT];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int v = 0; v < NT; ++v) {
            float s = 0.f;
            for (uint32_t q = 0; q < pl.P; ++q) s += part[(((ws * M + m) * pl.P + q) * NT + v) * 64 + lane];
            r[m][v] = s;
        }
    if (pl.KP > 1) {
        // hand-off between the workgroups of one slab's column parts
        float *dst = partial + (size_t(slab) * pl.KP + kp) * (M * NT * 64);
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int v = 0; v < NT; ++v)
                __hip_atomic_store(&dst[(m * NT + v) * 64 + lane], r[m][v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        uint32_t prev = 0;
        if (lane == 0) prev = __hip_atomic_fetch_add(&counters[slab], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        prev = __builtin_amdgcn_readfirstlane(__shfl(prev, 0));
        if (prev != pl.KP - 1) return;
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int v = 0; v < NT; ++v) r[m][v] = 0.f;
        const float *src = partial + size_t(slab) * pl.KP * (M * NT * 64);
        for (uint32_t q = 0; q < pl.KP; ++q)
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
                for (int v = 0; v < NT; ++v)
                    r[m][v] += __hip_atomic_load(&src[(q * M + m) * NT * 64 + v * 64 + lane], __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0) __hip_atomic_store(&counters[slab], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    store_out(r[0], r[M - 1]);
}

template <int TYPE, bool PAIR, bool XH>
constexpr auto mfma_kernel() {
    return &gemv_mfma_kernel<TYPE, PAIR, XH>;
}

// Plan: workgroups of four waves, so that two fill a CU (the kernel's ~250 VGPRs allow two waves
// per SIMD): four slabs per workgroup when the slabs alone give >= 1,024 waves (the lm-head),
// else four column parts of one slab (two per matrix for the gate/up pair).  MI355X, batch 4:
// the 60-block Q6_K down takes 17.7 us at 4 or 8 parts per slab, 20-23 us at 1, 3 or 5 (six and
// five waves leave a CU with one workgroup); the gate/up pair 24.5 us at 2 parts per matrix,
// ~30 us at 3.  More workgroups per slab (fewer super-blocks per wave) measured slower in every
// case (down 19-32 us, gate/up 34-67 us): each workgroup stages x and hands its part off.  A
// workgroup stages at most 15 super-blocks of x, in one round of kStage quads per thread.
Plan plan_mfma(uint32_t rows, uint32_t nb, bool pair, const Tuning &t) {
    Plan p{1, pair ? 2u : 1u, 1, (nb + kMaxSb - 1) / kMaxSb};
    const uint32_t slabs = rows / kRowTile;
    const uint32_t nsb = (nb + p.KP - 1) / p.KP;
    const uint32_t base = slabs * p.M * p.KP;
    const uint32_t pmax = __builtin_elementwise_min(uint32_t(kMaxWaves) / p.M, nsb);
    if (t.mt_parts > 0) p.P = __builtin_elementwise_min(uint32_t(t.mt_parts), pmax);
    else if (base < 1024) p.P = __builtin_elementwise_min(4 / p.M, pmax);
    if (t.mt_spw > 0) {  // super-blocks per wave: more workgroups per slab
        p.KP = __builtin_elementwise_max(p.KP, (nb + p.P * t.mt_spw - 1) / (p.P * t.mt_spw));
        p.P = __builtin_elementwise_max(1u, __builtin_elementwise_min(p.P, nb / p.KP));
    }
    if (p.P == 1 && p.KP == 1) {
        p.S = uint32_t(kMaxWaves / 2) / p.M;  // 4 waves per workgroup
        if (t.mt_slabs > 0) p.S = __builtin_elementwise_min(uint32_t(t.mt_slabs), uint32_t(kMaxWaves) / p.M);
    }
    // the staging round: 64 * waves * kStage quads >= 4 tokens * nsb * 64 quads
    const uint32_t nsb_wg = (nb + p.KP - 1) / p.KP;
    const uint32_t need = (nsb_wg * kQK + 64 * kStage - 1) / (64 * kStage);
    if (p.S * p.M * p.P < need) {
        if (p.P == 1 && p.KP == 1) p.S = (need + p.M - 1) / p.M;
        else p.P = __builtin_elementwise_min((need + p.M - 1) / p.M, pmax);
    }
    return p;
}

template <class Fn>
auto dispatch_mfma(int type, bool pair, bool xh, Fn &&fn) {
    if (pair) return fn(mfma_kernel<Q4_K, true, true>());
    if (type == Q4_K) return xh ? fn(mfma_kernel<Q4_K, false, true>()) : fn(mfma_kernel<Q4_K, false, false>());
    return xh ? fn(mfma_kernel<Q6_K, false, true>()) : fn(mfma_kernel<Q6_K, false, false>());
}

}  // namespace

// The gate/up pair (fp16 x) from two tokens on: at two tokens 22.7-22.9 us here against
// 25.1-25.2 us for the VALU kernel (same-box A/B, MI355X); every other shape is faster here too.
bool gemv_mfma_eligible(int layout, bool pair, bool xh, uint32_t batch, const Tuning &t) {
    return layout == CDNA4 && t.mt_mfma != 0 && (!pair || (xh && batch >= 2));
}

void gemv_mfma_workspace_need(uint32_t cols, uint32_t rows, bool pair, const Tuning &t, size_t *partial_floats,
                              size_t *counters) {
    const Plan p = plan_mfma(rows, cols / kQK, pair, t);
    const size_t slabs = rows / kRowTile;
    *partial_floats = p.KP > 1 ? slabs * p.KP * p.M * NT * 64 : 0;
    *counters = p.KP > 1 ? slabs : 0;
}

hipError_t launch_gemv_mfma(int type, const uint8_t *w, const uint8_t *up, const void *x, bool xh, uint32_t batch,
                            void *out, uint32_t cols, uint32_t rows, const Workspace &ws, hipStream_t stream) {
    const bool pair = up != nullptr;
    const uint32_t nb = cols / kQK;
    if (batch == 0 || batch > uint32_t(NT) || rows % kRowTile || cols % kQK || nb == 0) return hipErrorInvalidValue;
    const Plan p = plan_mfma(rows, nb, pair, ws.tune);
    const uint32_t slabs = rows / kRowTile;
    const uint32_t nsb = (nb + p.KP - 1) / p.KP, nwv = p.S * p.M * p.P;
    if (nwv > uint32_t(kMaxWaves) || nsb > uint32_t(kMaxSb) || nwv * 64 * kStage < nsb * kQK || p.P > nb / p.KP)
        return hipErrorInvalidValue;
    if (p.KP > 1 && (ws.partial_floats < size_t(slabs) * p.KP * p.M * NT * 64 || ws.counter_count < slabs))
        return hipErrorInvalidValue;
    const uint32_t nwg = (slabs + p.S - 1) / p.S * p.KP;
    return dispatch_mfma(type, pair, xh, [&](auto k) {
        k<<<dim3(nwg), dim3(p.S * p.M * p.P * 64), 0, stream>>>(w, up, x, batch, out, rows, nb, p, ws.partial,
                                                                 ws.counters);
        return hipGetLastError();
    });
}

}  // namespace ns
