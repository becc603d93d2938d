// ns_gemv.hip -- decode (batch 1) dequant-fused GEMV for gfx950.
//
// Replaces gemma_q4k_mv_fast[_metal], gemma_q6k_mv_fast[_metal] and
// gemma_q4k_gate_up_geglu_mv2[_metal] (metal/gemma4.metal:55-124, selected by
// matmul batch==1 at metal_engine.mm:272 and gate_up_geglu_decode at mm:290).
//
// Work decomposition (wave64, lane = weight row):
//   * one workgroup owns a 64-row slab (the .nsmffn row tile) and a contiguous
//     run of that slab's super-blocks; each of its waves takes a sub-run;
//   * every lane streams its own row's blocks: in the CDNA4 layout each of the
//     9 (Q4_K) or 13 (Q6_K) 16-byte chunk loads of a wave is one contiguous
//     1 KiB transaction; the next block is prefetched while one is computed;
//   * x is wave-uniform (every lane needs the same 256 values of a block) and
//     is read with scalar loads; per-group sums of x are built across lanes;
//   * partial sums meet in LDS (fixed wave order); when a slab's super-blocks
//     are split over several workgroups, each writes its partial to the
//     context workspace and the last one to arrive sums them in chunk order,
//     so results are deterministic.
//
// Per super-block the Q4_K dot is factorised as in the reference's
// q4k_mv_block_fast (metal:73):  sum_k w_k x_k = d * sum_g sc_g (sum_l q x)
//   - dmin * sum_g m_g (sum_l x).  The 4-bit q are widened without a convert:
// masking a dword with 0x000F000F leaves two fp16 subnormals q*2^-24 (and
// 0x00F000F0 gives q*2^-20 for the high nibble), which the fp32 FMA reads
// exactly; the 2^24 / 2^20 factors are folded into the group scale.
#include "ns_internal.hpp"
#include "ns_quant.hpp"

namespace ns {
namespace {

constexpr int kMaxWaves = 8;

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

// Q6_K (quant.cpp:13-18): element (half h, quarter q, l) uses scale 8h + l/16 + 2q;
// sum (v-32) x = sum v x - 32 sum x over each 16-wide scale group.
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
                const Q6Quarters q = q6_quarters(comp(c[4 * h + t], u), comp(c[4 * h + 2 + t], u),
                                                 comp(c[8 + 2 * h + t], u));
                const int l = 16 * t + 4 * u;
                const float *x0 = xb + 128 * h + l;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    A[8 * h + t + 0] = __builtin_fmaf(float(byte_of(q.v0, i)), x0[i], A[8 * h + t + 0]);
                    A[8 * h + t + 2] = __builtin_fmaf(float(byte_of(q.v1, i)), x0[32 + i], A[8 * h + t + 2]);
                    A[8 * h + t + 4] = __builtin_fmaf(float(byte_of(q.v2, i)), x0[64 + i], A[8 * h + t + 4]);
                    A[8 * h + t + 6] = __builtin_fmaf(float(byte_of(q.v3, i)), x0[96 + i], A[8 * h + t + 6]);
                }
            }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float sc = float(int8_t(byte_of(comp(c[12], i >> 2), i & 3)));
        s = __builtin_fmaf(sc, __builtin_fmaf(-32.0f, xs[i], A[i]), s);
    }
    return d * s;
}

// Sums of x over the block's groups of 32 (Q4_K, 8 values) or 16 (Q6_K, 16
// values), returned wave-uniform.  Each lane adds 4 values; the groups are
// completed with cross-lane exchanges and read back with readlane.
template <int GROUP>
__device__ __forceinline__ void group_sums(const float *__restrict__ xb, uint32_t lane, float *xs) {
    const float4 v = reinterpret_cast<const float4 *>(xb)[lane];
    float s = (v.x + v.y) + (v.z + v.w);
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    if constexpr (GROUP == 32) s += __shfl_xor(s, 4);
#pragma unroll
    for (int g = 0; g < 256 / GROUP; ++g)
        xs[g] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s), g * (GROUP / 4)));
}

template <int TYPE, int LAYOUT, bool PAIR>
__global__ __launch_bounds__(kMaxWaves * 64) void gemv_kernel(
    const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, const float *__restrict__ x,
    float *__restrict__ out, uint32_t rows, uint32_t nb, uint32_t kchunks, uint32_t nranges,
    float *__restrict__ partial, uint32_t *__restrict__ counters) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nwaves = blockDim.x >> 6;
    const uint32_t slab = blockIdx.x / kchunks, kc = blockIdx.x - slab * kchunks;
    const uint32_t row = slab * kRowTile + lane;
    const bool valid = row < rows;
    const uint32_t ri = kc * nwaves + wave;
    const uint32_t b0 = ri * nb / nranges, b1 = (ri + 1) * nb / nranges;

    float acc0 = 0.f, acc1 = 0.f;
    if constexpr (TYPE == Q4_K) {
        constexpr int N = PAIR ? 2 : 1;
        const uint8_t *wm[2] = {w0, w1};
        u32x4 c[N][kQ4Chunks];
        if (valid && b0 < b1)
#pragma unroll
            for (int n = 0; n < N; ++n) q4_load<LAYOUT>(wm[n], lane, row, slab, b0, nb, c[n]);
        for (uint32_t b = b0; b < b1; ++b) {
            u32x4 nx[N][kQ4Chunks];
            if (valid && b + 1 < b1)
#pragma unroll
                for (int n = 0; n < N; ++n) q4_load<LAYOUT>(wm[n], lane, row, slab, b + 1, nb, nx[n]);
            const float *xb = x + size_t(b) * kQK;
            float xs[8], r[N];
            group_sums<32>(xb, lane, xs);
            q4_dot<N>(c, xb, xs, r);
            acc0 += r[0];
            if constexpr (PAIR) acc1 += r[N - 1];
#pragma unroll
            for (int n = 0; n < N; ++n)
#pragma unroll
                for (int i = 0; i < int(kQ4Chunks); ++i) c[n][i] = nx[n][i];
        }
    } else {
        u32x4 c0[kQ6Chunks];
        uint32_t d0 = 0;
        if (valid && b0 < b1) q6_load<LAYOUT>(w0, lane, row, slab, b0, nb, c0, d0);
        for (uint32_t b = b0; b < b1; ++b) {
            u32x4 n0[kQ6Chunks];
            uint32_t dn = 0;
            if (valid && b + 1 < b1) q6_load<LAYOUT>(w0, lane, row, slab, b + 1, nb, n0, dn);
            const float *xb = x + size_t(b) * kQK;
            float xs[16];
            group_sums<16>(xb, lane, xs);
            acc0 += q6_dot(c0, d0, xb, xs);
#pragma unroll
            for (int i = 0; i < int(kQ6Chunks); ++i) c0[i] = n0[i];
            d0 = dn;
        }
    }

    __shared__ float red[PAIR ? 2 : 1][kMaxWaves][64];
    red[0][wave][lane] = acc0;
    if constexpr (PAIR) red[PAIR ? 1 : 0][wave][lane] = acc1;
    __syncthreads();
    if (wave != 0) return;
    float s0 = 0.f, s1 = 0.f;
    for (uint32_t w = 0; w < nwaves; ++w) {
        s0 += red[0][w][lane];
        if constexpr (PAIR) s1 += red[PAIR ? 1 : 0][w][lane];
    }
    if (kchunks > 1) {
        // Hand-off between workgroups through device-coherent (agent-scope)
        // atomic stores and loads only: the partials bypass the XCD-private L2,
        // so no L2-wide write-back/invalidate fence is needed.  The wait below
        // makes every partial store complete before the arrival is counted;
        // the last arrival reads them after its counter atomic has returned.
        if (valid) {
            __hip_atomic_store(&partial[size_t(kc) * rows + row], s0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if constexpr (PAIR)
                __hip_atomic_store(&partial[size_t(kchunks + kc) * rows + row], s1, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        uint32_t prev = 0;
        if (lane == 0)
            prev = __hip_atomic_fetch_add(&counters[slab], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        prev = __shfl(prev, 0);
        if (prev != kchunks - 1) return;
        s0 = 0.f;
        s1 = 0.f;
        if (valid)
            for (uint32_t k = 0; k < kchunks; ++k) {
                s0 += __hip_atomic_load(&partial[size_t(k) * rows + row], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if constexpr (PAIR)
                    s1 += __hip_atomic_load(&partial[size_t(kchunks + k) * rows + row], __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
            }
        if (lane == 0) __hip_atomic_store(&counters[slab], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!valid) return;
    if constexpr (PAIR) out[row] = gelu_tanh(s0) * s1;
    else out[row] = s0;
}

struct GemvPlan {
    uint32_t nslabs, nwaves, kchunks;
};

int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

// Splits each slab's nb super-blocks into nwaves*kchunks runs, aiming at
// ~4096 waves in flight (16 per CU on 256 CUs) with runs of >= 1 block.
GemvPlan plan_gemv(uint32_t cols, uint32_t rows) {
    GemvPlan p;
    const uint32_t nb = cols / kQK;
    p.nslabs = (rows + kRowTile - 1) / kRowTile;
    uint32_t want = (4096 + p.nslabs - 1) / p.nslabs;
    want = want < 1 ? 1 : (want > nb ? nb : want);
    p.kchunks = (want + kMaxWaves - 1) / kMaxWaves;
    p.nwaves = (want + p.kchunks - 1) / p.kchunks;
    while (p.nwaves * p.kchunks > nb && p.nwaves > 1) --p.nwaves;
    const int ew = env_int("NS_GEMV_WAVES", 0), ek = env_int("NS_GEMV_KCHUNKS", 0);
    if (ew > 0 && ew <= kMaxWaves) p.nwaves = uint32_t(ew);
    if (ek > 0) p.kchunks = uint32_t(ek);
    while (p.nwaves * p.kchunks > nb) {
        if (p.kchunks > 1) --p.kchunks;
        else --p.nwaves;
    }
    return p;
}

template <int TYPE, bool PAIR>
hipError_t launch_typed(int layout, const uint8_t *w, const uint8_t *up, const float *x, float *out,
                        uint32_t cols, uint32_t rows, const Workspace &ws, hipStream_t stream) {
    const GemvPlan p = plan_gemv(cols, rows);
    const uint32_t nb = cols / kQK;
    const dim3 grid(p.nslabs * p.kchunks), block(p.nwaves * 64);
    const uint32_t nr = p.nwaves * p.kchunks;
    if (layout == CDNA4)
        gemv_kernel<TYPE, CDNA4, PAIR><<<grid, block, 0, stream>>>(w, up, x, out, rows, nb, p.kchunks, nr, ws.partial, ws.counters);
    else if (layout == NSMFFN)
        gemv_kernel<TYPE, NSMFFN, PAIR><<<grid, block, 0, stream>>>(w, up, x, out, rows, nb, p.kchunks, nr, ws.partial, ws.counters);
    else
        gemv_kernel<TYPE, ROW_MAJOR, PAIR><<<grid, block, 0, stream>>>(w, up, x, out, rows, nb, p.kchunks, nr, ws.partial, ws.counters);
    return hipGetLastError();
}

}  // namespace

void gemv_workspace_need(uint32_t cols, uint32_t rows, bool pair, size_t *partial_floats, size_t *counters) {
    const GemvPlan p = plan_gemv(cols, rows);
    *partial_floats = p.kchunks > 1 ? size_t(p.kchunks) * rows * (pair ? 2 : 1) : 0;
    *counters = p.kchunks > 1 ? p.nslabs : 0;
}

hipError_t launch_gemv(int type, int layout, const uint8_t *w, const uint8_t *up, const float *x,
                       float *out, uint32_t cols, uint32_t rows, const Workspace &ws, hipStream_t stream) {
    if (up) return launch_typed<Q4_K, true>(layout, w, up, x, out, cols, rows, ws, stream);
    if (type == Q4_K) return launch_typed<Q4_K, false>(layout, w, nullptr, x, out, cols, rows, ws, stream);
    return launch_typed<Q6_K, false>(layout, w, nullptr, x, out, cols, rows, ws, stream);
}

}  // namespace ns
