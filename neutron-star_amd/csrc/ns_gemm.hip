// ns_gemm.hip -- prefill (batch > 1) quantised GEMM on fp16 MFMA for gfx950.
//
// Replaces, on the .nsmffn path, the reference's
//   gemma_q4k_gate_up_geglu_metal_rm32_f16 / _f16acc_f16 (metal/gemma4.metal:373-383,
//     gate_up_geglu_rm32 at metal_engine.mm:288)                        -> PAIR = true
//   gemma_q6k_mma_metal_f16[_f16acc_f16], gemma_q4k_mma_metal_f16[_f16acc_f16]
//     (metal:385-395, :480-490; ffn_down / matmul at mm:289, mm:271)    -> PAIR = false
//
// Integer-exact tiles.  Inside one 256-wide super-block every weight is
//   Q4_K: w = d * (sc_g * q) - dmin * m_g      (quant.cpp:11)
//   Q6_K: w = d * (sc_s * (v - 32))            (quant.cpp:17)
// where sc*q (<= 945) and sc*(v-32) (|.| <= 1024) are integers that fp16
// represents exactly.  The LDS weight tile therefore holds those integers, the
// MFMA products with fp16 x are exact, and the per-row factors are applied once
// per super-block on the accumulators:
//   Y += d * acc_sb  [- dmin * sum_g m_g * S_g(x)]            (S_g = sum of x over group g)
// The Q4_K min term is one extra MFMA per super-block whose K runs over the 8
// groups: A = the group sums of x split into fp16 hi + lo (k 0..7 and 8..15),
// B = m_g.  This keeps the FP32 mode at fp32 accuracy (a plain fp16 copy of the
// dequantised weights would add ~1e-3 relative error by itself) and needs fewer
// VALU operations per weight than materialising d*sc*q - dmin*m.
//
// Tiling: one workgroup (256 threads = 4 wave64) computes 128 tokens x 128
// columns with v_mfma_f32_32x32x16_f16; columns are 128 weight rows (plain) or
// 64 rows of gate followed by the same 64 rows of up (PAIR); each wave owns a
// 64 x 64 quadrant (2 x 2 MFMA tiles).  For PAIR a quadrant is 32 rows of gate
// plus the same 32 rows of up, so gate and up of one output meet in one lane
// and GeGLU runs on registers.  Per 64-wide k step, x is copied to LDS and two
// threads per column decode the step's weights into the LDS tile.  LDS rows are
// padded to 72 halfs so the ds_read_b128 operand fetches are conflict-free.
// The token tiles of a 1024-token batch map onto the 8 XCDs (workgroup i runs
// on XCD i % 8), so each XCD's L2 keeps its own 128 x K slice of x.
//
// Accumulation modes (metal_engine.mm:565):
//   FP32  Y accumulates in fp32.
//   FP16  Y is rounded to fp16 precision (11 significant bits, fp32 exponent
//         range) after every super-block update, so outputs carry fp16
//         precision (metal:394/:489 widen half tiles).  True fp16 range would
//         overflow on BASELINE's synthetic inputs (down outputs reach 1.7e5).
#include "ns_internal.hpp"
#include "ns_quant.hpp"

namespace ns {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int TT = 128;        // tokens per workgroup tile
constexpr int TC = 128;        // B columns per workgroup tile
constexpr int KS = 64;         // k per step
constexpr int LDSW = KS + 8;   // padded LDS row (halfs)
constexpr int kThreads = 256;

// FP16-mode rounding: nearest even at 11 significant bits (the fp16
// significand), fp32 exponent range.  Identical to fp16 rounding on the fp16
// normal range; values beyond 65504 keep their magnitude instead of becoming inf.
__device__ __forceinline__ float round_f16p(float v) {
    uint32_t b = __builtin_bit_cast(uint32_t, v);
    b = (b + 0x0fffu + ((b >> 13) & 1u)) & 0xffffe000u;
    return __builtin_bit_cast(float, b);
}

__device__ __forceinline__ half2_t h2(uint32_t bits) { return __builtin_bit_cast(half2_t, bits); }
__device__ __forceinline__ uint32_t u32(half2_t v) { return __builtin_bit_cast(uint32_t, v); }

// Two small unsigned fields (selected bytes of w, masked) as fp16 1024+f
// (0x6400 | f): v_perm spreads bytes into the two 16-bit lanes.
__device__ __forceinline__ half2_t magic_pair(uint32_t w, uint32_t sel, uint32_t mask) {
    return h2((__builtin_amdgcn_perm(w, w, sel) & mask) | 0x64006400u);
}
constexpr uint32_t kSel01 = 0x0c010c00u;  // [0, b1, 0, b0]
constexpr uint32_t kSel23 = 0x0c030c02u;  // [0, b3, 0, b2]

// sc*(1024+f) + bias with one rounding; exact because the result is an integer <= 2048.
__device__ __forceinline__ uint32_t scale_pair(half2_t t, half2_t sc, half2_t bias) {
    return u32(__builtin_elementwise_fma(t, sc, bias));
}

struct WRun {
    u32x4 v[4];  // v[0..1]: 16 halfs at k offset k_lo, v[2..3]: 16 halfs at k_hi
    int k_lo, k_hi;
};

// Q4_K producer.  Step s covers groups 2p, 2p+1 (p = s%4) of super-block s/4:
// qs bytes 32p..32p+31, low nibble -> group 2p, high -> group 2p+1.  Thread
// half hh takes bytes 32p+16hh..+15: run 0 = group 2p, l = 16hh..+15 (k offset
// 16hh); run 1 = group 2p+1, same l (k offset 32+16hh).  Values: sc_g * q.
template <int LAYOUT>
__device__ __forceinline__ void q4_tile(const uint8_t *__restrict__ w, uint32_t row, uint32_t nb, uint32_t s,
                                        uint32_t hh, WRun &out, u32x4 &hdr) {
    const uint32_t b = s >> 2, p = s & 3;
    u32x4 qs;
    if constexpr (LAYOUT == CDNA4) {
        const u32x4 *base = reinterpret_cast<const u32x4 *>(w + region_offset(Q4_K, row / kRowTile, b, nb)) +
                            (row % kRowTile);
        hdr = base[0];
        qs = base[(1 + 2 * p + hh) * kRowTile];
    } else {
        const u32x4 *blk = reinterpret_cast<const u32x4 *>(w + block_index(NSMFFN, row, b, nb) * kQ4Bytes);
        hdr = blk[0];
        qs = blk[1 + 2 * p + hh];
    }
    const Q4Scales sc = q4_scales(hdr.y, hdr.z, hdr.w);
    const _Float16 s0 = _Float16(float(q4_sc(sc, int(2 * p)))), s1 = _Float16(float(q4_sc(sc, int(2 * p + 1))));
    const half2_t sc0 = {s0, s0}, sc1 = {s1, s1};
    const half2_t nb0 = {_Float16(-1024.f) * s0, _Float16(-1024.f) * s0};
    const half2_t nb1 = {_Float16(-1024.f) * s1, _Float16(-1024.f) * s1};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t wv = qs[i], wh = wv >> 4;
        out.v[i >> 1][(i & 1) * 2 + 0] = scale_pair(magic_pair(wv, kSel01, 0x000F000Fu), sc0, nb0);
        out.v[i >> 1][(i & 1) * 2 + 1] = scale_pair(magic_pair(wv, kSel23, 0x000F000Fu), sc0, nb0);
        out.v[2 + (i >> 1)][(i & 1) * 2 + 0] = scale_pair(magic_pair(wh, kSel01, 0x000F000Fu), sc1, nb1);
        out.v[2 + (i >> 1)][(i & 1) * 2 + 1] = scale_pair(magic_pair(wh, kSel23, 0x000F000Fu), sc1, nb1);
    }
    out.k_lo = 16 * int(hh);
    out.k_hi = 32 + 16 * int(hh);
}

__device__ __forceinline__ u32x4 load_chunk_q6(const uint8_t *__restrict__ blk, uint32_t chunk) {
    // NSMFFN Q6_K blocks are 2-byte aligned only
    const uint16_t *h = reinterpret_cast<const uint16_t *>(blk) + 8 * chunk;
    return u32x4{h[0] | (uint32_t(h[1]) << 16), h[2] | (uint32_t(h[3]) << 16), h[4] | (uint32_t(h[5]) << 16),
                 h[6] | (uint32_t(h[7]) << 16)};
}

// Q6_K producer.  Step s covers elements 64*(s%4)..+63 of super-block s/4:
// half h = (s%4)/2, quarters 2*(s%2) and 2*(s%2)+1.  Thread half hh takes
// quarter qa = 2*(s%2)+hh, l = 0..31 (k offsets 32hh..32hh+31):
//   v = nibble of ql[64h + 32*(qa&1) + l] (low if qa < 2) | (qh[32h + l] >> 2qa & 3) << 4.
// Values: sc * (v - 32), sc = scales[8h + 2qa + l/16].
template <int LAYOUT>
__device__ __forceinline__ void q6_tile(const uint8_t *__restrict__ w, uint32_t row, uint32_t nb, uint32_t s,
                                        uint32_t hh, WRun &out, uint32_t &dbits) {
    const uint32_t b = s >> 2, sr = s & 3, h = sr >> 1, qa = 2 * (sr & 1) + hh;
    u32x4 ql[2], qh[2], scw;
    const uint32_t cl = 4 * h + 2 * (qa & 1), chh = 8 + 2 * h;
    if constexpr (LAYOUT == CDNA4) {
        const uint8_t *reg = w + region_offset(Q6_K, row / kRowTile, b, nb);
        const u32x4 *base = reinterpret_cast<const u32x4 *>(reg) + (row % kRowTile);
        ql[0] = base[cl * kRowTile];
        ql[1] = base[(cl + 1) * kRowTile];
        qh[0] = base[chh * kRowTile];
        qh[1] = base[(chh + 1) * kRowTile];
        scw = base[12 * kRowTile];
        dbits = reinterpret_cast<const uint16_t *>(reg + kQ6Chunks * 1024)[row % kRowTile];
    } else {
        const uint8_t *blk = w + block_index(NSMFFN, row, b, nb) * kQ6Bytes;
        ql[0] = load_chunk_q6(blk, cl);
        ql[1] = load_chunk_q6(blk, cl + 1);
        qh[0] = load_chunk_q6(blk, chh);
        qh[1] = load_chunk_q6(blk, chh + 1);
        scw = load_chunk_q6(blk, 12);
        dbits = reinterpret_cast<const uint16_t *>(blk)[104];
    }
    const uint32_t si = 8 * h + 2 * qa;
    const uint32_t nshift = qa >= 2 ? 4 : 0, hshift = 2 * qa;
#pragma unroll
    for (int c = 0; c < 2; ++c) {  // l = 16c .. 16c+15
        const _Float16 s16 = _Float16(float(int8_t(byte_of(scw[(si + c) >> 2], int((si + c) & 3)))));
        const half2_t sc2 = {s16, s16};
        const half2_t nb2 = {_Float16(-1056.f) * s16, _Float16(-1056.f) * s16};
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // l = 16c + 4i .. +3
            const uint32_t v = ((ql[c][i] >> nshift) & 0x0F0F0F0Fu) | (((qh[c][i] >> hshift) & 0x03030303u) << 4);
            out.v[2 * c + (i >> 1)][(i & 1) * 2 + 0] = scale_pair(magic_pair(v, kSel01, 0x003F003Fu), sc2, nb2);
            out.v[2 * c + (i >> 1)][(i & 1) * 2 + 1] = scale_pair(magic_pair(v, kSel23, 0x003F003Fu), sc2, nb2);
        }
    }
    out.k_lo = 32 * int(hh);
    out.k_hi = 32 * int(hh) + 16;
}

template <int TYPE, int LAYOUT, int ACC, bool PAIR>
__global__ __launch_bounds__(kThreads, 2) void gemm_kernel(
    const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, const uint16_t *__restrict__ x,
    const uint16_t *__restrict__ xs_hi, const uint16_t *__restrict__ xs_lo, void *__restrict__ out,
    uint32_t cols, uint32_t rows, uint32_t batch, uint32_t ntok_tiles) {
    __shared__ __attribute__((aligned(16))) _Float16 Xs[TT * LDSW];
    __shared__ __attribute__((aligned(16))) _Float16 Ws[TC * LDSW];
    __shared__ float colD[TC];
    __shared__ float colDmin[TYPE == Q4_K ? TC : 1];
    __shared__ __attribute__((aligned(16))) _Float16 colM[TYPE == Q4_K ? TC * 8 : 8];

    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wt = wave >> 1, wn = wave & 1;
    // token tile fastest, so that token tile == XCD when ntok_tiles == 8
    const uint32_t tt = blockIdx.x % ntok_tiles, ct = blockIdx.x / ntok_tiles;
    const uint32_t t0 = tt * TT;
    constexpr uint32_t kRowsPerTile = PAIR ? TC / 2 : TC;
    const uint32_t r0 = ct * kRowsPerTile;
    const uint32_t nb = cols / kQK, nsteps = cols / KS, ngroups = cols / 32;

    // producer role: column wc of the tile, k half hh
    const uint32_t wc = tid >> 1, hh = tid & 1;
    const uint8_t *wsrc = (PAIR && wc >= TC / 2) ? w1 : w0;
    const uint32_t wrow = r0 + (PAIR ? (wc % (TC / 2)) : wc);
    const bool wvalid = wrow < rows;

    float16_t acc[2][2], tot[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = tot[i][j][v] = 0.f;

    auto bcol = [&](int j) -> uint32_t {
        if constexpr (PAIR) return uint32_t(j) * (TC / 2) + wn * 32;  // gate / up of the same 32 rows
        else return wn * 64 + uint32_t(j) * 32;
    };

    for (uint32_t s = 0; s < nsteps; ++s) {
        // ---- global -> registers
        u32x4 xr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t idx = tid + kThreads * i, tok = idx >> 3, part = idx & 7;
            const uint32_t t = t0 + tok;
            xr[i] = t < batch ? *reinterpret_cast<const u32x4 *>(x + size_t(t) * cols + s * KS + part * 8)
                              : u32x4{0u, 0u, 0u, 0u};
        }
        WRun wr;
        u32x4 hdr = {0u, 0u, 0u, 0u};
        uint32_t dbits = 0;
        if (wvalid) {
            if constexpr (TYPE == Q4_K) q4_tile<LAYOUT>(wsrc, wrow, nb, s, hh, wr, hdr);
            else q6_tile<LAYOUT>(wsrc, wrow, nb, s, hh, wr, dbits);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) wr.v[i] = u32x4{0u, 0u, 0u, 0u};
            wr.k_lo = TYPE == Q4_K ? 16 * int(hh) : 32 * int(hh);
            wr.k_hi = TYPE == Q4_K ? 32 + 16 * int(hh) : 32 * int(hh) + 16;
        }
        __syncthreads();  // the previous step's fragments and column factors are consumed
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t idx = tid + kThreads * i, tok = idx >> 3, part = idx & 7;
            *reinterpret_cast<u32x4 *>(&Xs[tok * LDSW + part * 8]) = xr[i];
        }
        {
            _Float16 *wl = &Ws[wc * LDSW];
            *reinterpret_cast<u32x4 *>(wl + wr.k_lo) = wr.v[0];
            *reinterpret_cast<u32x4 *>(wl + wr.k_lo + 8) = wr.v[1];
            *reinterpret_cast<u32x4 *>(wl + wr.k_hi) = wr.v[2];
            *reinterpret_cast<u32x4 *>(wl + wr.k_hi + 8) = wr.v[3];
        }
        if ((s & 3) == 0 && hh == 0) {  // per-column factors of this super-block
            if constexpr (TYPE == Q4_K) {
                colD[wc] = lo_half(hdr.x);
                colDmin[wc] = hi_half(hdr.x);
                const Q4Scales sc = q4_scales(hdr.y, hdr.z, hdr.w);
                u32x4 mv;
#pragma unroll
                for (int g = 0; g < 8; g += 2)
                    mv[g / 2] = uint32_t(__builtin_bit_cast(uint16_t, _Float16(float(q4_m(sc, g))))) |
                                (uint32_t(__builtin_bit_cast(uint16_t, _Float16(float(q4_m(sc, g + 1))))) << 16);
                *reinterpret_cast<u32x4 *>(&colM[wc * 8]) = mv;
            } else {
                colD[wc] = lo_half(dbits);
            }
        }
        __syncthreads();

        // ---- MFMA over the 4 k16 sub-steps
#pragma unroll
        for (int kk = 0; kk < KS / 16; ++kk) {
            const uint32_t koff = 16 * kk + 8 * (lane >> 5);
            half8_t a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i] = *reinterpret_cast<const half8_t *>(&Xs[(wt * 64 + i * 32 + (lane & 31)) * LDSW + koff]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[j] = *reinterpret_cast<const half8_t *>(&Ws[(bcol(j) + (lane & 31)) * LDSW + koff]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }

        if ((s & 3) == 3) {  // end of a super-block: apply the per-row factors
            const uint32_t sb = s >> 2;
            float dcol[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) dcol[j] = colD[bcol(j) + (lane & 31)];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        tot[i][j][v] = __builtin_fmaf(dcol[j], acc[i][j][v], tot[i][j][v]);
                        acc[i][j][v] = 0.f;
                    }
            if constexpr (TYPE == Q4_K) {
                // min term: A = group sums of x (hi in k 0..7, lo in k 8..15), B = m_g
                half8_t am[2], bm[2];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const uint32_t t = t0 + wt * 64 + i * 32 + (lane & 31);
                    const uint16_t *src = (lane < 32 ? xs_hi : xs_lo) + size_t(t) * ngroups + 8 * sb;
                    am[i] = t < batch ? *reinterpret_cast<const half8_t *>(src) : half8_t{};
                }
                float dmin[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const uint32_t c = bcol(j) + (lane & 31);
                    bm[j] = *reinterpret_cast<const half8_t *>(&colM[c * 8]);
                    dmin[j] = colDmin[c];
                }
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const float16_t mt = __builtin_amdgcn_mfma_f32_32x32x16_f16(am[i], bm[j], float16_t{}, 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 16; ++v) tot[i][j][v] = __builtin_fmaf(-dmin[j], mt[v], tot[i][j][v]);
                    }
            }
            if constexpr (ACC == ACC_FP16) {
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
#pragma unroll
                        for (int v = 0; v < 16; ++v) tot[i][j][v] = round_f16p(tot[i][j][v]);
            }
        }
    }

    // ---- epilogue.  32x32 D layout: lane holds column lane%32 and rows
    // 8*(v/4) + 4*(lane/32) + v%4 for v = 0..15.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const uint32_t t = t0 + wt * 64 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
            if (t >= batch) continue;
            if constexpr (PAIR) {
                const uint32_t r = r0 + wn * 32 + (lane & 31);
                const float g = tot[i][0][v], u = tot[i][1][v];
                reinterpret_cast<_Float16 *>(out)[size_t(t) * rows + r] = _Float16(gelu_tanh(g) * u);
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const uint32_t r = r0 + wn * 64 + j * 32 + (lane & 31);
                    if (r < rows) reinterpret_cast<float *>(out)[size_t(t) * rows + r] = tot[i][j][v];
                }
            }
        }
    }
}

// Group sums of x for the Q4_K min term: s = sum of 32 fp16 values in fp32,
// stored as hi = fp16(s) and lo = fp16(s - hi) (together ~22 significant bits).
__global__ void group_sums_kernel(const uint16_t *__restrict__ x, uint32_t cols, uint32_t batch,
                                  uint16_t *__restrict__ hi, uint16_t *__restrict__ lo) {
    const uint32_t ng = cols / 32;
    const uint64_t idx = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= uint64_t(batch) * ng) return;
    const uint32_t t = uint32_t(idx / ng), g = uint32_t(idx % ng);
    const half8_t *p = reinterpret_cast<const half8_t *>(x + size_t(t) * cols + size_t(g) * 32);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const half8_t v = p[i];
#pragma unroll
        for (int e = 0; e < 8; ++e) s += float(v[e]);
    }
    const _Float16 h = _Float16(s);
    hi[idx] = __builtin_bit_cast(uint16_t, h);
    lo[idx] = __builtin_bit_cast(uint16_t, _Float16(s - float(h)));
}

template <int TYPE, int LAYOUT, bool PAIR>
hipError_t launch_mode(int acc, const uint8_t *w, const uint8_t *up, const uint16_t *x, const uint16_t *xh,
                       const uint16_t *xl, void *out, uint32_t cols, uint32_t rows, uint32_t batch,
                       hipStream_t stream) {
    const uint32_t ntok = (batch + TT - 1) / TT;
    const uint32_t rows_per_tile = PAIR ? TC / 2 : TC;
    const uint32_t ncol = (rows + rows_per_tile - 1) / rows_per_tile;
    const dim3 grid(ntok * ncol), block(kThreads);
    if (acc == ACC_FP16)
        gemm_kernel<TYPE, LAYOUT, ACC_FP16, PAIR><<<grid, block, 0, stream>>>(w, up, x, xh, xl, out, cols, rows,
                                                                              batch, ntok);
    else
        gemm_kernel<TYPE, LAYOUT, ACC_FP32, PAIR><<<grid, block, 0, stream>>>(w, up, x, xh, xl, out, cols, rows,
                                                                              batch, ntok);
    return hipGetLastError();
}

template <int TYPE, bool PAIR>
hipError_t launch_layout(int layout, int acc, const uint8_t *w, const uint8_t *up, const uint16_t *x,
                         const uint16_t *xh, const uint16_t *xl, void *out, uint32_t cols, uint32_t rows,
                         uint32_t batch, hipStream_t stream) {
    if (layout == CDNA4) return launch_mode<TYPE, CDNA4, PAIR>(acc, w, up, x, xh, xl, out, cols, rows, batch, stream);
    return launch_mode<TYPE, NSMFFN, PAIR>(acc, w, up, x, xh, xl, out, cols, rows, batch, stream);
}

}  // namespace

size_t gemm_workspace_floats(int type, uint32_t cols, uint32_t batch) {
    // two fp16 planes of batch x cols/32 group sums, counted in floats
    return type == Q4_K ? (size_t(batch) * (cols / 32) + 1) : 0;
}

hipError_t launch_gemm(int type, int layout, int acc, const uint8_t *w, const uint8_t *up, const uint16_t *x,
                       void *out, uint32_t cols, uint32_t rows, uint32_t batch, const Workspace &ws,
                       hipStream_t stream) {
    uint16_t *xh = nullptr, *xl = nullptr;
    if (type == Q4_K) {
        const size_t n = size_t(batch) * (cols / 32);
        xh = reinterpret_cast<uint16_t *>(ws.partial);
        xl = xh + n;
        group_sums_kernel<<<dim3(uint32_t((n + 255) / 256)), dim3(256), 0, stream>>>(x, cols, batch, xh, xl);
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    }
    if (up) return launch_layout<Q4_K, true>(layout, acc, w, up, x, xh, xl, out, cols, rows, batch, stream);
    if (type == Q4_K) return launch_layout<Q4_K, false>(layout, acc, w, nullptr, x, xh, xl, out, cols, rows, batch, stream);
    return launch_layout<Q6_K, false>(layout, acc, w, nullptr, x, xh, xl, out, cols, rows, batch, stream);
}

}  // namespace ns
