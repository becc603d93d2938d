// ns_gemm.hip -- prefill (batch > 1) dequant-into-LDS fp16 MFMA GEMM for gfx950.
//
// Replaces, on the .nsmffn path, the reference's
//   gemma_q4k_gate_up_geglu_metal_rm32_f16 / _f16acc_f16 (metal/gemma4.metal:373-383,
//     gate_up_geglu_rm32 at metal_engine.mm:288) -> PAIR = true
//   gemma_q6k_mma_metal_f16[_f16acc_f16], gemma_q4k_mma_metal_f16[_f16acc_f16]
//     (metal:385-395, :480-490; ffn_down / matmul at mm:289, mm:271)  -> PAIR = false
//
// One workgroup (256 threads = 4 wave64) computes a 128-token x 128-column tile
// of Y = X . W^T with v_mfma_f32_32x32x16_f16.  Columns are 128 weight rows
// (plain) or 64 rows of gate followed by the same 64 rows of up (PAIR); each
// wave owns a 64-token x 64-column quadrant, i.e. 2 x 2 MFMA tiles.  For PAIR
// the quadrant is 32 rows of gate plus the same 32 rows of up, so gate and up
// of one output land in the same lane and GeGLU runs on registers.
//
// Per 64-wide k step: fp16 X is copied to LDS, and the quantised weights are
// loaded (16-byte chunks, coalesced in the CDNA4 layout) and dequantised by
// two threads per column straight into an fp16 LDS tile (RNE of the exact fp32
// value, so the tile is bit-identical to ns_dequant's fp16 output).  LDS rows
// are padded to 72 halfs so the ds_read_b128 operand fetches are conflict-free.
//
// Accumulation modes (metal_engine.mm:565):
//   FP32  fp32 MFMA accumulation through the whole K.
//   FP16  the accumulators are rounded to fp16 at every super-block (256)
//         boundary and the output is fp16 (widened to fp32 for the down
//         projection, as metal:394 / :489 do).
//
// The 8 token tiles of a 1024-token batch map to the 8 XCDs (workgroup i runs
// on XCD i % 8), so each XCD's L2 keeps its own 128 x K slice of X.
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

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    return uint32_t(__builtin_bit_cast(uint16_t, _Float16(a))) |
           (uint32_t(__builtin_bit_cast(uint16_t, _Float16(b))) << 16);
}

__device__ __forceinline__ float round_f16(float v) { return float(_Float16(v)); }

// ---- weight tile producers ----------------------------------------------
// Each thread produces 32 fp16 values of one column for k step `s`; they are
// returned as 4 x u32x4 = two 16-value runs: run 0 at k offset k_lo, run 1 at k_hi.

struct WRun {
    u32x4 v[4];   // v[0..1]: run 0 (16 halfs), v[2..3]: run 1
    int k_lo, k_hi;
};

// Q4_K: k step s covers groups 2p, 2p+1 (p = s%4) of super-block s/4, i.e.
// qs bytes 32p..32p+31 (low nibbles -> group 2p, high -> group 2p+1).  Thread
// half hh takes bytes 32p+16hh..+15: run 0 = group 2p, l = 16hh..16hh+15 (k
// offset 16hh), run 1 = group 2p+1, same l (k offset 32+16hh).
template <int LAYOUT>
__device__ __forceinline__ void q4_tile(const uint8_t *__restrict__ w, uint32_t row, uint32_t nb, uint32_t s,
                                        uint32_t hh, WRun &out) {
    const uint32_t b = s >> 2, p = s & 3;
    u32x4 hdr, qs;
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
    const float d = lo_half(hdr.x), dmin = hi_half(hdr.x);
    const Q4Scales sc = q4_scales(hdr.y, hdr.z, hdr.w);
    const uint32_t g0 = 2 * p, g1 = 2 * p + 1;
    const float D0 = d * float(q4_sc(sc, int(g0))), M0 = dmin * float(q4_m(sc, int(g0)));
    const float D1 = d * float(q4_sc(sc, int(g1))), M1 = dmin * float(q4_m(sc, int(g1)));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t wv = qs[i];
        const uint32_t lo = wv & 0x0F0F0F0Fu, hi = (wv >> 4) & 0x0F0F0F0Fu;
        const float a0 = q4_value(D0, M0, byte_of(lo, 0)), a1 = q4_value(D0, M0, byte_of(lo, 1));
        const float a2 = q4_value(D0, M0, byte_of(lo, 2)), a3 = q4_value(D0, M0, byte_of(lo, 3));
        const float b0 = q4_value(D1, M1, byte_of(hi, 0)), b1 = q4_value(D1, M1, byte_of(hi, 1));
        const float b2 = q4_value(D1, M1, byte_of(hi, 2)), b3 = q4_value(D1, M1, byte_of(hi, 3));
        out.v[i >> 1][(i & 1) * 2 + 0] = pack_f16x2(a0, a1);
        out.v[i >> 1][(i & 1) * 2 + 1] = pack_f16x2(a2, a3);
        out.v[2 + (i >> 1)][(i & 1) * 2 + 0] = pack_f16x2(b0, b1);
        out.v[2 + (i >> 1)][(i & 1) * 2 + 1] = pack_f16x2(b2, b3);
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

// Q6_K: k step s covers elements 64*(s%4)..+63 of super-block s/4: half
// h = (s%4)/2, quarters 2*(s%2) and 2*(s%2)+1.  Thread half hh takes quarter
// qa = 2*(s%2)+hh, l = 0..31 (k offsets 32hh .. 32hh+31):
//   v = nibble of ql[64h + 32*(qa&1) + l] (low if qa < 2) | qh[32h + l] bits 2qa..2qa+1 << 4.
template <int LAYOUT>
__device__ __forceinline__ void q6_tile(const uint8_t *__restrict__ w, uint32_t row, uint32_t nb, uint32_t s,
                                        uint32_t hh, WRun &out) {
    const uint32_t b = s >> 2, sr = s & 3, h = sr >> 1, qa = 2 * (sr & 1) + hh;
    u32x4 ql[2], qh[2], scw;
    uint32_t dbits;
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
    const float d = lo_half(dbits);
    // scales for l < 16 and l >= 16: sc[8h + 2qa + (l/16)]
    const uint32_t si = 8 * h + 2 * qa;
    const float Dl = d * float(int8_t(byte_of(scw[si >> 2], int(si & 3))));
    const float Dh = d * float(int8_t(byte_of(scw[(si + 1) >> 2], int((si + 1) & 3))));
    const uint32_t nshift = qa >= 2 ? 4 : 0, hshift = 2 * qa;
#pragma unroll
    for (int c = 0; c < 2; ++c)        // l = 16c .. 16c+15
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // l = 16c + 4i .. +3
            const uint32_t nib = (ql[c][i] >> nshift) & 0x0F0F0F0Fu;
            const uint32_t hb = ((qh[c][i] >> hshift) & 0x03030303u) << 4;
            const uint32_t v = nib | hb;
            const float D = c ? Dh : Dl;
            const float e0 = q6_value(D, byte_of(v, 0)), e1 = q6_value(D, byte_of(v, 1));
            const float e2 = q6_value(D, byte_of(v, 2)), e3 = q6_value(D, byte_of(v, 3));
            out.v[2 * c + (i >> 1)][(i & 1) * 2 + 0] = pack_f16x2(e0, e1);
            out.v[2 * c + (i >> 1)][(i & 1) * 2 + 1] = pack_f16x2(e2, e3);
        }
    out.k_lo = 32 * int(hh);
    out.k_hi = 32 * int(hh) + 16;
}

template <int TYPE, int LAYOUT, int ACC, bool PAIR>
__global__ __launch_bounds__(kThreads, 2) void gemm_kernel(
    const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, const uint16_t *__restrict__ x,
    void *__restrict__ out, uint32_t cols, uint32_t rows, uint32_t batch, uint32_t ntok_tiles) {
    __shared__ __attribute__((aligned(16))) _Float16 Xs[TT * LDSW];
    __shared__ __attribute__((aligned(16))) _Float16 Ws[TC * LDSW];

    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wt = wave >> 1, wn = wave & 1;
    // token tile fastest so that token tile == XCD when ntok_tiles == 8
    const uint32_t tt = blockIdx.x % ntok_tiles, ct = blockIdx.x / ntok_tiles;
    const uint32_t t0 = tt * TT;
    constexpr uint32_t kRowsPerTile = PAIR ? TC / 2 : TC;
    const uint32_t r0 = ct * kRowsPerTile;
    const uint32_t nb = cols / kQK, nsteps = cols / KS;

    // weight producer role: column wc of the tile, k half hh
    const uint32_t wc = tid >> 1, hh = tid & 1;
    const uint8_t *wsrc = (PAIR && wc >= TC / 2) ? w1 : w0;
    const uint32_t wrow = r0 + (PAIR ? (wc % (TC / 2)) : wc);
    const bool wvalid = wrow < rows;

    float16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    // LDS column of B fragment j for this wave
    auto bcol = [&](int j) -> uint32_t {
        if constexpr (PAIR) return uint32_t(j) * (TC / 2) + wn * 32;   // gate / up of the same 32 rows
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
        if (wvalid) {
            if constexpr (TYPE == Q4_K) q4_tile<LAYOUT>(wsrc, wrow, nb, s, hh, wr);
            else q6_tile<LAYOUT>(wsrc, wrow, nb, s, hh, wr);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) wr.v[i] = u32x4{0u, 0u, 0u, 0u};
            wr.k_lo = TYPE == Q4_K ? 16 * int(hh) : 32 * int(hh);
            wr.k_hi = TYPE == Q4_K ? 32 + 16 * int(hh) : 32 * int(hh) + 16;
        }
        __syncthreads();  // previous step's fragments are consumed
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t idx = tid + kThreads * i, tok = idx >> 3, part = idx & 7;
            *reinterpret_cast<u32x4 *>(&Xs[tok * LDSW + part * 8]) = xr[i];
        }
        {
            _Float16 *wrow_lds = &Ws[wc * LDSW];
            *reinterpret_cast<u32x4 *>(wrow_lds + wr.k_lo) = wr.v[0];
            *reinterpret_cast<u32x4 *>(wrow_lds + wr.k_lo + 8) = wr.v[1];
            *reinterpret_cast<u32x4 *>(wrow_lds + wr.k_hi) = wr.v[2];
            *reinterpret_cast<u32x4 *>(wrow_lds + wr.k_hi + 8) = wr.v[3];
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
        if constexpr (ACC == ACC_FP16) {
            if ((s & 3) == 3) {
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
#pragma unroll
                        for (int v = 0; v < 16; ++v) acc[i][j][v] = round_f16(acc[i][j][v]);
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
                const float g = acc[i][0][v], u = acc[i][1][v];
                reinterpret_cast<_Float16 *>(out)[size_t(t) * rows + r] = _Float16(gelu_tanh(g) * u);
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const uint32_t r = r0 + wn * 64 + j * 32 + (lane & 31);
                    if (r < rows) reinterpret_cast<float *>(out)[size_t(t) * rows + r] = acc[i][j][v];
                }
            }
        }
    }
}

template <int TYPE, int LAYOUT, bool PAIR>
hipError_t launch_mode(int acc, const uint8_t *w, const uint8_t *up, const uint16_t *x, void *out, uint32_t cols,
                       uint32_t rows, uint32_t batch, hipStream_t stream) {
    const uint32_t ntok = (batch + TT - 1) / TT;
    const uint32_t rows_per_tile = PAIR ? TC / 2 : TC;
    const uint32_t ncol = (rows + rows_per_tile - 1) / rows_per_tile;
    const dim3 grid(ntok * ncol), block(kThreads);
    if (acc == ACC_FP16)
        gemm_kernel<TYPE, LAYOUT, ACC_FP16, PAIR><<<grid, block, 0, stream>>>(w, up, x, out, cols, rows, batch, ntok);
    else
        gemm_kernel<TYPE, LAYOUT, ACC_FP32, PAIR><<<grid, block, 0, stream>>>(w, up, x, out, cols, rows, batch, ntok);
    return hipGetLastError();
}

template <int TYPE, bool PAIR>
hipError_t launch_layout(int layout, int acc, const uint8_t *w, const uint8_t *up, const uint16_t *x, void *out,
                         uint32_t cols, uint32_t rows, uint32_t batch, hipStream_t stream) {
    if (layout == CDNA4) return launch_mode<TYPE, CDNA4, PAIR>(acc, w, up, x, out, cols, rows, batch, stream);
    return launch_mode<TYPE, NSMFFN, PAIR>(acc, w, up, x, out, cols, rows, batch, stream);
}

}  // namespace

hipError_t launch_gemm(int type, int layout, int acc, const uint8_t *w, const uint8_t *up, const uint16_t *x,
                       void *out, uint32_t cols, uint32_t rows, uint32_t batch, const Workspace &ws,
                       hipStream_t stream) {
    (void)ws;
    if (up) return launch_layout<Q4_K, true>(layout, acc, w, up, x, out, cols, rows, batch, stream);
    if (type == Q4_K) return launch_layout<Q4_K, false>(layout, acc, w, nullptr, x, out, cols, rows, batch, stream);
    return launch_layout<Q6_K, false>(layout, acc, w, nullptr, x, out, cols, rows, batch, stream);
}

}  // namespace ns
