// ns_gemm_f16.hip -- prefill GEMM in the FP16 mode on the CDNA4 layout, for gfx950.
//
// Replaces, for the FP16-accumulation (fast_swa) layers of the .nsmffn path,
//   gemma_q4k_gate_up_geglu_metal_rm32_f16acc_f16 (metal/gemma4.metal:379-383;
//     gate_up_geglu_rm32 with fast_swa, metal_engine.mm:288, :566)   -> Q4_K, PAIR
//   gemma_q4k_mma_metal_f16acc_f16 / gemma_q6k_mma_metal_f16acc_f16 (metal:391-395,
//     :486-490; ffn_down with fast_swa, mm:289, :573)                -> Q4_K / Q6_K
//
// Tile values are the fp16 form of ns_tile16.hpp: F = RNE16(q*2^-24*A + B), one
// packed FMA per two weights straight from the quant bits, with the row's
// power-of-two scale c_r folded into A and B.  Nothing is rescaled per
// super-block and the Q4_K min term rides in the tile, so the only per-weight
// VALU work is the unpack and that FMA.
//
// Work split.  One workgroup = 4 waves, one wave per SIMD, one workgroup per CU
// (128 KiB of LDS).  A workgroup computes 256 tokens x 256 B columns; each wave
// owns all 256 tokens (8 MFMA tiles of v_mfma_f32_32x32x16_f16) and 64 columns
// (2 tiles): for the gate/up pair, 32 gate rows and the same 32 up rows, so
// GeGLU runs in registers.  The 256 fp32 accumulators of a wave live in AGPRs.
// Each wave decodes the B fragments its own MFMAs consume straight from the
// CDNA4 image into registers: lane l holds weight row l%32 at 8 consecutive k,
// which in the CDNA4 layout are 8 contiguous bytes of that row's 16-byte chunk
// (lanes 0-31 and 32-63 take the two halves, so one load instruction reads
// 512 contiguous bytes).  Each decoded fragment feeds 8 MFMAs.  x streams into
// LDS by buffer_load ... lds (four 32 KiB buffers, one barrier per 64-wide k
// step) and each A fragment (ds_read_b128) feeds 2 MFMAs.
//
// Row scales: every wave first reads the d (and dmin) of all super-blocks of its
// rows and forms c_r (ns_tile16.hpp), so a row's tiles do not depend on how K
// is split.  Split K (the 3840-row down projection) writes fp32 parts already
// multiplied by 1/c_r; the last workgroup of a tile to arrive adds them in part
// order and rounds once (FP16 mode output: 11 significant bits, fp32 range).
#include <type_traits>

#include "ns_internal.hpp"
#include "ns_quant.hpp"
#include "ns_tile16.hpp"

namespace ns {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int TT = 256;               // tokens per workgroup (= per wave)
constexpr int MI = TT / 32;           // 32-token MFMA tiles per wave
constexpr int NJ = 2;                 // 32-column MFMA tiles per wave
constexpr int TC = kWaves * NJ * 32;  // B columns per workgroup
constexpr int KS = 64;                // k per step
constexpr int XBUF = 4;               // x buffers in LDS (x streams three steps ahead)
constexpr int XDMA = TT * KS * 2 / 16 / kThreads;  // 16-byte x chunks per thread per step

__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, int(bytes), 0x00020000);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, int(off), 0, 0); }
__device__ __forceinline__ u32x2 bload8(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b64(r, int(off), 0, 0); }
__device__ __forceinline__ uint32_t bload4(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b32(r, int(off), 0, 0); }
__device__ __forceinline__ uint32_t bload2(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b16(r, int(off), 0, 0); }

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt bits 3:0 and 15:14; expcnt and lgkmcnt left at max).
template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ float round_f16p(float v) {
    uint32_t b = __builtin_bit_cast(uint32_t, v);
    b = (b + 0x0fffu + ((b >> 13) & 1u)) & 0xffffe000u;
    return __builtin_bit_cast(float, b);
}

// Raw bytes of one column (lane row) that the decode of one step needs.
//   Q4_K, per step s (groups 2p, 2p+1 of super-block s/4, p = s%4): qs bytes
//     8hl..8hl+7 of chunks 1+2p (qa) and 2+2p (qb), and the block header.
//   Q6_K, per step pair (s/2: half h = (s%4)/2 of the super-block): ql bytes
//     8hl..+7 of chunks 4h..4h+3, qh bytes 8hl..+7 of chunks 8+2h, 9+2h, the
//     scales (chunk 12) and d.
// Only bytes a step uses are loaded: a loaded register the step leaves unused would be
// reused by the register allocator while its load is in flight, and the compiler would
// then wait for that load at once.
struct RawQ4 {
    u32x2 qa, qb;
    u32x4 hdr;  // d, dmin, scales[0..7] (steps p = 0, 1; .w unset) or scales[0..11] (p = 2, 3)
};
struct RawQ6 {
    u32x2 ql[4], qh[2];
    u32x2 sc;  // scales[8h .. 8h+7] of the step pair's half h
    uint32_t d;
};
typedef unsigned int u32x3 __attribute__((ext_vector_type(3)));

template <int TYPE, bool PAIR>
__global__ __launch_bounds__(kThreads, 1) void gemm_f16_kernel(
    const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, const uint16_t *__restrict__ x,
    void *__restrict__ out, float *__restrict__ partial, uint32_t *__restrict__ counters, uint32_t cols,
    uint32_t rows, uint32_t batch, uint32_t ntok_tiles, uint32_t ncol_tiles, uint32_t kparts, uint32_t wbytes,
    uint32_t rs_spin, uint32_t *__restrict__ err) {
    constexpr bool Q4 = TYPE == Q4_K;
    using Raw = typename std::conditional<Q4, RawQ4, RawQ6>::type;
    // Four separate LDS objects rather than one array: the compiler then sees that a DMA into
    // one buffer cannot alias the fragment reads of another, and issues those reads without
    // first waiting for every DMA in flight.
    __shared__ __attribute__((aligned(16))) u32x4 Xs0[TT * 8], Xs1[TT * 8], Xs2[TT * 8], Xs3[TT * 8];
    static_assert(XBUF == 4, "one LDS object per x buffer");
    auto xbuf = [&](int buf) -> u32x4 * { return buf == 0 ? Xs0 : buf == 1 ? Xs1 : buf == 2 ? Xs2 : Xs3; };
    __shared__ uint32_t last_flag, late_flag;

    uint32_t tid = threadIdx.x, lane = tid & 63, hl = lane >> 5;  // formed again after the main loop
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // XCD-aware order: workgroup L runs on XCD L % 8; work item q = (kp * ntok + tt) * ncol + ct,
    // and XCD x takes the contiguous run [x*W/8, (x+1)*W/8), so its L2 holds whole x slices.
    const uint32_t nwg = gridDim.x, w8 = nwg / 8, L = blockIdx.x;
    const uint32_t q = L < 8 * w8 ? (L % 8) * w8 + L / 8 : L;
    const uint32_t ct = q % ncol_tiles, g = q / ncol_tiles, tt = g % ntok_tiles, kp = g / ntok_tiles;
    const uint32_t tile = tt + ntok_tiles * ct;
    const uint32_t t0 = tt * TT;
    const uint32_t nb = cols / kQK;
    const uint32_t sb0 = kp * nb / kparts, sb1 = (kp + 1) * nb / kparts;

    // B column of tile j for this lane (a weight row), and the matrix it comes from.
    constexpr uint32_t kRowsPerTile = PAIR ? TC / 2 : TC;
    const uint32_t r0 = ct * kRowsPerTile;
    auto brow = [&](int j) -> uint32_t {
        if constexpr (PAIR) return r0 + wave * 32 + (lane & 31);  // j 0 = gate, 1 = up, same row
        else return r0 + wave * 64 + uint32_t(j) * 32 + (lane & 31);
    };
    const rsrc_t wsrc0 = make_rsrc(w0, wbytes);
    const rsrc_t wsrc1 = make_rsrc(PAIR ? w1 : w0, wbytes);
    auto wsrc = [&](int j) { return (PAIR && j == 1) ? wsrc1 : wsrc0; };
    const rsrc_t xsrc = make_rsrc(x, batch * cols * 2);

    // byte offset of chunk c of row r, super-block b, in the CDNA4 image
    auto chunk_off = [&](uint32_t r, uint32_t b, uint32_t c) -> uint32_t {
        return uint32_t(region_offset(TYPE, r / kRowTile, b, nb)) + (c * kRowTile + r % kRowTile) * 16;
    };

    // ---- row scales (rows past `rows` read zeros: M = 0, c = 1, tiles 0).  The two lane
    // halves hold the same rows: each reads every other super-block's factors, 16 loads in
    // flight per round trip, and the halves swap their maxima.
    float c24[NJ], inv_c[NJ];
    {
        float M[NJ] = {};
        for (uint32_t b0 = 0; b0 < nb; b0 += 32) {
            uint32_t dd[NJ][16];
#pragma unroll
            for (int u = 0; u < 16; ++u)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const uint32_t b = b0 + 2 * uint32_t(u) + hl, r = brow(j);
                    // a block past nb reads the next slab or beyond the tensor: zeros or
                    // another row's factors, so it is masked below
                    if constexpr (Q4) dd[j][u] = bload4(wsrc(j), chunk_off(r, b, 0));
                    else dd[j][u] = bload2(wsrc(j), uint32_t(region_offset(TYPE, r / kRowTile, b, nb)) +
                                                        kQ6Chunks * 1024 + (r % kRowTile) * 2);
                }
#pragma unroll
            for (int u = 0; u < 16; ++u)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const bool in = b0 + 2 * uint32_t(u) + hl < nb;
                    const float a = __builtin_fabsf(lo_half(dd[j][u]));
                    const float m = Q4 ? __builtin_fmaxf(a, __builtin_fabsf(hi_half(dd[j][u]))) : a;
                    M[j] = in ? __builtin_fmaxf(M[j], m) : M[j];
                }
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            M[j] = __builtin_fmaxf(M[j], __shfl_xor(M[j], 32));
            row_scale(M[j], c24[j], inv_c[j], !Q4);
        }
    }

    // ---- raw loads: Q4_K one slot per step, Q6_K one per step pair.  The lane's part of an
    // offset (row, lane half) is a VGPR fixed for the kernel; the step's part (super-block,
    // chunk) goes in the instruction's uniform soffset, so a load costs no address VALU.
    uint32_t voff[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const uint32_t r = brow(j);
        voff[j] = uint32_t(region_offset(TYPE, r / kRowTile, 0, nb)) + (r % kRowTile) * 16;
    }
    constexpr uint32_t kRegion = kRowTile * block_bytes(TYPE);  // bytes of one (slab, super-block) region
    // Column jc's raw bytes of step s (jc < 0: every column).
    auto load_raw = [&](uint32_t s, Raw (&raw)[NJ], int jc = -1) {
        const uint32_t b = s >> 2;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            if (jc >= 0 && j != jc) continue;
            if constexpr (Q4) {
                const uint32_t p = s & 3;
                raw[j].qa = __builtin_amdgcn_raw_buffer_load_b64(wsrc(j), int(voff[j] + 8 * hl), int(b * kRegion + (1 + 2 * p) * 1024), 0);
                raw[j].qb = __builtin_amdgcn_raw_buffer_load_b64(wsrc(j), int(voff[j] + 8 * hl), int(b * kRegion + (2 + 2 * p) * 1024), 0);
                if (p < 2) {  // groups 0-3: d, dmin, scales[0..7]
                    const u32x3 t = __builtin_amdgcn_raw_buffer_load_b96(wsrc(j), int(voff[j]), int(b * kRegion), 0);
                    raw[j].hdr = u32x4{t.x, t.y, t.z, 0u};
                } else {
                    raw[j].hdr = __builtin_amdgcn_raw_buffer_load_b128(wsrc(j), int(voff[j]), int(b * kRegion), 0);
                }
            } else {
                const uint32_t h = (s >> 1) & 1;
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
                    raw[j].ql[kk] = __builtin_amdgcn_raw_buffer_load_b64(wsrc(j), int(voff[j] + 8 * hl),
                                                                         int(b * kRegion + (4 * h + kk) * 1024), 0);
#pragma unroll
                for (int c = 0; c < 2; ++c)
                    raw[j].qh[c] = __builtin_amdgcn_raw_buffer_load_b64(wsrc(j), int(voff[j] + 8 * hl),
                                                                        int(b * kRegion + (8 + 2 * h + c) * 1024), 0);
                raw[j].sc = __builtin_amdgcn_raw_buffer_load_b64(wsrc(j), int(voff[j] + 8 * h), int(b * kRegion + 12 * 1024), 0);
                // d of row r: region + 13 KiB + 2*(r%64) = voff - 14*(r%64) + 13 KiB
                raw[j].d = __builtin_amdgcn_raw_buffer_load_b16(wsrc(j), int(voff[j] - 14 * (brow(j) % kRowTile)),
                                                                int(b * kRegion + kQ6Chunks * 1024), 0);
            }
        }
    };
    constexpr int kRawLoads = Q4 ? 3 * NJ : 8 * NJ;  // vector loads per load_raw
    // VALU instructions placed after each MFMA of a k16 sub-step (a scheduling hint: the
    // next step's fragment decode, ~24 (Q4_K) or ~36 (Q6_K) per sub-step)
    constexpr int kValuPerMfma = Q4 ? 2 : 3;
    // the first sub-step also carries the factors of the next step
    constexpr int kValuFirst = Q4 ? 4 : 5;

    // ---- fragments of step s from its raw bytes: fb[j][kk] covers k 16kk + 8hl + 0..7.
    // Factors first (one set per column and step, Q6_K one per k16 sub-step), then
    // one fragment at a time, so the decode of the next step can be spread over the
    // MFMAs of this one.
    struct Factors {
        half2_t A[NJ][Q4 ? 2 : 4], B[NJ][Q4 ? 2 : 4];
    };
    auto factors = [&](uint32_t s, const Raw (&raw)[NJ], Factors &F) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            if constexpr (Q4) {
                const uint32_t p = s & 3;
                const float d = lo_half(raw[j].hdr.x), dmin = hi_half(raw[j].hdr.x);
                const Q4Scales sc = q4_scales(raw[j].hdr.y, raw[j].hdr.z, raw[j].hdr.w);
                const float dc = d * c24[j], mc = -dmin * (c24[j] * 5.9604644775390625e-08f);  // c = c24 * 2^-24
#pragma unroll
                for (int hi = 0; hi < 2; ++hi) {
                    F.A[j][hi] = splat(_Float16(dc * float(q4_sc(sc, int(2 * p) + hi))));
                    F.B[j][hi] = splat(_Float16(mc * float(q4_m(sc, int(2 * p) + hi))));
                }
            } else {
                // step s: half h = (s%4)/2, quarters Q = 2*(s%2) + kk/2; scale sc[8h + kk%2 + 2Q]
                const uint32_t sr = s & 3, qb2 = 2 * (sr & 1);
                const float d = lo_half(raw[j].d);
                const float dc = d * c24[j], dm = -32.0f * d * (c24[j] * 5.9604644775390625e-08f);
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    const uint32_t si = uint32_t(kk & 1) + 2 * (qb2 + uint32_t(kk >> 1));  // scale 8h + si
                    const float scf = float(int(int8_t(byte_of(raw[j].sc[si >> 2], int(si & 3)))));
                    F.A[j][kk] = splat(_Float16(dc * scf));
                    F.B[j][kk] = splat(_Float16(dm * scf));
                }
            }
        }
    };
    auto frag = [&](uint32_t s, const Raw (&raw)[NJ], const Factors &F, int j, int kk) -> half8_t {
        u32x4 f;
        if constexpr (Q4) {
            // kk 0: qa low nibbles (group 2p, l = 8hl..), 1: qb low (l = 16 + 8hl..), 2, 3: high nibbles
            const u32x2 w = (kk & 1) ? raw[j].qb : raw[j].qa;
            const int hi = kk >> 1;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                uint32_t lo[2], hv[2];
                q4_f16x8(w[e], F.A[j][0], F.B[j][0], F.A[j][1], F.B[j][1], lo, hv);
                f[2 * e] = hi ? hv[0] : lo[0];
                f[2 * e + 1] = hi ? hv[1] : lo[1];
            }
        } else {
            // v = (ql nibble) | ((qh >> 2Q) & 3) << 4 for quarter Q = 2*(s%2) + kk/2, l = 16*(kk%2) + 8hl + 0..7
            const uint32_t sr = s & 3, Q = 2 * (sr & 1) + uint32_t(kk >> 1);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t lq = raw[j].ql[kk][e], hq = raw[j].qh[kk & 1][e];
                const uint32_t lo4 = (sr & 1) ? (lq >> 4) & 0x0F0F0F0Fu : lq & 0x0F0F0F0Fu;
                const uint32_t v = lo4 | (((hq >> (2 * Q)) & 0x03030303u) << 4);
                uint32_t o[2];
                q6_f16x4(v, F.A[j][kk], F.B[j][kk], o);
                f[2 * e] = o[0];
                f[2 * e + 1] = o[1];
            }
        }
        return __builtin_bit_cast(half8_t, f);
    };

    // x(s) -> Xs[s % 4] by LDS DMA: instruction i of wave w fills rows 8*(w + 4i) .. +7;
    // lane L writes chunk L of that 1 KiB block (row +L/8, position L%8), i.e. global
    // chunk (L%8) ^ ((R>>1)&7) of the row, which keeps fragment reads conflict-free.
    // The lane's global offset is fixed; the step adds s*128 bytes as the uniform soffset.
    uint32_t xoff[XDMA];
#pragma unroll
    for (int i = 0; i < XDMA; ++i) {
        const uint32_t R = 8 * (wave + kWaves * uint32_t(i)) + (lane >> 3), c = (lane & 7) ^ ((R >> 1) & 7);
        xoff[i] = ((t0 + R) * cols + 8 * c) * 2;
    }
    auto dma_x = [&](uint32_t s, int buf, int i0 = 0, int i1 = XDMA) {  // instructions i0 .. i1-1
#pragma unroll
        for (int i = 0; i < XDMA; ++i) {
            if (i < i0 || i >= i1) continue;
            const uint32_t rbase = 8 * (wave + kWaves * uint32_t(i));
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xsrc, (__attribute__((address_space(3))) void *)(xbuf(buf) + rbase * 8), 16, xoff[i], s * KS * 2, 0, 0);
        }
    };
    // A fragment (token tile i, k16 sub-step kk) of buffer buf: row R = 32i + l, chunk 2kk + hl
    const uint32_t aoff = (lane & 31) * 8 + 0;  // row part of the LDS index (in 16-byte chunks)
    const uint32_t aswz = ((lane & 31) >> 1) & 7;  // (R >> 1) & 7 is the same for every i
    auto load_a = [&](int buf, int kk, half8_t (&dst)[MI]) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
            dst[i] = __builtin_bit_cast(half8_t, xbuf(buf)[i * 256 + aoff + ((2 * kk + hl) ^ aswz)]);
    };

    float16_t acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    // Pipeline.  x streams three steps ahead through four LDS buffers (step s reads buffer
    // s % 4 = its index within the super-block, a compile-time constant; x(s+3) goes into
    // buffer (s-1) % 4, whose last reads, at step s-1, every wave finished before the
    // barrier ending step s-1; the barrier ending step s makes x(s+2) visible).  Raw weights:
    // Q4_K step s decodes from slot s % 4, refilled with raw(s+4) during step s; Q6_K step
    // pair u = s/2 uses slot u&1, refilled with pair u+2 during step 2u+1.  A refill has
    // landed by the end of the step after the one that issued it.  The decode of step s+1
    // runs during the MFMAs of step s, so fragments are double-buffered.
    constexpr int kSlots = Q4 ? 4 : 2;
    Raw raw[kSlots][NJ];
    const uint32_t sbeg = 4 * sb0, send = 4 * sb1;
    dma_x(sbeg, 0);
    dma_x(sbeg + 1, 1);
    dma_x(sbeg + 2, 2);
    if constexpr (Q4) {
#pragma unroll
        for (int k = 0; k < kSlots; ++k) load_raw(sbeg + uint32_t(k), raw[k]);
    } else {
        load_raw(sbeg, raw[0]);
        load_raw(sbeg + 2, raw[1]);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    half8_t fb[2][NJ][4];
    // A fragments: a[kk & 1] feeds sub-step kk; the kk = 0 fragments of step s+1 are read
    // during the last sub-step of step s, before the barrier that ends it.
    half8_t a[2][MI];
    load_a(0, 0, a[0]);
    {
        Factors F;
        factors(sbeg, raw[0], F);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) fb[0][j][kk] = frag(sbeg, raw[0], F, j, kk);
    }

    for (uint32_t sb = sb0; sb < sb1; ++sb) {
#pragma unroll
        for (int jstep = 0; jstep < 4; ++jstep) {
            const uint32_t s = 4 * sb + uint32_t(jstep);
            const int cur = jstep & 1, nxt = cur ^ 1;
            // slot holding raw(s+1)
            const int rn = Q4 ? ((jstep + 1) & 3) : (((jstep + 1) >> 1) & 1);
            // Refills and the next step's decode run unconditionally, also past the last step:
            // such loads read in-bounds or descriptor-clamped bytes (zeros) into registers and
            // into an x buffer no wave reads again, and a branch around them would make the
            // compiler wait for every load at the merge.
            // Each k16 sub-step is its own scheduling region: its 16 MFMAs (independent
            // accumulators), the next sub-step's 8 A reads (in the last sub-step: the first
            // ones of step s+1, from buffer (s+1) % 4, whose x every wave waited for before
            // the barrier that ended step s-1) and one fragment per column of the next
            // step's decode, issued interleaved so that the LDS and VALU work runs in the
            // MFMA shadow.  The next step's factors precede.
            Factors F;
            factors(s + 1, raw[rn], F);
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                // The step's global loads, spread over its four sub-steps: x(s+3) into buffer
                // (s-1) % 4, two instructions per sub-step, and the raw refill, one column per
                // sub-step (Q4_K: slot s % 4, decoded during step s-1; Q6_K at odd steps: the
                // pair slot of steps s-1 and s).  Issued as one burst after the barrier, the
                // four waves' loads stalled the matrix pipe for ~15% of every step.
                static_assert(XDMA == 8, "two x instructions per sub-step");
                dma_x(s + 3, (jstep + 3) & 3, 2 * kk, 2 * kk + 2);
                if (kk < NJ) {
                    if constexpr (Q4) load_raw(s + 4, raw[jstep], kk);
                    else if (jstep & 1) load_raw(s + 3, raw[(jstep >> 1) & 1], kk);
                }
                if (kk < 3) load_a(jstep, kk + 1, a[(kk + 1) & 1]);
                else load_a((jstep + 1) & 3, 0, a[0]);
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[kk & 1][i], fb[cur][j][kk], acc[i][j], 0, 0, 0);
#pragma unroll
                for (int j = 0; j < NJ; ++j) fb[nxt][j][kk] = frag(s + 1, raw[rn], F, j, kk);
#pragma unroll
                for (int m = 0; m < MI; ++m) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    if (kk == 0) __builtin_amdgcn_sched_group_barrier(0x002, kValuFirst, 0);
                    else __builtin_amdgcn_sched_group_barrier(0x002, kValuPerMfma, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    if (kk == 0) __builtin_amdgcn_sched_group_barrier(0x002, kValuFirst, 0);
                    else __builtin_amdgcn_sched_group_barrier(0x002, kValuPerMfma, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            // x(s+2) must be in LDS for every wave (step s+1 reads its first fragments in its
            // last sub-step): wait for its DMA (issued at step s-1), then meet at the barrier.
            // The wait leaves in flight exactly the loads issued during step s (x(s+3), and the
            // raw refill: Q4_K every step, Q6_K at odd steps), so it does not depend on the
            // order in which the compiler schedules them within the step; everything issued
            // at step s-1, x(s+2) included, has landed.  The barrier also orders every wave's
            // reads of buffer s % 4 (the fragments of step s, all consumed by its MFMAs) before
            // step s+1's DMA of x(s+4) into that buffer.
            // The barrier is the bare s_barrier: __syncthreads() adds a workgroup fence, which
            // the compiler implements by waiting for every LDS DMA in flight (x(s+2), x(s+3)
            // too).  The explicit wait above covers what the other waves read next, and the
            // signal fences keep the compiler from moving memory accesses across the barrier.
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (Q4) vm_wait<kRawLoads + XDMA>();
            else if (jstep & 1) vm_wait<kRawLoads + XDMA>();
            else vm_wait<XDMA>();
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_barrier();
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
        }
    }
    vm_wait<0>();  // the refills issued past the last step have landed
    // Past the main loop the lane values and 1/c_r = 2^24 / (c_r 2^24) (exact: powers of two)
    // are formed again rather than kept live across it, where every VGPR is taken and they
    // would go to scratch.  The lane index comes from a volatile asm so that the compiler
    // cannot hoist it above the loop.
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane));
    hl = lane >> 5;
    tid = wave * 64 + lane;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
        inv_c[j] = __builtin_bit_cast(float, (uint32_t(2 * 127 + 24) << 23) - __builtin_bit_cast(uint32_t, c24[j]));

    // ---- outputs.  32x32 D layout: lane holds column lane%32 and rows
    // 8*(v/4) + 4*(lane/32) + v%4 for v = 0..15.
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] *= inv_c[j];
    auto tok_of = [&](int i, int v) -> uint32_t {
        return t0 + uint32_t(i) * 32 + 8 * uint32_t(v >> 2) + 4 * hl + uint32_t(v & 3);
    };
    auto emit = [&](uint32_t t, const float (&val)[NJ]) {
        if (t >= batch) return;
        if constexpr (PAIR) {
            const uint32_t r = brow(0);
            const float gv = round_f16p(val[0]), uv = round_f16p(val[1]);
            if (r < rows) reinterpret_cast<_Float16 *>(out)[size_t(t) * rows + r] = _Float16(gelu_tanh(gv) * uv);
        } else {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const uint32_t r = brow(j);
                if (r < rows) reinterpret_cast<float *>(out)[size_t(t) * rows + r] = round_f16p(val[j]);
            }
        }
    };
    auto write_out = [&](int i, auto get) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            float val[NJ];
#pragma unroll
            for (int j = 0; j < NJ; ++j) val[j] = get(v, j);
            emit(tok_of(i, v), val);
        }
    };

    if (kparts == 1) {
#pragma unroll
        for (int i = 0; i < MI; ++i) write_out(i, [&](int v, int j) { return acc[i][j][v]; });
        return;
    }

    // ---- split K.  Parts [kp][plane][ntok*TT][ncol*rows per tile] (PAIR: gate, up), padded
    // to whole tiles so no part store or load needs a guard; a slot is a 32-bit byte offset
    // from the part's (uniform) base (the host keeps one part under 4 GiB).
    constexpr uint32_t kPlanes = PAIR ? 2 : 1;
    const uint32_t tpad = ntok_tiles * TT, rpad = ncol_tiles * kRowsPerTile;
    const size_t pstride = size_t(kPlanes) * tpad * rpad;
    const uint32_t rstride = rpad * 4u;
    uint32_t lane_off[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
        lane_off[j] = ((PAIR ? uint32_t(j) : 0u) * tpad + t0 + 4 * hl) * rstride + brow(j) * 4u;
    auto poff = [&](int i, int v, int j) -> uint32_t {
        return (uint32_t(i) * 32 + 8 * uint32_t(v >> 2) + uint32_t(v & 3)) * rstride + lane_off[j];
    };
    auto pbase = [&](uint32_t part) -> char * { return reinterpret_cast<char *>(partial + part * pstride); };
    if (rs_spin != 0) {
        // Reduce-scatter (the host launches it only when the whole grid fits on the device at
        // once, so the kparts workgroups of a tile run together): part kp owns token sub-tiles
        // [own_lo, own_hi) of the tile.  Each part stores the sub-tiles it does not own, keeps
        // its own in LDS (slot k in x buffer k, free after the main loop), counts one arrival on
        // written[tile] once its stores are acknowledged, waits until every part has, then adds
        // the parts of its own sub-tiles in part order (its own from LDS) and writes them.  Every
        // part reads and writes a 1/kparts share, where the last arrival of the other form reads
        // every part alone.  The wait is bounded: a part whose limit runs out writes its
        // sub-tiles as NaN.  The last part past the wait clears both counters.
        const uint32_t ntiles = ntok_tiles * ncol_tiles;
        uint32_t *written = counters + tile, *departed = counters + ntiles + tile;
        const uint32_t own_lo = kp * MI / kparts, own_hi = (kp + 1) * MI / kparts;
        __syncthreads();  // every wave is past its last read of the x buffers
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            if (uint32_t(i) >= own_lo && uint32_t(i) < own_hi) {
                float *slot = reinterpret_cast<float *>(xbuf(int(uint32_t(i) - own_lo) & 3));
#pragma unroll
                for (int v = 0; v < 16; ++v)
#pragma unroll
                    for (int j = 0; j < NJ; ++j) slot[(v * NJ + j) * kThreads + tid] = acc[i][j][v];
            } else {
#pragma unroll
                for (int v = 0; v < 16; ++v)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        __hip_atomic_store(reinterpret_cast<float *>(pbase(kp) + poff(i, v, j)), acc[i][j][v],
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __syncthreads();
        if (tid == 0) {
            __hip_atomic_fetch_add(written, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            uint32_t late = 0;
            for (uint32_t it = 0; __hip_atomic_load(written, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < kparts;) {
                __builtin_amdgcn_s_sleep(2);
                if (++it >= rs_spin) {
                    late = 1;
                    record_wait_timeout(err, kWaitGemm);
                    break;
                }
            }
            late_flag = late;
            if (__hip_atomic_fetch_add(departed, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == kparts - 1) {
                __hip_atomic_store(written, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(departed, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __syncthreads();
        const bool late = late_flag != 0;
        for (uint32_t i = own_lo; i < own_hi; ++i) {
            const float *slot = reinterpret_cast<const float *>(xbuf(int(i - own_lo) & 3));
            float sum[16][NJ];
            for (uint32_t p0 = 0; p0 < kparts; p0 += 4) {
                float pv[4][16][NJ];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    // this part's own slot holds no value for these sub-tiles: read from LDS below
                    const uint32_t part = __builtin_elementwise_min(p0 + uint32_t(u), kparts - 1);
#pragma unroll
                    for (int v = 0; v < 16; ++v)
#pragma unroll
                        for (int j = 0; j < NJ; ++j)
                            pv[u][v][j] = __hip_atomic_load(reinterpret_cast<float *>(pbase(part) + poff(int(i), v, j)),
                                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
#pragma unroll
                for (int v = 0; v < 16; ++v)
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        float t = p0 == 0 ? 0.f : sum[v][j];
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const uint32_t part = p0 + uint32_t(u);
                            const float val = part == kp ? slot[(v * NJ + j) * kThreads + tid] : pv[u][v][j];
                            t = part == 0 ? val : part < kparts ? t + val : t;
                        }
                        sum[v][j] = t;
                    }
            }
            write_out(int(i), [&](int v, int j) { return late ? __builtin_nanf("") : sum[v][j]; });
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                __hip_atomic_store(reinterpret_cast<float *>(pbase(kp) + poff(i, v, j)), acc[i][j][v],
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // The parts are device-coherent atomic stores (they bypass the XCD-private L2); the
    // wait makes every one of them complete before this workgroup's arrival is counted.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&counters[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_flag = prev == kparts - 1;
    }
    __syncthreads();
    if (!last_flag) return;
    if (tid == 0) __hip_atomic_store(&counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Last arrival: the parts are added in part order (deterministic), four parts of one token
    // sub-tile per round trip (4 x 32 loads per lane, unconditional: a slot past kparts re-reads
    // the last part and is not added).  A loop that loads and adds one value at a time waits for
    // every load (each reuses the register the add just read): at 8 parts that took the Q6_K
    // down at batch 512 from ~100 to ~520 us.  The accumulators are not read here (their index
    // would be a loop variable).
    for (int i = 0; i < MI; ++i) {
        float sum[16][NJ];
        for (uint32_t p0 = 0; p0 < kparts; p0 += 4) {
            float pv[4][16][NJ];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t part = __builtin_elementwise_min(p0 + uint32_t(u), kparts - 1);
#pragma unroll
                for (int v = 0; v < 16; ++v)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        pv[u][v][j] = __hip_atomic_load(reinterpret_cast<float *>(pbase(part) + poff(i, v, j)),
                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
            for (int v = 0; v < 16; ++v)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    float t = p0 == 0 ? pv[0][v][j] : sum[v][j] + pv[0][v][j];
#pragma unroll
                    for (int u = 1; u < 4; ++u) t = p0 + uint32_t(u) < kparts ? t + pv[u][v][j] : t;
                    sum[v][j] = t;
                }
        }
        write_out(i, [&](int v, int j) { return sum[v][j]; });
    }
}

// Workgroups of one instance the device holds at once (one per CU at 128 KiB of LDS), per device.
template <class K>
uint64_t resident_wgs(K kernel) {
    static int cache[64][3] = {};
    int dev = 0;
    (void)hipGetDevice(&dev);
    const int slot = kernel == &gemm_f16_kernel<Q4_K, true> ? 0 : kernel == &gemm_f16_kernel<Q4_K, false> ? 1 : 2;
    int &n = cache[dev & 63][slot];
    if (n == 0) {
        int wgs = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&wgs, kernel, kThreads, 0) != hipSuccess || wgs <= 0 ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            n = -1;  // unknown: never taken as room
        else
            n = wgs * cus;
    }
    return n > 0 ? uint64_t(n) : 0;
}

struct F16Plan {
    uint32_t ntok, ncol, kparts;
};

F16Plan plan_f16(uint32_t cols, uint32_t rows, uint32_t batch, bool pair, const Tuning &t) {
    F16Plan p;
    p.ntok = (batch + TT - 1) / TT;
    const uint32_t rows_per_tile = pair ? TC / 2 : TC;
    p.ncol = (rows + rows_per_tile - 1) / rows_per_tile;
    const uint32_t nb = cols / kQK, tiles = p.ntok * p.ncol;
    p.kparts = 1;
    // one workgroup per CU on 256 CUs: split K until the grid covers most of them
    while (tiles * p.kparts < 200 && p.kparts * 2 <= nb / 4) p.kparts *= 2;
    if (t.gemm_kparts >= 1 && uint32_t(t.gemm_kparts) <= nb) p.kparts = uint32_t(t.gemm_kparts);
    if (uint64_t(pair ? 2 : 1) * p.ntok * TT * p.ncol * rows_per_tile * 4 >= (uint64_t(1) << 32)) p.kparts = 1;
    return p;
}

}  // namespace

void gemm_f16_workspace_need(uint32_t cols, uint32_t rows, uint32_t batch, bool pair, const Tuning &t,
                             size_t *part_floats, size_t *counters) {
    const F16Plan p = plan_f16(cols, rows, batch, pair, t);
    *part_floats = p.kparts > 1 ? size_t(p.kparts) * (pair ? 2 : 1) * (p.ntok * TT) * (p.ncol * (pair ? TC / 2 : TC)) : 0;
    *counters = 2 * size_t(p.ntok) * p.ncol;  // arrivals; and departures of the reduce-scatter
}

hipError_t launch_gemm_f16(int type, const uint8_t *w, const uint8_t *up, const uint16_t *x, void *out, uint32_t cols,
                           uint32_t rows, uint32_t batch, float *partial, uint32_t *counters, uint32_t *err,
                           const Tuning &t, hipStream_t stream) {
    const bool pair = up != nullptr;
    const F16Plan p = plan_f16(cols, rows, batch, pair, t);
    const dim3 grid(p.ntok * p.ncol * p.kparts), block(kThreads);
    const uint32_t wbytes = rows * (cols / kQK) * block_bytes(type);
    // the reduce-scatter needs every part of a tile running at once: the whole grid resident
    const auto kernel = pair ? &gemm_f16_kernel<Q4_K, true>
                             : type == Q4_K ? &gemm_f16_kernel<Q4_K, false> : &gemm_f16_kernel<Q6_K, false>;
    uint32_t rs_spin = 0;
    if (p.kparts > 1 && MI % p.kparts == 0 && t.gemm_rs != 0 && waits_allowed(t) &&
        uint64_t(grid.x) <= resident_wgs(kernel))
        rs_spin = t.gemm_rs > 1 ? uint32_t(t.gemm_rs) : 1u << 22;  // 2^22 polls of s_sleep 2: seconds
    kernel<<<grid, block, 0, stream>>>(w, pair ? up : w, x, out, partial, counters, cols, rows, batch, p.ntok, p.ncol,
                                       p.kparts, wbytes, rs_spin, err);
    return hipGetLastError();
}

}  // namespace ns
