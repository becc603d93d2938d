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
// where sc*q (<= 945) and sc*(v-32) are integers that fp16 represents exactly
// (Q6_K: while |sc| <= 64; the int8 scales of real tensors can need one more bit,
// and those tile values are rounded once, see decode(RawQ6)).  The LDS weight tile therefore holds those integers, the
// MFMA products with fp16 x are exact, and the per-row factors are applied once
// per super-block on the accumulators:
//   Y += d * acc_sb  [- dmin * sum_g m_g * S_g(x)]            (S_g = sum of x over group g)
// The Q4_K min term is two extra MFMAs per super-block whose K runs over the 8
// groups: A = the group sums of x split into fp16 hi + lo (k 0..7 and 8..15),
// B = the min factors, likewise as fp16 hi + lo.  This keeps the FP32 mode at fp32 accuracy (a plain fp16 copy of the
// dequantised weights would add ~1e-3 relative error by itself) and needs fewer
// VALU operations per weight than materialising d*sc*q - dmin*m.  A token whose group
// sums pass fp16's range enters as x * 2^-k (group_sums_kernel, copy_scaled_kernel) and
// its outputs are multiplied by 2^k after the loop.
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
//   FP32  the exact integer tiles above, Y accumulated in fp32.
//   FP16  the reference's fp16 weight tiles with a per-row power-of-two scale
//         (ns_tile16.hpp; no rescale, no min-term MFMAs), Y accumulated in fp32
//         and rounded once to fp16 precision (11 significant bits, fp32 exponent
//         range; metal:394/:489 write a half tile).  True fp16 range would
//         overflow on BASELINE's synthetic inputs (down outputs reach 1.7e5).
//         The CDNA4 layout runs this mode in ns_gemm_f16.hip.
#include <algorithm>
#include <type_traits>

#include "ns_internal.hpp"
#include "ns_quant.hpp"
#include "ns_tile16.hpp"

namespace ns {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int TT = 256;        // tokens per workgroup tile
static_assert(256 % TT == 0, "a token tile lies inside one 256-token block of the rescaled copy");
constexpr int TC = 256;        // B columns per workgroup tile
constexpr int kWaves = 8;      // 2 (tokens) x 4 (columns)
constexpr int kThreads = 64 * kWaves;
constexpr int WT = 128;        // tokens per wave
constexpr int WC = 64;         // B columns per wave
constexpr int MI = WT / 32;    // 32x32 MFMA tiles per wave along tokens
constexpr int NJ = WC / 32;    // ... along columns
constexpr int KS = 64;         // k per step
constexpr int LDSW = KS + 8;   // padded LDS row of the weight tile (halfs)
constexpr int XDMA = TT * KS * 2 / 16 / kThreads;  // 16-byte x chunks each thread moves per step

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

// Two small unsigned fields (selected bytes of w, masked) as fp16 1024+f: one
// v_perm places bytes b_i of w under 0x64 exponent bytes, one AND keeps the field.
__device__ __forceinline__ half2_t magic_pair(uint32_t w, uint32_t sel, uint32_t mask) {
    return h2(__builtin_amdgcn_perm(0x64646464u, w, sel) & mask);
}
constexpr uint32_t kSel01 = 0x04010400u;  // [0x64, b1, 0x64, b0]
constexpr uint32_t kSel23 = 0x04030402u;  // [0x64, b3, 0x64, b2]
constexpr uint32_t kMask4 = 0xFF0FFF0Fu;
constexpr uint32_t kMask6 = 0xFF3FFF3Fu;

// sc*(1024+f) + bias with one rounding; exact because the result is an integer <= 2048.
__device__ __forceinline__ uint32_t scale_pair(half2_t t, half2_t sc, half2_t bias) {
    return u32(__builtin_elementwise_fma(t, sc, bias));
}

// Buffer-resource loads: bounds-checked by the descriptor (reads at or past
// `bytes` return 0), so no per-lane branch guards a load.  A guarded load would
// make the compiler wait for it at once, defeating the prefetch below.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, int(bytes), 0x00020000);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, int(off), 0, 0);
}
__device__ __forceinline__ uint32_t bload2(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, int(off), 0, 0);
}

struct WRun {
    u32x4 v[4];  // v[0..1]: 16 halfs at k offset k_lo, v[2..3]: 16 halfs at k_hi
};

// Raw bytes one producer thread loads for one k step.
struct RawQ4 {
    u32x4 hdr, qs;
};
struct RawQ6 {
    u32x4 ql[2], qh[2], scw;
    uint32_t dbits;
};
template <int TYPE>
using Raw = typename std::conditional<TYPE == Q4_K, RawQ4, RawQ6>::type;

// Q4_K step s covers groups 2p, 2p+1 (p = s%4) of super-block s/4: qs bytes
// 32p..32p+31, low nibble -> group 2p, high -> group 2p+1.  Thread half hh
// takes bytes 32p+16hh..+15: run 0 = group 2p, l = 16hh..+15 (k offset 16hh);
// run 1 = group 2p+1, same l (k offset 32+16hh).
template <int LAYOUT>
__device__ __forceinline__ void load_raw(rsrc_t w, uint32_t row, uint32_t nb, uint32_t s, uint32_t hh, RawQ4 &r) {
    const uint32_t b = s >> 2, p = s & 3;
    if constexpr (LAYOUT == CDNA4) {
        const uint32_t base = uint32_t(region_offset(Q4_K, row / kRowTile, b, nb)) + (row % kRowTile) * 16;
        r.hdr = bload16(w, base);
        r.qs = bload16(w, base + (1 + 2 * p + hh) * kRowTile * 16);
    } else {
        const uint32_t blk = uint32_t(block_index(LAYOUT, row, b, nb)) * kQ4Bytes;
        r.hdr = bload16(w, blk);
        r.qs = bload16(w, blk + (1 + 2 * p + hh) * 16);
    }
}

// Values: sc_g * q, exact in fp16.
// z scales the tile: 1 normally (values exact), 0 for d == 0, d/e < 1 for the
// rare blocks whose d is far below dmin (then rounded; see the kernel comment).
__device__ __forceinline__ void decode(const RawQ4 &r, uint32_t s, uint32_t hh, float z, WRun &out) {
    (void)hh;
    const uint32_t p = s & 3;
    const Q4Scales sc = q4_scales(r.hdr.y, r.hdr.z, r.hdr.w);
    const _Float16 s0 = _Float16(z * float(q4_sc(sc, int(2 * p)))), s1 = _Float16(z * float(q4_sc(sc, int(2 * p + 1))));
    const half2_t sc0 = {s0, s0}, sc1 = {s1, s1};
    const half2_t nb0 = {_Float16(-1024.f) * s0, _Float16(-1024.f) * s0};
    const half2_t nb1 = {_Float16(-1024.f) * s1, _Float16(-1024.f) * s1};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t wv = r.qs[i], wh = wv >> 4;
        out.v[i >> 1][(i & 1) * 2 + 0] = scale_pair(magic_pair(wv, kSel01, kMask4), sc0, nb0);
        out.v[i >> 1][(i & 1) * 2 + 1] = scale_pair(magic_pair(wv, kSel23, kMask4), sc0, nb0);
        out.v[2 + (i >> 1)][(i & 1) * 2 + 0] = scale_pair(magic_pair(wh, kSel01, kMask4), sc1, nb1);
        out.v[2 + (i >> 1)][(i & 1) * 2 + 1] = scale_pair(magic_pair(wh, kSel23, kMask4), sc1, nb1);
    }
}

__device__ __forceinline__ uint32_t k_lo(int type, uint32_t hh) { return type == Q4_K ? 16 * hh : 32 * hh; }
__device__ __forceinline__ uint32_t k_hi(int type, uint32_t hh) { return type == Q4_K ? 32 + 16 * hh : 32 * hh + 16; }

// NSMFFN Q6_K blocks are only 2-byte aligned: assemble a 16-byte chunk from halves.
__device__ __forceinline__ u32x4 load_chunk_q6(rsrc_t w, uint32_t blk, uint32_t chunk) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        v[i] = bload2(w, blk + 16 * chunk + 4 * i) | (bload2(w, blk + 16 * chunk + 4 * i + 2) << 16);
    return v;
}

// Q6_K step s covers elements 64*(s%4)..+63 of super-block s/4: half
// h = (s%4)/2, quarters 2*(s%2) and 2*(s%2)+1.  Thread half hh takes quarter
// qa = 2*(s%2)+hh, l = 0..31 (k offsets 32hh..32hh+31):
//   v = nibble of ql[64h + 32*(qa&1) + l] (low if qa < 2) | (qh[32h + l] >> 2qa & 3) << 4.
template <int LAYOUT>
__device__ __forceinline__ void load_raw(rsrc_t w, uint32_t row, uint32_t nb, uint32_t s, uint32_t hh, RawQ6 &r) {
    const uint32_t b = s >> 2, sr = s & 3, h = sr >> 1, qa = 2 * (sr & 1) + hh;
    const uint32_t cl = 4 * h + 2 * (qa & 1), chh = 8 + 2 * h;
    if constexpr (LAYOUT == CDNA4) {
        const uint32_t reg = uint32_t(region_offset(Q6_K, row / kRowTile, b, nb));
        const uint32_t base = reg + (row % kRowTile) * 16;
        r.ql[0] = bload16(w, base + cl * kRowTile * 16);
        r.ql[1] = bload16(w, base + (cl + 1) * kRowTile * 16);
        r.qh[0] = bload16(w, base + chh * kRowTile * 16);
        r.qh[1] = bload16(w, base + (chh + 1) * kRowTile * 16);
        r.scw = bload16(w, base + 12 * kRowTile * 16);
        r.dbits = bload2(w, reg + kQ6Chunks * 1024 + (row % kRowTile) * 2);
    } else {
        const uint32_t blk = uint32_t(block_index(LAYOUT, row, b, nb)) * kQ6Bytes;
        r.ql[0] = load_chunk_q6(w, blk, cl);
        r.ql[1] = load_chunk_q6(w, blk, cl + 1);
        r.qh[0] = load_chunk_q6(w, blk, chh);
        r.qh[1] = load_chunk_q6(w, blk, chh + 1);
        r.scw = load_chunk_q6(w, blk, 12);
        r.dbits = bload2(w, blk + 208);
    }
}

// Values: sc * (v - 32), sc = scales[8h + 2qa + l/16]: v - 32 exactly (one packed add to the
// fp16 1024 + v), then one rounding of the product.  The product is exact while it fits 11
// significant bits (always for |sc| <= 64, the synthetic generator's -32..31 included); real
// int8 scales (llama.cpp puts one group of every Q6_K block at -128) reach |sc*(v-32)| = 4096,
// where odd products need 12 bits and round (relative error <= 2^-12 on those weights).  The
// single FMA sc*(1024+v) - 1056*sc would need the bias 1056*sc, which is not an fp16 past
// |sc| = 62.
__device__ __forceinline__ void decode(const RawQ6 &r, uint32_t s, uint32_t hh, float z, WRun &out) {
    const uint32_t sr = s & 3, h = sr >> 1, qa = 2 * (sr & 1) + hh;
    const uint32_t si = 8 * h + 2 * qa;
    const uint32_t nshift = qa >= 2 ? 4 : 0, hshift = 2 * qa;
    const half2_t m1056 = {_Float16(-1056.f), _Float16(-1056.f)};
    auto scaled = [&](half2_t t, half2_t sc2) { return u32((t + m1056) * sc2); };
#pragma unroll
    for (int c = 0; c < 2; ++c) {  // l = 16c .. 16c+15
        const _Float16 s16 = _Float16(z * float(int8_t(byte_of(r.scw[(si + c) >> 2], int((si + c) & 3)))));
        const half2_t sc2 = {s16, s16};
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // l = 16c + 4i .. +3
            const uint32_t v = ((r.ql[c][i] >> nshift) & 0x0F0F0F0Fu) | (((r.qh[c][i] >> hshift) & 0x03030303u) << 4);
            out.v[2 * c + (i >> 1)][(i & 1) * 2 + 0] = scaled(magic_pair(v, kSel01, kMask6), sc2);
            out.v[2 * c + (i >> 1)][(i & 1) * 2 + 1] = scaled(magic_pair(v, kSel23, kMask6), sc2);
        }
    }
}

// FP16-mode tiles (ns_tile16.hpp): F = RNE16(q*2^-24*A + B) with the row scale in
// c24 = c * 2^24; same element placement as the exact decode above.
__device__ __forceinline__ void decode_f16(const RawQ4 &r, uint32_t s, float c24, WRun &out) {
    const uint32_t p = s & 3;
    const float d = lo_half(r.hdr.x), dmin = hi_half(r.hdr.x);
    const Q4Scales sc = q4_scales(r.hdr.y, r.hdr.z, r.hdr.w);
    const float dc = d * c24, mc = -dmin * (c24 * 5.9604644775390625e-08f);
    const half2_t Alo = splat(_Float16(dc * float(q4_sc(sc, int(2 * p))))), Ahi = splat(_Float16(dc * float(q4_sc(sc, int(2 * p + 1)))));
    const half2_t Blo = splat(_Float16(mc * float(q4_m(sc, int(2 * p))))), Bhi = splat(_Float16(mc * float(q4_m(sc, int(2 * p + 1)))));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t lo[2], hi[2];
        q4_f16x8(r.qs[i], Alo, Blo, Ahi, Bhi, lo, hi);
        out.v[i >> 1][(i & 1) * 2 + 0] = lo[0];
        out.v[i >> 1][(i & 1) * 2 + 1] = lo[1];
        out.v[2 + (i >> 1)][(i & 1) * 2 + 0] = hi[0];
        out.v[2 + (i >> 1)][(i & 1) * 2 + 1] = hi[1];
    }
}
__device__ __forceinline__ void decode_f16(const RawQ6 &r, uint32_t s, uint32_t hh, float c24, WRun &out) {
    const uint32_t sr = s & 3, h = sr >> 1, qa = 2 * (sr & 1) + hh;
    const uint32_t si = 8 * h + 2 * qa;
    const uint32_t nshift = qa >= 2 ? 4 : 0, hshift = 2 * qa;
    const float d = lo_half(r.dbits);
    const float dc = d * c24, dm = -32.0f * d * (c24 * 5.9604644775390625e-08f);
#pragma unroll
    for (int c = 0; c < 2; ++c) {  // l = 16c .. 16c+15
        const float scf = float(int(int8_t(byte_of(r.scw[(si + c) >> 2], int((si + c) & 3)))));
        const half2_t A = splat(_Float16(dc * scf)), B = splat(_Float16(dm * scf));
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // l = 16c + 4i .. +3
            const uint32_t v = ((r.ql[c][i] >> nshift) & 0x0F0F0F0Fu) | (((r.qh[c][i] >> hshift) & 0x03030303u) << 4);
            uint32_t o[2];
            q6_f16x4(v, A, B, o);
            out.v[2 * c + (i >> 1)][(i & 1) * 2 + 0] = o[0];
            out.v[2 * c + (i >> 1)][(i & 1) * 2 + 1] = o[1];
        }
    }
}

// Running sum in one accumulator.  Within super-block sb the MFMA accumulator
// holds S/e_sb, where S is the running sum of the output and e_sb is a per-row
// factor: e = d for Q6_K; e = max(d, dmin/1024) for Q4_K (e = 1 if that is 0).
// The tile holds z*sc*q with z = d/e, i.e. the exact integers sc*q whenever
// e = d; the rare Q4_K blocks with d < dmin/1024 get z < 1 (rounded in fp16,
// an error on a term at most ~1e-3 of the block's own min term).  The Q4_K
// min term -dmin/e * sum_g m_g S_g(x) is two more MFMAs accumulating into the
// same registers: A = the group sums of x split into fp16 hi (k 0..7) and lo
// (k 8..15); B = b_g = fp16(-dmin/e * m_g) (|.| <= 1024*63) in both halves, then
// the residues fp16(-dmin/e * m_g - b_g) against the hi sums only.  With b_g
// alone the min term carried 11 significant bits, which on blocks with d = 0
// (pure min term) put the gate/up output 1.2e-3 off.  Entering super-block sb+1
// multiplies the accumulator by e_sb / e_sb+1.
//
// Pipeline, per 64-wide k step s (one barrier per step):
//   decode raw(s) into LDS weight buffer s&1 (raw(s) was loaded two steps ago);
//   wait for the LDS-DMA of x(s) (issued one step ago); barrier;
//   issue the LDS-DMA of x(s+1) into x buffer (s+1)&1 and the loads of raw(s+2);
//   MFMAs on buffers s&1.
// Buffers written at step s were last read by MFMAs of step s-2 (weights) or
// s-1 (x), which every wave finished before it passed barrier s-1 or s.
// x rows are unpadded (128 bytes) with 16-byte chunk c of row R stored at
// position c ^ ((R >> 1) & 7), which keeps 16 consecutive rows' fragment reads
// on distinct LDS banks; weight rows are padded to 72 halfs for the same reason.
//
// Split K (gridDim.y > 1): workgroup y covers super-blocks [y*nb/Y, (y+1)*nb/Y);
// each writes its S tile to the workspace, and the last workgroup of a tile to
// arrive (counted with a device-scope atomic) adds the parts in y order and
// runs the epilogue, so results do not depend on arrival order.  The hand-off
// uses device-coherent atomic stores/loads only (no L2-wide fences).
template <int TYPE, int LAYOUT, int ACC, bool PAIR>
__global__ __launch_bounds__(kThreads, 1) void gemm_kernel(
    const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, const uint16_t *__restrict__ x,
    const uint16_t *__restrict__ xsums, void *__restrict__ out, float *__restrict__ partial,
    uint32_t *__restrict__ counters, uint32_t cols, uint32_t rows, uint32_t batch, uint32_t ntok_tiles,
    uint32_t ncol_tiles, uint32_t kparts_total, uint32_t wbytes, uint32_t rs_spin, uint32_t *__restrict__ err) {
    constexpr bool Q4 = TYPE == Q4_K;
    constexpr bool F16 = ACC == ACC_FP16;  // fp16 tiles (ns_tile16.hpp) instead of exact ones
    constexpr uint32_t kRawLoads = Q4 ? 2 : (LAYOUT == CDNA4 ? 6 : 41);  // vector loads per load_raw
    __shared__ __attribute__((aligned(16))) _Float16 Ws[2][TC * LDSW];
    __shared__ __attribute__((aligned(16))) u32x4 Xs[2][TT * 8];
    __shared__ float colE[2][TC];
    __shared__ float colInv[TC];  // FP16 mode: 1/c of each column's row
    // Q4_K min factors per column: 8 fp16 values b_g, then their 8 rounding residues
    __shared__ __attribute__((aligned(16))) _Float16 colB[2][Q4 ? TC * 16 : 16];
    __shared__ uint32_t last_flag, late_flag;

    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wt = wave >> 2, wn = wave & 3;
    // XCD-aware order.  Workgroup L is dispatched to XCD L % 8; the work items are
    // numbered q = (kp * ntok + tt) * ncol + ct (one x slice = fixed (tt, kp) and
    // all its column tiles) and XCD x takes the contiguous run q in
    // [x * W/8, (x+1) * W/8), so each XCD's L2 holds whole x slices and the
    // column tiles that share one are resident together.
    const uint32_t nwg = gridDim.x, w8 = nwg / 8, L = blockIdx.x;
    const uint32_t q = L < 8 * w8 ? (L % 8) * w8 + L / 8 : L;
    const uint32_t ncol = ncol_tiles, kparts = kparts_total;
    const uint32_t ct = q % ncol, g = q / ncol, tt = g % ntok_tiles, kp = g / ntok_tiles;
    const uint32_t tile = tt + ntok_tiles * ct;  // counter slot of the output tile
    const uint32_t t0 = tt * TT;
    constexpr uint32_t kRowsPerTile = PAIR ? TC / 2 : TC;
    const uint32_t r0 = ct * kRowsPerTile;
    const uint32_t nb = cols / kQK, ngroups = cols / 32;
    const uint32_t sb0 = kp * nb / kparts, sb1 = (kp + 1) * nb / kparts;

    // producer role: column wc of the tile, k half hh (waves 0-3: hh 0, waves 4-7: hh 1)
    const uint32_t wc = tid & (TC - 1), hh = tid / TC;
    // PAIR: gate columns 0..127 come from waves with (wave & 3) < 2: wave-uniform
    const rsrc_t wsrc = make_rsrc((PAIR && (wave & 3) >= 2) ? w1 : w0, wbytes);
    const uint32_t wrow = r0 + (PAIR ? (wc % (TC / 2)) : wc);
    // x group sums: plane hi [batch][ngroups] then plane lo; rows past batch are
    // never stored, so their (lo-plane) contents do not matter
    const rsrc_t xssrc = make_rsrc(xsums, (Q4 && !F16) ? 2 * batch * ngroups * 2 : 0);
    // Q4_K FP32 mode: a tile in a 256-token block with a rescaled token reads x from the
    // rescaled copy, which holds every row of that block, and multiplies its tokens'
    // outputs back by their factor (TT divides 256)
    const float *xsb = reinterpret_cast<const float *>(xsums);
    const XsLayout xl = xs_layout(cols, batch);
    uint32_t tile_scaled = 0;  // one uniform load
    if constexpr (Q4 && !F16)
        tile_scaled = __builtin_amdgcn_readfirstlane(reinterpret_cast<const uint32_t *>(xsb + xl.bflag)[t0 / 256]);
    const rsrc_t xsrc = make_rsrc(tile_scaled ? static_cast<const void *>(xsb + xl.xcopy) : x, batch * cols * 2);

    float16_t acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    auto bcol = [&](int j) -> uint32_t {
        if constexpr (PAIR) return uint32_t(j) * (TC / 2) + wn * 32;  // gate / up of the same 32 rows
        else return wn * WC + uint32_t(j) * 32;
    };
    // x(s) -> Xs[buf] by LDS DMA: instruction i of wave w fills rows 8*(w + 8i) .. +7;
    // lane L writes LDS chunk L of that 1 KiB block, i.e. row +L/8, position L%8,
    // so it fetches global chunk (L%8) ^ swizzle(row).  Rows past batch read 0.
    auto dma_x = [&](uint32_t s, uint32_t buf) {
#pragma unroll
        for (int i = 0; i < XDMA; ++i) {
            const uint32_t rbase = 8 * (wave + kWaves * uint32_t(i));
            const uint32_t R = rbase + (lane >> 3), c = (lane & 7) ^ ((R >> 1) & 7);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xsrc, (__attribute__((address_space(3))) void *)(&Xs[buf][rbase * 8]), 16,
                ((t0 + R) * cols + s * KS + 8 * c) * 2, 0, 0, 0);
        }
    };
    auto load_w = [&](uint32_t s, Raw<TYPE> &raw) { load_raw<LAYOUT>(wsrc, wrow, nb, s, hh, raw); };

    Raw<TYPE> raw[2] = {};
    u32x4 xsf[MI] = {};  // Q4_K: group sums of x for this super-block (hi in lanes 0-31, lo in 32-63)

    // FP16 mode: the row scale of this producer's column (rows past `rows` read zeros: c = 1)
    float c24 = 0.f;
    if constexpr (F16) {
        float M = 0.f;
        for (uint32_t b = 0; b < nb; ++b) {
            if constexpr (Q4) {
                const uint32_t off = uint32_t(byte_offset(TYPE, LAYOUT, wrow, b, nb, 0));
                const uint32_t dd = bload2(wsrc, off) | (bload2(wsrc, off + 2) << 16);
                M = __builtin_fmaxf(M, __builtin_fmaxf(__builtin_fabsf(lo_half(dd)), __builtin_fabsf(hi_half(dd))));
            } else {
                M = __builtin_fmaxf(M, __builtin_fabsf(lo_half(bload2(wsrc, uint32_t(byte_offset(TYPE, LAYOUT, wrow, b, nb, 208))))));
            }
        }
        float inv_c;
        row_scale(M, c24, inv_c, TYPE == Q6_K);
        if (hh == 0) colInv[wc] = inv_c;
    }

    // Decode raw weights of step s into weight buffer s&1 (and, on the first step
    // of a super-block, its per-row factors).
    auto produce = [&](uint32_t s, const Raw<TYPE> &rw) {
        const uint32_t buf = s & 1, pb = ((s >> 2) - sb0) & 1;
        float d, e;
        if constexpr (Q4) {
            d = lo_half(rw.hdr.x);
            e = __builtin_fmaxf(d, hi_half(rw.hdr.x) * 0.0009765625f);
            e = e > 0.f ? e : 1.f;
        } else {
            d = lo_half(rw.dbits);
            e = d != 0.f ? d : 1.f;
        }
        const float re = __builtin_amdgcn_rcpf(e);  // ~1 ulp; exactness is kept by z = 1 when e == d
        const float z = d == e ? 1.f : d * re;
        WRun wr;
        if constexpr (F16) {
            if constexpr (Q4) decode_f16(rw, s, c24, wr);
            else decode_f16(rw, s, hh, c24, wr);
        } else {
            decode(rw, s, hh, z, wr);
        }
        _Float16 *wl = &Ws[buf][wc * LDSW];
        *reinterpret_cast<u32x4 *>(wl + k_lo(TYPE, hh)) = wr.v[0];
        *reinterpret_cast<u32x4 *>(wl + k_lo(TYPE, hh) + 8) = wr.v[1];
        *reinterpret_cast<u32x4 *>(wl + k_hi(TYPE, hh)) = wr.v[2];
        *reinterpret_cast<u32x4 *>(wl + k_hi(TYPE, hh) + 8) = wr.v[3];
        if (!F16 && (s & 3) == 0 && hh == 0) {
            colE[pb][wc] = e;
            if constexpr (Q4) {
                const float f = -hi_half(rw.hdr.x) * re;
                const Q4Scales sc = q4_scales(rw.hdr.y, rw.hdr.z, rw.hdr.w);
                half8_t bh, bl;
#pragma unroll
                for (int g = 0; g < 8; ++g) {
                    const float v = f * float(q4_m(sc, g));
                    bh[g] = _Float16(v);
                    bl[g] = _Float16(v - float(bh[g]));
                }
                *reinterpret_cast<half8_t *>(&colB[pb][wc * 16]) = bh;
                *reinterpret_cast<half8_t *>(&colB[pb][wc * 16 + 8]) = bl;
            }
        }
    };
    // The x DMA of the next step is issued before the next raw loads: wait for
    // it but let those raw loads stay in flight.
    auto wait_x = [&]() {
        __builtin_amdgcn_s_waitcnt(int((kRawLoads & 15) | ((kRawLoads >> 4) << 14) | (7 << 4) | (15 << 8)));
    };

    // prologue: step sbeg ready in LDS, raw(sbeg+1) in flight
    const uint32_t sbeg = 4 * sb0;
    load_w(sbeg, raw[0]);
    dma_x(sbeg, 0);
    load_w(sbeg + 1, raw[1]);
    produce(sbeg, raw[0]);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // Step s: issue x(s+1) -> Xs[buf^1] and raw(s+2); MFMAs of s on buffers buf,
    // with the decode of raw(s+1) into Ws[buf^1] placed among them so the VALU
    // work runs in the MFMA shadow; then wait for x(s+1) and meet at the barrier.
    // Buffers buf^1 were last read by MFMAs of step s-1, finished before barrier s.
    for (uint32_t sb = sb0; sb < sb1; ++sb) {
        const uint32_t pb = (sb - sb0) & 1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t s = 4 * sb + uint32_t(j), buf = uint32_t(j) & 1;
            const bool more = s + 1 < 4 * sb1;
            if constexpr (Q4 && !F16) {
                if (j == 0) {
#pragma unroll
                    for (int i = 0; i < MI; ++i)
                        xsf[i] = bload16(xssrc, ((lane >> 5) * batch * ngroups +
                                                 (t0 + wt * WT + i * 32 + (lane & 31)) * ngroups + 8 * sb) * 2);
                }
            }
            if (more) dma_x(s + 1, buf ^ 1);
            load_w(s + 2, raw[j & 1]);  // slot of raw(s), decoded during step s-1

            if (!F16 && j == 0 && sb > sb0) {  // enter super-block sb: S/e_prev -> S/e_sb
#pragma unroll
                for (int jj = 0; jj < NJ; ++jj) {
                    const uint32_t c = bcol(jj) + (lane & 31);
                    const float e_prev = colE[pb ^ 1][c], e_cur = colE[pb][c];
                    const float rinv = __builtin_amdgcn_rcpf(e_cur), r = e_prev * rinv;
#pragma unroll
                    for (int i = 0; i < MI; ++i)
#pragma unroll
                        for (int v = 0; v < 16; ++v) {
                            acc[i][jj][v] *= r;
                        }
                }
            }

            // ---- MFMAs of step s over 4 k16 sub-steps, decode of step s+1 in between.
            // Fragments of sub-step kk+1 are read from LDS while kk's MFMAs run.
            half8_t a[2][MI], b[2][NJ];
            auto frags = [&](int kk, half8_t (&fa)[MI], half8_t (&fb)[NJ]) {
                const uint32_t koff = 16 * kk + 8 * (lane >> 5);
#pragma unroll
                for (int jj = 0; jj < NJ; ++jj)
                    fb[jj] = *reinterpret_cast<const half8_t *>(&Ws[buf][(bcol(jj) + (lane & 31)) * LDSW + koff]);
#pragma unroll
                for (int i = 0; i < MI; ++i) {
                    const uint32_t R = wt * WT + i * 32 + (lane & 31);
                    const uint32_t c = 2 * kk + (lane >> 5);
                    fa[i] = __builtin_bit_cast(half8_t, Xs[buf][R * 8 + (c ^ ((R >> 1) & 7))]);
                }
            };
            frags(0, a[0], b[0]);
#pragma unroll
            for (int kk = 0; kk < KS / 16; ++kk) {
                if (kk + 1 < KS / 16) frags(kk + 1, a[(kk + 1) & 1], b[(kk + 1) & 1]);
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int jj = 0; jj < NJ; ++jj)
                        acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[kk & 1][i], b[kk & 1][jj], acc[i][jj], 0, 0, 0);
                if (kk == 1 && more) produce(s + 1, raw[(j + 1) & 1]);
            }

            if constexpr (Q4 && !F16) {
                if (j == 3) {  // min term of super-block sb
                    // b_g in k 0-7 (hi sums) and k 8-15 (lo sums); the residues of b_g in k 0-7
                    // only (against the hi sums), so the min term keeps ~22 significant bits
#pragma unroll
                    for (int jj = 0; jj < NJ; ++jj) {
                        const _Float16 *cb = &colB[pb][(bcol(jj) + (lane & 31)) * 16];
                        const half8_t bm = *reinterpret_cast<const half8_t *>(cb);
                        half8_t bl = *reinterpret_cast<const half8_t *>(cb + 8);
                        if (lane >= 32) bl = half8_t{};
#pragma unroll
                        for (int i = 0; i < MI; ++i)
                            acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                                __builtin_bit_cast(half8_t, xsf[i]), bl,
                                __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, xsf[i]), bm,
                                                                       acc[i][jj], 0, 0, 0),
                                0, 0, 0);
                    }
                }
            }
            wait_x();
            __syncthreads();
        }
    }

    // ---- S = acc * e_last.  32x32 D layout: lane holds column lane%32 and
    // rows 8*(v/4) + 4*(lane/32) + v%4 for v = 0..15.
    const uint32_t pl = (sb1 - 1 - sb0) & 1;
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
        // FP16 mode: the tiles carry the row scale c, so S = acc / c
        const float el = F16 ? colInv[bcol(jj) + (lane & 31)] : colE[pl][bcol(jj) + (lane & 31)];
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][jj][v] *= el;
    }
    auto tok_of = [&](int i, int v) -> uint32_t {
        return t0 + wt * WT + uint32_t(i) * 32 + 8 * uint32_t(v >> 2) + 4 * (lane >> 5) + uint32_t(v & 3);
    };
    // rescaled tokens: times 2^k_t, exact in fp32, so also before the split-K parts are added
    if (tile_scaled) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const uint32_t t = tok_of(i, v);
                const float tf = t < batch ? xsb[xl.tfac + t] : 1.f;
#pragma unroll
                for (int jj = 0; jj < NJ; ++jj) acc[i][jj][v] *= tf;
            }
    }
    auto col_row = [&](int jj) -> uint32_t {  // weight row of B fragment jj
        if constexpr (PAIR) return r0 + wn * 32 + (lane & 31);
        else return r0 + bcol(jj) + (lane & 31);
    };

    // Outputs of token sub-tile i: fp16 GeGLU (PAIR) or fp32 per column, from
    // val(v, jj) = the value of accumulator element v of column fragment jj.
    auto write_out = [&](int i, auto val) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const uint32_t t = tok_of(i, v);
            if (t >= batch) continue;
            if constexpr (PAIR) {
                const uint32_t r = col_row(0);
                if (r < rows)
                    reinterpret_cast<_Float16 *>(out)[size_t(t) * rows + r] = _Float16(gelu_tanh(val(v, 0)) * val(v, 1));
            } else {
#pragma unroll
                for (int jj = 0; jj < NJ; ++jj) {
                    const uint32_t r = col_row(jj);
                    if (r < rows) reinterpret_cast<float *>(out)[size_t(t) * rows + r] = val(v, jj);
                }
            }
        }
    };

    // FP16 mode rounds the finished sum once: here, or after the split-K parts are added
    if (kparts == 1) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
            write_out(i, [&](int v, int jj) { return ACC == ACC_FP16 ? round_f16p(acc[i][jj][v]) : acc[i][jj][v]; });
        return;
    }

    // ---- split K.  Parts [kp][plane][ntok*TT][ncol*rows per tile] (PAIR: gate, up):
    // padded to whole tiles, so every position of a tile has a slot and no part
    // store or load needs a guard.  One part is under 4 GiB (checked by the host
    // plan), so a slot is a 32-bit byte offset from the part's (uniform) base.
    constexpr uint32_t kPlanes = PAIR ? 2 : 1;
    const uint32_t tpad = ntok_tiles * TT, rpad = ncol_tiles * kRowsPerTile;
    const size_t pstride = size_t(kPlanes) * tpad * rpad;  // floats per part
    // Slot of (part, plane, token tok_of(i, v), column): the part's wave-uniform
    // base plus a 32-bit byte offset (lane_off holds the lane's plane, token and
    // column terms).
    const uint32_t rstride = rpad * 4u;
    uint32_t lane_off[NJ];
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj)
        lane_off[jj] = ((PAIR ? uint32_t(jj) : 0u) * tpad + t0 + wt * WT + 4 * (lane >> 5)) * rstride + col_row(jj) * 4u;
    // byte offset of (token sub-tile i, element v, fragment jj) within one part,
    // given the lane terms lo
    auto poff = [&](const uint32_t (&lo)[NJ], int i, int v, int jj) -> uint32_t {
        return (uint32_t(i) * 32 + 8 * uint32_t(v >> 2) + uint32_t(v & 3)) * rstride + lo[jj];
    };
    auto pbase = [&](uint32_t part) -> char * { return reinterpret_cast<char *>(partial + part * pstride); };  // uniform
    if (rs_spin != 0) {
        // Reduce-scatter (launched only when the whole grid fits on the device at once, so the
        // kparts workgroups of a tile run together; kparts divides MI): part kp owns token
        // sub-tiles [own_lo, own_hi) of every wave.  Each part stores the sub-tiles it does not
        // own, parks its own in LDS (slot 0 in the x tiles, slot 1 in the weight tiles, both
        // free after the main loop), counts one arrival on written[tile] once its stores are
        // acknowledged, waits until every part has, then adds the parts of its own sub-tiles in
        // part order (its own from LDS) and writes them.  The wait is bounded: a part whose limit
        // runs out writes its sub-tiles as NaN.  The last part past the wait clears both counters.
        const uint32_t ntiles = ntok_tiles * ncol_tiles;
        uint32_t *written = counters + tile, *departed = counters + ntiles + tile;
        const uint32_t own_lo = kp * MI / kparts, own_hi = (kp + 1) * MI / kparts;
        auto slot_of = [&](uint32_t k) -> float * {
            return k == 0 ? reinterpret_cast<float *>(&Xs[0][0]) : reinterpret_cast<float *>(&Ws[0][0]);
        };
        __syncthreads();  // every wave is past its last read of the tiles
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            if (uint32_t(i) >= own_lo && uint32_t(i) < own_hi) {
                float *slot = slot_of(uint32_t(i) - own_lo);
#pragma unroll
                for (int v = 0; v < 16; ++v)
#pragma unroll
                    for (int jj = 0; jj < NJ; ++jj) slot[(v * NJ + jj) * kThreads + tid] = acc[i][jj][v];
            } else {
#pragma unroll
                for (int v = 0; v < 16; ++v)
#pragma unroll
                    for (int jj = 0; jj < NJ; ++jj)
                        __hip_atomic_store(reinterpret_cast<float *>(pbase(kp) + poff(lane_off, i, v, jj)),
                                           acc[i][jj][v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
            const float *slot = slot_of(i - own_lo);
            float sum[16][NJ];
            for (uint32_t p0 = 0; p0 < kparts; p0 += 2) {  // two parts per round trip
                float pv[2][16][NJ];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    // this part's own slot holds no value for these sub-tiles: read from LDS below
                    const uint32_t part = __builtin_elementwise_min(p0 + uint32_t(u), kparts - 1);
                    uint32_t lo[NJ];  // recomputed per round trip, not kept live (see the last arrival)
#pragma unroll
                    for (int jj = 0; jj < NJ; ++jj) {
                        lo[jj] = lane_off[jj];
                        asm volatile("" : "+v"(lo[jj]));
                    }
#pragma unroll
                    for (int v = 0; v < 16; ++v)
#pragma unroll
                        for (int jj = 0; jj < NJ; ++jj)
                            pv[u][v][jj] = __hip_atomic_load(reinterpret_cast<float *>(pbase(part) + poff(lo, int(i), v, jj)),
                                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
#pragma unroll
                for (int v = 0; v < 16; ++v)
#pragma unroll
                    for (int jj = 0; jj < NJ; ++jj) {
                        float t = sum[v][jj];
#pragma unroll
                        for (int u = 0; u < 2; ++u) {
                            const uint32_t part = p0 + uint32_t(u);
                            const float val = part == kp ? slot[(v * NJ + jj) * kThreads + tid] : pv[u][v][jj];
                            // the last arrival's order: (0 + part 0) + part 1 + ...
                            t = part < kparts ? (part == 0 ? 0.f : t) + val : t;
                        }
                        sum[v][jj] = t;
                    }
            }
            write_out(int(i), [&](int v, int jj) {
                const float r = ACC == ACC_FP16 ? round_f16p(sum[v][jj]) : sum[v][jj];
                return late ? __builtin_nanf("") : r;
            });
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
#pragma unroll
            for (int jj = 0; jj < NJ; ++jj) {
                __hip_atomic_store(reinterpret_cast<float *>(pbase(kp) + poff(lane_off, i, v, jj)), acc[i][jj][v],
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();  // every wave's parts are stored
    if (tid == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&counters[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_flag = prev == kparts - 1;
    }
    __syncthreads();
    if (!last_flag) return;
    if (tid == 0) __hip_atomic_store(&counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Last arrival: the parts are added in part order (deterministic).  One round
    // trip loads one part of two token sub-tiles (64 values per lane, all in flight
    // before any is added); the two sub-tiles are then written out.
#pragma unroll
    for (int i0 = 0; i0 < MI; i0 += 2) {
        float sum[2][16][NJ];
        for (uint32_t part = 0; part < kparts; ++part) {
            // the lane terms pass through an empty asm, so the compiler recomputes
            // the 64 offsets in each iteration instead of keeping them all live
            uint32_t lo[NJ];
#pragma unroll
            for (int jj = 0; jj < NJ; ++jj) {
                lo[jj] = lane_off[jj];
                asm volatile("" : "+v"(lo[jj]));
            }
            float pv[2][16][NJ];
#pragma unroll
            for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                for (int v = 0; v < 16; ++v)
#pragma unroll
                    for (int jj = 0; jj < NJ; ++jj)
                        pv[ii][v][jj] = __hip_atomic_load(reinterpret_cast<float *>(pbase(part) + poff(lo, i0 + ii, v, jj)),
                                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                for (int v = 0; v < 16; ++v)
#pragma unroll
                    for (int jj = 0; jj < NJ; ++jj)
                        sum[ii][v][jj] = (part == 0 ? 0.f : sum[ii][v][jj]) + pv[ii][v][jj];
        }
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
            write_out(i0 + ii, [&](int v, int jj) { return ACC == ACC_FP16 ? round_f16p(sum[ii][v][jj]) : sum[ii][v][jj]; });
    }
}

// Group sums of x for the Q4_K min term (the XsLayout block): one workgroup per 8
// tokens, one wave per token.  s = sum of 32 fp16 values in fp32, stored as
// hi = fp16(s) and lo = fp16(s - hi) (together ~22 significant bits).  A token whose
// largest |s| exceeds 65504 (fp16's largest finite value) gets the smallest k_t with
// max |s| * 2^-k_t <= 65504, and its sums are taken again over fp16(x * 2^-k_t), the
// values copy_scaled_kernel writes for it, so the GEMM's x tile and its min term see
// the same operands.  Finite x needs k_t <= 6.
__global__ __launch_bounds__(512) void group_sums_kernel(const uint16_t *__restrict__ x, uint32_t cols,
                                                         uint32_t batch, float *__restrict__ xs) {
    __shared__ uint32_t kshift[8];
    const XsLayout L = xs_layout(cols, batch);
    const uint32_t ng = cols / 32, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t t = blockIdx.x * 8 + w;
    const bool live = t < batch;
    uint16_t *hi = reinterpret_cast<uint16_t *>(xs + L.sums), *lo = hi + size_t(batch) * ng;
    const uint16_t *row = x + size_t(t) * cols;
    auto sum32 = [&](uint32_t g, _Float16 f) {
        const half8_t *p = reinterpret_cast<const half8_t *>(row + size_t(g) * 32);
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const half8_t v = p[i] * f;  // f = 2^-k: exact but for fp16 subnormal results
#pragma unroll
            for (int e = 0; e < 8; ++e) s += float(v[e]);
        }
        return s;
    };
    auto put = [&](uint32_t g, float s) {
        const _Float16 h = _Float16(s);
        hi[size_t(t) * ng + g] = __builtin_bit_cast(uint16_t, h);
        lo[size_t(t) * ng + g] = __builtin_bit_cast(uint16_t, _Float16(s - float(h)));
    };
    float mx = 0.f;
    if (live)
        for (uint32_t g = lane; g < ng; g += 64) {
            const float s = sum32(g, _Float16(1.0f));
            put(g, s);
            mx = __builtin_fmaxf(mx, __builtin_fabsf(s));
        }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = __builtin_fmaxf(mx, __shfl_xor(mx, o));
    uint32_t k = 0;
    while (mx > 65504.f && k < 6) {  // finite x: |s| <= 32 * 65504 < 65504 * 2^5
        mx *= 0.5f;
        ++k;
    }
    if (lane == 0) kshift[w] = k;
    __syncthreads();
    uint32_t any = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) any |= kshift[i];
    if (threadIdx.x == 0) reinterpret_cast<uint32_t *>(xs + L.gflag)[blockIdx.x] = any != 0;
    if (!live) return;
    if (lane == 0) xs[L.tfac + t] = float(1u << k);
    if (k != 0) {
        const _Float16 f = _Float16(1.0f / float(1u << k));
        for (uint32_t g = lane; g < ng; g += 64) put(g, sum32(g, f));
    }
}

// The rescaled copy of x: every token of a 256-token block (the GEMM token tiles lie
// inside such blocks) with any flagged 8-row group is copied as fp16(x * 2^-k_t), so a
// GEMM tile with a rescaled token reads all its rows from xcopy; the block's flag goes to
// bflag, the one word a GEMM workgroup reads.  One workgroup per 8 tokens; blocks without
// a flag return at once.
__global__ __launch_bounds__(512) void copy_scaled_kernel(const uint16_t *__restrict__ x, uint32_t cols,
                                                          uint32_t batch, float *__restrict__ xs) {
    const XsLayout L = xs_layout(cols, batch);
    const uint32_t *gflag = reinterpret_cast<const uint32_t *>(xs + L.gflag);
    const uint32_t ng8 = (batch + 7) / 8, b0 = blockIdx.x / 32 * 32;
    const uint32_t t = blockIdx.x * 8 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const uint32_t gi = b0 + (lane & 31);  // lanes 32-63 repeat lanes 0-31
    const bool any = __ballot(gi < ng8 && gflag[gi] != 0) != 0;
    if (blockIdx.x % 32 == 0 && threadIdx.x == 0) reinterpret_cast<uint32_t *>(xs + L.bflag)[blockIdx.x / 32] = any;
    if (!any || t >= batch) return;
    const _Float16 f = _Float16(1.0f / xs[L.tfac + t]);
    const half8_t *src = reinterpret_cast<const half8_t *>(x + size_t(t) * cols);
    half8_t *dst = reinterpret_cast<half8_t *>(reinterpret_cast<uint16_t *>(xs + L.xcopy) + size_t(t) * cols);
    for (uint32_t c = lane; c < cols / 8; c += 64) dst[c] = src[c] * f;
}

struct GemmPlan {
    uint32_t ntok, ncol, kparts;
};

// Output tiles and split of K: enough workgroups to cover most of the 256 CUs
// (the 3840-row down projection has only 4 x 15 tiles at batch 1024).
GemmPlan plan_gemm(uint32_t cols, uint32_t rows, uint32_t batch, bool pair, const Tuning &t) {
    GemmPlan p;
    p.ntok = (batch + TT - 1) / TT;
    const uint32_t rows_per_tile = pair ? TC / 2 : TC;
    p.ncol = (rows + rows_per_tile - 1) / rows_per_tile;
    const uint32_t nb = cols / kQK, tiles = p.ntok * p.ncol;
    p.kparts = 1;
    while (tiles * p.kparts < 200 && p.kparts * 2 <= nb / 4) p.kparts *= 2;
    if (t.gemm_kparts >= 1 && uint32_t(t.gemm_kparts) <= nb) p.kparts = uint32_t(t.gemm_kparts);
    // one split-K part (padded to whole tiles) must stay under 4 GiB: 32-bit offsets in the kernel
    if (uint64_t(pair ? 2 : 1) * p.ntok * TT * p.ncol * rows_per_tile * 4 >= (uint64_t(1) << 32)) p.kparts = 1;
    return p;
}

// Workgroups of one instance the device holds at once, per device and instance.
template <class K>
uint64_t resident_wgs(K kernel) {
    struct Entry {
        const void *k;
        int dev, n;
    };
    static Entry cache[64] = {};
    int dev = 0;
    (void)hipGetDevice(&dev);
    const void *key = reinterpret_cast<const void *>(kernel);
    for (Entry &e : cache)
        if (e.k == key && e.dev == dev) return e.n > 0 ? uint64_t(e.n) : 0;
    int wgs = 0, cus = 0, n = -1;  // unknown: never taken as room
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&wgs, kernel, kThreads, 0) == hipSuccess && wgs > 0 &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0)
        n = wgs * cus;
    for (Entry &e : cache)
        if (e.k == nullptr) {
            e = Entry{key, dev, n};
            break;
        }
    return n > 0 ? uint64_t(n) : 0;
}

template <int TYPE, int LAYOUT, bool PAIR>
hipError_t launch_mode(int acc, const uint8_t *w, const uint8_t *up, const uint16_t *x, const uint16_t *xh,
                       void *out, uint32_t cols, uint32_t rows, uint32_t batch, const Workspace &ws,
                       size_t ws_offset, hipStream_t stream) {
    const GemmPlan p = plan_gemm(cols, rows, batch, PAIR, ws.tune);
    const dim3 grid(p.ntok * p.ncol * p.kparts), block(kThreads);
    const uint32_t wbytes = rows * (cols / kQK) * block_bytes(TYPE);
    float *partial = ws.partial + ws_offset;
    // the FP16 mode on the CDNA4 layout runs ns_gemm_f16.hip: no FP16 instance is built for it
    constexpr bool kHasFp16 = LAYOUT != CDNA4;
    if (!kHasFp16 && acc == ACC_FP16) return hipErrorInvalidValue;
    const auto kernel = acc == ACC_FP16 ? &gemm_kernel<TYPE, LAYOUT, kHasFp16 ? ACC_FP16 : ACC_FP32, PAIR>
                                        : &gemm_kernel<TYPE, LAYOUT, ACC_FP32, PAIR>;
    // the reduce-scatter needs every part of a tile running at once: the whole grid resident
    uint32_t rs_spin = 0;
    if (p.kparts > 1 && MI % p.kparts == 0 && ws.tune.gemm_rs != 0 && waits_allowed(ws.tune) &&
        uint64_t(grid.x) <= resident_wgs(kernel))
        rs_spin = ws.tune.gemm_rs > 1 ? uint32_t(ws.tune.gemm_rs) : 1u << 22;  // 2^22 polls of s_sleep 2: seconds
    kernel<<<grid, block, 0, stream>>>(w, up, x, xh, out, partial, ws.counters, cols, rows, batch, p.ntok, p.ncol,
                                       p.kparts, wbytes, rs_spin, ws.err);
    return hipGetLastError();
}

template <int TYPE, bool PAIR>
hipError_t launch_layout(int layout, int acc, const uint8_t *w, const uint8_t *up, const uint16_t *x,
                         const uint16_t *xh, void *out, uint32_t cols, uint32_t rows, uint32_t batch,
                         const Workspace &ws, size_t ws_offset, hipStream_t stream) {
    if (layout == CDNA4)
        return launch_mode<TYPE, CDNA4, PAIR>(acc, w, up, x, xh, out, cols, rows, batch, ws, ws_offset, stream);
    if (layout == NSMFFN)
        return launch_mode<TYPE, NSMFFN, PAIR>(acc, w, up, x, xh, out, cols, rows, batch, ws, ws_offset, stream);
    return launch_mode<TYPE, ROW_MAJOR, PAIR>(acc, w, up, x, xh, out, cols, rows, batch, ws, ws_offset, stream);
}

}  // namespace

// Workspace layout: [Q4_K: the XsLayout block (group sums of x, token factors, the
// rescaled copy of x)] [split-K parts: kparts x planes x tokens x rows, both padded to
// whole tiles].
static size_t xs_floats(int type, uint32_t cols, uint32_t batch) {
    return type == Q4_K ? xs_layout(cols, batch).total : 0;
}

static void gemm_fp32_workspace_need(int type, int layout, uint32_t cols, uint32_t rows, uint32_t batch, bool pair,
                                     const Tuning &t, size_t *floats, size_t *counters);

// Q4_K on the CDNA4 layout runs the register-fragment kernel (ns_gemm_reg.hip)
// unless Tuning::gemm_q4_reg = 0 selects the LDS-tile kernel here.
static bool use_gemm_reg(int type, int layout, const Tuning &t) {
    return layout == CDNA4 && type == Q4_K && t.gemm_q4_reg != 0;
}

void gemm_workspace_need(int type, int layout, uint32_t cols, uint32_t rows, uint32_t batch, bool pair,
                         const Tuning &t, size_t *floats, size_t *counters) {
    // FP16 mode on CDNA4 runs ns_gemm_f16.hip; the need covers both modes
    size_t f16_floats = 0, f16_counters = 0;
    if (layout == CDNA4) gemm_f16_workspace_need(cols, rows, batch, pair, t, &f16_floats, &f16_counters);
    size_t f32_floats = 0, f32_counters = 0;
    gemm_fp32_workspace_need(type, layout, cols, rows, batch, pair, t, &f32_floats, &f32_counters);
    *floats = std::max(f16_floats, f32_floats);
    *counters = std::max(f16_counters, f32_counters);
}

static void gemm_fp32_workspace_need(int type, int layout, uint32_t cols, uint32_t rows, uint32_t batch, bool pair,
                                     const Tuning &t, size_t *floats, size_t *counters) {
    if (use_gemm_reg(type, layout, t)) {
        size_t part = 0;
        gemm_reg_workspace_need(cols, rows, batch, pair, t, &part, counters);
        *floats = xs_floats(type, cols, batch) + part;
        return;
    }
    const GemmPlan p = plan_gemm(cols, rows, batch, pair, t);
    *floats = xs_floats(type, cols, batch) +
              (p.kparts > 1 ? size_t(p.kparts) * (pair ? 2 : 1) * (p.ntok * TT) * (p.ncol * (pair ? TC / 2 : TC)) : 0);
    *counters = 2 * size_t(p.ntok) * p.ncol;  // arrivals; and departures of the reduce-scatter
}

hipError_t launch_gemm(int type, int layout, int acc, const uint8_t *w, const uint8_t *up, const uint16_t *x,
                       void *out, uint32_t cols, uint32_t rows, uint32_t batch, const Workspace &ws,
                       hipStream_t stream) {
    if (layout == CDNA4 && acc == ACC_FP16)
        return launch_gemm_f16(type, w, up, x, out, cols, rows, batch, ws.partial, ws.counters, ws.err, ws.tune,
                               stream);
    uint16_t *xh = nullptr;
    if (type == Q4_K && acc == ACC_FP32) {  // the exact tiles' min term needs the group sums of x
        xh = reinterpret_cast<uint16_t *>(ws.partial);
        group_sums_kernel<<<dim3((batch + 7) / 8), dim3(512), 0, stream>>>(x, cols, batch, ws.partial);
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
        copy_scaled_kernel<<<dim3((batch + 7) / 8), dim3(512), 0, stream>>>(x, cols, batch, ws.partial);
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    }
    const size_t off = xs_floats(type, cols, batch);
    if (use_gemm_reg(type, layout, ws.tune))  // CDNA4 and FP32 mode: the FP16 mode returned above
        return launch_gemm_reg(w, up, x, xh, out, cols, rows, batch, ws.partial + off, ws.counters, ws.err, ws.tune,
                               stream);
    if (up) return launch_layout<Q4_K, true>(layout, acc, w, up, x, xh, out, cols, rows, batch, ws, off, stream);
    if (type == Q4_K)
        return launch_layout<Q4_K, false>(layout, acc, w, nullptr, x, xh, out, cols, rows, batch, ws, off, stream);
    return launch_layout<Q6_K, false>(layout, acc, w, nullptr, x, xh, out, cols, rows, batch, ws, off, stream);
}

}  // namespace ns
