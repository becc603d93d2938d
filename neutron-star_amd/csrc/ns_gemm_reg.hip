// ns_gemm_reg.hip -- prefill Q4_K GEMM with register-resident weight fragments
// (CDNA4 layout), for gfx950.
//
// Replaces, for the Q4_K tensors of the .nsmffn path, the reference's
//   gemma_q4k_gate_up_geglu_metal_rm32_f16 / _f16acc_f16 (metal/gemma4.metal:373-383,
//     gate_up_geglu_rm32 at metal_engine.mm:288)                         -> PAIR = true
//   gemma_q4k_mma_metal_f16[_f16acc_f16] (metal:385-395; ffn_down / matmul at
//     mm:289, mm:271, Q4_K down layers)                                  -> PAIR = false
//
// Each wave decodes its own B fragments (the weights) straight from the CDNA4
// image into registers: lane l of a 32x32x16 MFMA B operand holds weight row
// l%32 at 8 consecutive k, and in the CDNA4 layout those are 4 bytes of qs of
// that row's 16-byte chunk, so one 8-byte load per (row, chunk) feeds two
// fragments (low nibbles: group 2p, high nibbles: group 2p+1).  Only x goes
// through LDS (buffer_load ... lds, three buffers, one barrier per 64-wide k
// step); no decoded weight tile is written to or read from LDS.
//
// Values stay integer-exact as in ns_gemm.hip: the fragment holds
// z * sc * q * 2^-14, z = d/e (1 except for blocks whose d is far below dmin),
// which fp16 represents exactly (sc*q <= 945).  A qs dword is byte-permuted to
// [b0, b2, b1, b3] so that masking it with 0x000F000F leaves the nibbles of k
// and k+1 as fp16 subnormals q * 2^-24 in its two halves (0x00F000F0: 16q *
// 2^-24 for the high nibbles); one packed fp16 multiply by sc * 2^10 (sc * 2^6)
// gives the fragment values with one rounding of an exact product.  The
// accumulator holds S / E with E = e * 2^14 per column and super-block; the
// Q4_K min term is two extra MFMAs per super-block over the group sums of x
// (hi + lo fp16 planes; the min factors as fp16 hi + lo), and entering a new super-block rescales the
// accumulator by E_prev / E_cur.  FP32 mode only: the FP16 mode on this layout runs
// ns_gemm_f16.hip.
//
// Tiling: a workgroup of 4 waves computes 128 tokens x 256 B columns; each
// wave owns all 128 tokens (4 MFMA tiles) and 64 columns (2 tiles): for PAIR
// 32 gate rows and the same 32 up rows, so GeGLU runs in registers.  Two
// workgroups run per CU.  Work items map onto XCDs so that one XCD's L2 holds
// one 128-token slice of x.  Split K and its deterministic last-arriver
// reduction work as in ns_gemm.hip.
#include "ns_internal.hpp"
#include "ns_quant.hpp"

namespace ns {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int TT = 128;              // tokens per workgroup (= per wave)
static_assert(256 % TT == 0, "a token tile lies inside one 256-token block of the rescaled copy");
constexpr int MI = TT / 32;          // 32-token MFMA tiles per wave
constexpr int NJ = 2;                // 32-column MFMA tiles per wave
constexpr int TC = kWaves * NJ * 32; // B columns per workgroup
constexpr int KS = 64;               // k per step
constexpr int XBUF = 3;              // x buffers in LDS
constexpr int XDMA = TT * KS * 2 / 16 / kThreads;  // 16-byte x chunks per thread per step
constexpr int kRawLoads = NJ * 3;    // vector loads per step: 2 x 8 B qs + 16 B header per column

__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, int(bytes), 0x00020000);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, int(off), 0, 0); }
__device__ __forceinline__ u32x2 bload8(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b64(r, int(off), 0, 0); }

// Raw bytes of one column for one k step: qs bytes 8*hl..8*hl+7 of chunks
// 1+2p and 2+2p, and the block header (d, dmin, scales).
struct Raw {
    u32x2 qa, qb;
    u32x4 hdr;
};

// Four fragments of one column for one step: frag[kk] covers k 16kk + 8hl + 0..7.
struct Frags {
    half8_t f[4];
};

__device__ __forceinline__ uint32_t pk_mul(uint32_t a, half2_t s) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, a) * s);
}

// 8 qs bytes (dwords w0, w1) -> low-nibble fragment (scale slo) and high-nibble
// fragment (scale shi), k order 0..7.
__device__ __forceinline__ void decode8(u32x2 w, half2_t slo, half2_t shi, half8_t &lo, half8_t &hi) {
    u32x4 L, H;
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        const uint32_t p = __builtin_amdgcn_perm(w[d], w[d], 0x03010200u);  // [b0, b2, b1, b3]
        const uint32_t p8 = p >> 8;
        L[2 * d] = pk_mul(p & 0x000F000Fu, slo);
        L[2 * d + 1] = pk_mul(p8 & 0x000F000Fu, slo);
        H[2 * d] = pk_mul(p & 0x00F000F0u, shi);
        H[2 * d + 1] = pk_mul(p8 & 0x00F000F0u, shi);
    }
    lo = __builtin_bit_cast(half8_t, L);
    hi = __builtin_bit_cast(half8_t, H);
}

template <bool PAIR>
__global__ __launch_bounds__(kThreads, 2) void gemm_reg_kernel(
    const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, const uint16_t *__restrict__ x,
    const uint16_t *__restrict__ xsums, void *__restrict__ out, float *__restrict__ partial,
    uint32_t *__restrict__ counters, uint32_t cols, uint32_t rows, uint32_t batch, uint32_t ntok_tiles,
    uint32_t ncol_tiles, uint32_t kparts, uint32_t wbytes, uint32_t rs_spin, uint32_t *__restrict__ err) {
    __shared__ __attribute__((aligned(16))) u32x4 Xs[XBUF][TT * 8];
    __shared__ uint32_t last_flag, late_flag;

    const uint32_t tid = threadIdx.x, lane = tid & 63, hl = lane >> 5;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // XCD-aware order: workgroup L runs on XCD L % 8; work item q = (kp * ntok + tt) * ncol + ct,
    // and XCD x takes the contiguous run [x*W/8, (x+1)*W/8), so its L2 holds whole x slices.
    const uint32_t nwg = gridDim.x, w8 = nwg / 8, L = blockIdx.x;
    const uint32_t q = L < 8 * w8 ? (L % 8) * w8 + L / 8 : L;
    const uint32_t ct = q % ncol_tiles, g = q / ncol_tiles, tt = g % ntok_tiles, kp = g / ntok_tiles;
    const uint32_t tile = tt + ntok_tiles * ct;
    const uint32_t t0 = tt * TT;
    const uint32_t nb = cols / kQK, ngroups = cols / 32;
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
    const rsrc_t xssrc = make_rsrc(xsums, 2 * batch * ngroups * 2);
    // A tile in a 256-token block with a rescaled token reads x from the rescaled copy,
    // which holds every row of that block, and multiplies its tokens' outputs back by
    // their factor (TT divides 256).
    const float *xsb = reinterpret_cast<const float *>(xsums);
    const XsLayout xl = xs_layout(cols, batch);
    // (one uniform load; the prologue issues the weight loads before the first x DMA, so
    // its latency overlaps theirs)
    const uint32_t tile_scaled = __builtin_amdgcn_readfirstlane(reinterpret_cast<const uint32_t *>(xsb + xl.bflag)[t0 / 256]);
    const rsrc_t xsrc = make_rsrc(tile_scaled ? static_cast<const void *>(xsb + xl.xcopy) : x, batch * cols * 2);

    // byte offset of chunk c of row r, super-block b, in the CDNA4 image
    auto chunk_off = [&](uint32_t r, uint32_t b, uint32_t c) -> uint32_t {
        return uint32_t(region_offset(Q4_K, r / kRowTile, b, nb)) + (c * kRowTile + r % kRowTile) * 16;
    };
    auto load_raw = [&](uint32_t s, Raw (&raw)[NJ]) {
        const uint32_t b = s >> 2, p = s & 3;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const rsrc_t src = (PAIR && j == 1) ? wsrc1 : wsrc0;
            const uint32_t r = brow(j);
            raw[j].qa = bload8(src, chunk_off(r, b, 1 + 2 * p) + 8 * hl);
            raw[j].qb = bload8(src, chunk_off(r, b, 2 + 2 * p) + 8 * hl);
            raw[j].hdr = bload16(src, chunk_off(r, b, 0));
        }
    };
    // x(s) -> Xs[buf] by LDS DMA: instruction i of wave w fills rows 8*(w + 4i) .. +7;
    // lane L writes chunk L of that 1 KiB block (row +L/8, position L%8), i.e. global
    // chunk (L%8) ^ ((R>>1)&7) of the row, which keeps fragment reads conflict-free.
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

    float16_t acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    // Per-column super-block state: E (the accumulator is S / E) and the
    // fragment scales (low / high nibble) of the current group pair.
    float Ecur[NJ] = {}, Eprev[NJ] = {};
    // Two raw slots: step s decodes slot s&1, then reloads it with raw(s+2).
    Raw raw[2][NJ];

    const uint32_t sbeg = 4 * sb0, send = 4 * sb1;
    // prologue: x(sbeg), x(sbeg+1) in LDS; raw(sbeg), raw(sbeg+1) in flight
    load_raw(sbeg, raw[0]);
    if (sbeg + 1 < send) load_raw(sbeg + 1, raw[1]);
    dma_x(sbeg, sbeg % XBUF);
    if (sbeg + 1 < send) dma_x(sbeg + 1, (sbeg + 1) % XBUF);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // Step s: decode raw(s); issue x(s+2) and raw(s+2) (into the slot raw(s) just
    // left); run the MFMAs of s; then make x(s+1) visible (wait for its DMA,
    // barrier).  x buffer (s+2)%3 was last read at step s-1, which every wave
    // finished before passing the barrier of step s-1.
    for (uint32_t sb = sb0; sb < sb1; ++sb) {
        u32x4 xsf[MI];  // group sums of x for the min term: hi in lanes 0-31, lo in 32-63
#pragma unroll
        for (int i = 0; i < MI; ++i)
            xsf[i] = bload16(xssrc, (hl * batch * ngroups + (t0 + i * 32 + (lane & 31)) * ngroups + 8 * sb) * 2);
#pragma unroll
        for (int jstep = 0; jstep < 4; ++jstep) {
            const uint32_t s = 4 * sb + uint32_t(jstep);
            const int ri = jstep & 1;  // (s - sbeg) & 1, sbeg being a multiple of 4

            // super-block entry: E of each column, rescale of the accumulator
            half2_t slo[NJ], shi[NJ];
            half8_t bmin[NJ], bmin_lo[NJ];
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const Raw &rw = raw[ri][j];
                const float d = lo_half(rw.hdr.x), dmin = hi_half(rw.hdr.x);
                float e = __builtin_fmaxf(d, dmin * 0.0009765625f);
                e = e > 0.f ? e : 1.f;
                const float re = __builtin_amdgcn_rcpf(e);
                const float z = d == e ? 1.f : d * re;
                const Q4Scales sc = q4_scales(rw.hdr.y, rw.hdr.z, rw.hdr.w);
                const uint32_t p = uint32_t(jstep);
                const _Float16 a = _Float16(z * float(q4_sc(sc, int(2 * p))) * 1024.0f);
                const _Float16 b = _Float16(z * float(q4_sc(sc, int(2 * p + 1))) * 64.0f);
                slo[j] = half2_t{a, a};
                shi[j] = half2_t{b, b};
                if (jstep == 0) {
                    Eprev[j] = Ecur[j];
                    Ecur[j] = e * 16384.0f;
                }
                if (jstep == 3) {
                    // Min term B fragments.  b_g = fp16(m_g * (-dmin / E)) sits in k 0-7 (against
                    // the hi sums) and again in k 8-15 (against the lo sums); its rounding residue
                    // fp16(m_g * (-dmin / E) - b_g) is a second fragment, k 0-7 only, against the
                    // hi sums, so the min term keeps ~22 significant bits (b_g alone: 11).
                    const float f = -dmin * re * 0.00006103515625f;
                    half8_t bh, bl;
#pragma unroll
                    for (int gg = 0; gg < 8; ++gg) {
                        const float v = f * float(q4_m(sc, gg));
                        bh[gg] = _Float16(v);
                        bl[gg] = hl == 0 ? _Float16(v - float(bh[gg])) : _Float16(0.0f);
                    }
                    bmin[j] = bh;
                    bmin_lo[j] = bl;
                }
            }
            // fragments of step s: frag[kk] for kk = 0 (qa lo), 1 (qb lo), 2 (qa hi), 3 (qb hi)
            Frags fb[NJ];
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                decode8(raw[ri][j].qa, slo[j], shi[j], fb[j].f[0], fb[j].f[2]);
                decode8(raw[ri][j].qb, slo[j], shi[j], fb[j].f[1], fb[j].f[3]);
            }
            // No scheduling fence around the decode, the loads and the MFMAs: the
            // scheduler may move decode and rescale work between the MFMAs (MI355X,
            // gate/up pair at batch 1024: 1-3% faster than with fences).  The loads
            // of s+2 overwrite raw(s)'s registers, so they follow its decode anyway.
            if (s + 2 < send) {
                dma_x(s + 2, (s + 2) % XBUF);
                load_raw(s + 2, raw[ri]);
            }
            if (jstep == 0 && sb > sb0) {
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const float rinv = __builtin_amdgcn_rcpf(Ecur[j]), r = Eprev[j] * rinv;
#pragma unroll
                    for (int i = 0; i < MI; ++i)
#pragma unroll
                        for (int v = 0; v < 16; ++v) acc[i][j][v] *= r;
                }
            }

            const uint32_t buf = s % XBUF;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                half8_t a[MI];
#pragma unroll
                for (int i = 0; i < MI; ++i) {
                    const uint32_t R = i * 32 + (lane & 31), c = 2 * kk + hl;
                    a[i] = __builtin_bit_cast(half8_t, Xs[buf][R * 8 + (c ^ ((R >> 1) & 7))]);
                }
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], fb[j].f[kk], acc[i][j], 0, 0, 0);
            }
            if (jstep == 3) {  // min term of super-block sb
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            __builtin_bit_cast(half8_t, xsf[i]), bmin_lo[j],
                            __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, xsf[i]), bmin[j],
                                                                   acc[i][j], 0, 0, 0),
                            0, 0, 0);
            }
            // x(s+1) must be in LDS for every wave: wait for its DMA (issued one step
            // ago; the loads issued after it -- raw(s+1), x(s+2), raw(s+2) -- may stay
            // in flight), then meet at the barrier.  The barrier is the bare s_barrier:
            // __syncthreads() adds a workgroup fence, which the compiler implements by also
            // waiting for x(s+2)'s DMA, issued this step.  The barrier orders every wave's
            // reads of buffer s % 3 (all consumed by this step's MFMAs) before the DMA of
            // x(s+3) into it; the signal fences keep the compiler from moving memory
            // accesses across it.
            __builtin_amdgcn_sched_barrier(0);
            if (s + 2 < send) {
                constexpr int n = kRawLoads + XDMA + kRawLoads;
                __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
            } else {
                __builtin_amdgcn_s_waitcnt(0);
            }
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_barrier();
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
        }
    }

    // ---- S = acc * E_last.  32x32 D layout: lane holds column lane%32 and rows
    // 8*(v/4) + 4*(lane/32) + v%4 for v = 0..15.
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] *= Ecur[j];
    auto tok_of = [&](int i, int v) -> uint32_t {
        return t0 + uint32_t(i) * 32 + 8 * uint32_t(v >> 2) + 4 * hl + uint32_t(v & 3);
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
                for (int j = 0; j < NJ; ++j) acc[i][j][v] *= tf;
            }
    }

    // output of one (token, column pair): fp16 GeGLU (PAIR) or fp32 per column
    auto emit = [&](uint32_t t, const float (&val)[NJ]) {
        if (t >= batch) return;
        if constexpr (PAIR) {
            const uint32_t r = brow(0);
            if (r < rows) reinterpret_cast<_Float16 *>(out)[size_t(t) * rows + r] = _Float16(gelu_tanh(val[0]) * val[1]);
        } else {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const uint32_t r = brow(j);
                if (r < rows) reinterpret_cast<float *>(out)[size_t(t) * rows + r] = val[j];
            }
        }
    };

    // outputs of token sub-tile i, from get(v, j) = accumulator element v of fragment j
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

    // ---- split K.  Parts [kp][plane][ntok*TT][ncol*rows per tile] (PAIR: gate, up; plain: one plane):
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
    for (int j = 0; j < NJ; ++j)
        lane_off[j] = ((PAIR ? uint32_t(j) : 0u) * tpad + t0 + 4 * hl) * rstride + brow(j) * 4u;
    // byte offset of (token sub-tile i, element v, fragment j) within one part,
    // given the lane terms lo
    auto poff = [&](const uint32_t (&lo)[NJ], int i, int v, int j) -> uint32_t {
        return (uint32_t(i) * 32 + 8 * uint32_t(v >> 2) + uint32_t(v & 3)) * rstride + lo[j];
    };
    auto pbase = [&](uint32_t part) -> char * { return reinterpret_cast<char *>(partial + part * pstride); };  // uniform
    if (rs_spin != 0) {
        // Reduce-scatter (launched only when the whole grid fits on the device at once, so the
        // kparts workgroups of a tile run together; kparts == MI): part kp owns token sub-tile
        // kp of every wave.  Each part stores the sub-tiles it does not own, parks its own in
        // LDS (the x buffers, free after the main loop), counts one arrival on written[tile]
        // once its stores are acknowledged, waits until every part has, then adds the parts of
        // its sub-tile in part order (its own from LDS) and writes it.  The wait is bounded: a
        // part whose limit runs out writes its sub-tile as NaN.  The last part past the wait
        // clears both counters.
        const uint32_t ntiles = ntok_tiles * ncol_tiles;
        uint32_t *written = counters + tile, *departed = counters + ntiles + tile;
        float *slot = reinterpret_cast<float *>(&Xs[0][0]);
        __syncthreads();  // every wave is past its last read of the x buffers
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            if (uint32_t(i) == kp) {
#pragma unroll
                for (int v = 0; v < 16; ++v)
#pragma unroll
                    for (int j = 0; j < NJ; ++j) slot[(v * NJ + j) * kThreads + tid] = acc[i][j][v];
            } else {
#pragma unroll
                for (int v = 0; v < 16; ++v)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        __hip_atomic_store(reinterpret_cast<float *>(pbase(kp) + poff(lane_off, i, v, j)), acc[i][j][v],
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
        float sum[16][NJ];
        for (uint32_t p0 = 0; p0 < kparts; p0 += 2) {  // two parts per round trip
            float pv[2][16][NJ];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                // this part's own slot holds no value for its sub-tile: read from LDS below
                const uint32_t part = __builtin_elementwise_min(p0 + uint32_t(u), kparts - 1);
                uint32_t lo[NJ];
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    lo[j] = lane_off[j];
                    asm volatile("" : "+v"(lo[j]));
                }
#pragma unroll
                for (int v = 0; v < 16; ++v)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        pv[u][v][j] = __hip_atomic_load(reinterpret_cast<float *>(pbase(part) + poff(lo, int(kp), v, j)),
                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
            for (int v = 0; v < 16; ++v)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    float t = sum[v][j];
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const uint32_t part = p0 + uint32_t(u);
                        const float val = part == kp ? slot[(v * NJ + j) * kThreads + tid] : pv[u][v][j];
                        // the last arrival's order: (0 + part 0) + part 1 + ...
                        t = part < kparts ? (part == 0 ? 0.f : t) + val : t;
                    }
                    sum[v][j] = t;
                }
        }
        write_out(int(kp), [&](int v, int j) {
            return late ? __builtin_nanf("") : sum[v][j];
        });
        return;
    }
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                __hip_atomic_store(reinterpret_cast<float *>(pbase(kp) + poff(lane_off, i, v, j)), acc[i][j][v],
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    // Device-coherent atomics only: the parts bypass the XCD-private L2; the wait
    // makes every part store complete before the arrival is counted.
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
            for (int j = 0; j < NJ; ++j) {
                lo[j] = lane_off[j];
                asm volatile("" : "+v"(lo[j]));
            }
            float pv[2][16][NJ];
#pragma unroll
            for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                for (int v = 0; v < 16; ++v)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        pv[ii][v][j] = __hip_atomic_load(reinterpret_cast<float *>(pbase(part) + poff(lo, i0 + ii, v, j)),
                                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                for (int v = 0; v < 16; ++v)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        sum[ii][v][j] = (part == 0 ? 0.f : sum[ii][v][j]) + pv[ii][v][j];
        }
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
            write_out(i0 + ii, [&](int v, int j) { return sum[ii][v][j]; });
    }
}

// Workgroups of one instance the device holds at once (two per CU), per device and instance.
template <class K>
uint64_t resident_wgs(K kernel) {
    static int cache[64][2] = {};
    int dev = 0;
    (void)hipGetDevice(&dev);
    const int slot = kernel == &gemm_reg_kernel<true> ? 0 : 1;
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

struct RegPlan {
    uint32_t ntok, ncol, kparts;
};

RegPlan plan_reg(uint32_t cols, uint32_t rows, uint32_t batch, bool pair, const Tuning &t) {
    RegPlan p;
    p.ntok = (batch + TT - 1) / TT;
    const uint32_t rows_per_tile = pair ? TC / 2 : TC;
    p.ncol = (rows + rows_per_tile - 1) / rows_per_tile;
    const uint32_t nb = cols / kQK, tiles = p.ntok * p.ncol;
    p.kparts = 1;
    // two workgroups per CU on 256 CUs: split K until the grid covers most of them
    while (tiles * p.kparts < 400 && p.kparts * 2 <= nb / 2) p.kparts *= 2;
    if (t.gemm_kparts >= 1 && uint32_t(t.gemm_kparts) <= nb) p.kparts = uint32_t(t.gemm_kparts);
    // one split-K part (padded to whole tiles) must stay under 4 GiB: 32-bit offsets in the kernel
    if (uint64_t(pair ? 2 : 1) * p.ntok * TT * p.ncol * rows_per_tile * 4 >= (uint64_t(1) << 32)) p.kparts = 1;
    return p;
}

}  // namespace

void gemm_reg_workspace_need(uint32_t cols, uint32_t rows, uint32_t batch, bool pair, const Tuning &t,
                             size_t *part_floats, size_t *counters) {
    const RegPlan p = plan_reg(cols, rows, batch, pair, t);
    *part_floats = p.kparts > 1 ? size_t(p.kparts) * (pair ? 2 : 1) * (p.ntok * TT) * (p.ncol * (pair ? TC / 2 : TC)) : 0;
    *counters = 2 * size_t(p.ntok) * p.ncol;  // written, then departed (reduce-scatter); the first alone otherwise
}

hipError_t launch_gemm_reg(const uint8_t *w, const uint8_t *up, const uint16_t *x, const uint16_t *xsums,
                           void *out, uint32_t cols, uint32_t rows, uint32_t batch, float *partial,
                           uint32_t *counters, uint32_t *err, const Tuning &t, hipStream_t stream) {
    const bool pair = up != nullptr;
    const RegPlan p = plan_reg(cols, rows, batch, pair, t);
    const dim3 grid(p.ntok * p.ncol * p.kparts), block(kThreads);
    const uint32_t wbytes = rows * (cols / kQK) * kQ4Bytes;
    const auto kernel = pair ? &gemm_reg_kernel<true> : &gemm_reg_kernel<false>;
    // the reduce-scatter needs every part of a tile running at once (the whole grid resident) and
    // one token sub-tile per part (its LDS slot)
    uint32_t rs_spin = 0;
    if (p.kparts == uint32_t(MI) && t.gemm_rs != 0 && waits_allowed(t) && uint64_t(grid.x) <= resident_wgs(kernel))
        rs_spin = t.gemm_rs > 1 ? uint32_t(t.gemm_rs) : 1u << 22;  // 2^22 polls of s_sleep 2: seconds
    kernel<<<grid, block, 0, stream>>>(w, pair ? up : w, x, xsums, out, partial, counters, cols, rows, batch, p.ntok,
                                       p.ncol, p.kparts, wbytes, rs_spin, err);
    return hipGetLastError();
}

}  // namespace ns
