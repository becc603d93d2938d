/*
 * ns_oracle.h -- CPU restatement of Neutron Star's quantized FFN path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or as the timed CPU baseline).  The product library never links it.
 *
 * Every function restates a piece of the reference (paths relative to the
 * reference repository):
 *   src/native/quant.cpp:9-12   Q4_K element value          -> nso_q4k_value
 *   src/native/quant.cpp:13-18  Q6_K element value          -> nso_q6k_value
 *   src/native/quant.cpp:20     dequant(tensor, element)    -> nso_dequant_row
 *   src/native/quant.cpp:21     dot_row(tensor, row, x)     -> nso_dot_row / nso_gemv
 *   metal/gemma4.metal:78       GeGLU expression            -> nso_gelu_tanh
 *   src/native/metal_ffn.cpp:135-149  .nsmffn slab reorder  -> nso_block_index
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   f16 <-> f32 conversions: numpy float16 over all 65536 bit patterns.
 *   q4k/q6k values: oracle/_ref (the reference quant.cpp compiled as-is),
 *     committed golden vectors from it, closed-form hand-built blocks.
 *   dot_row: oracle/_ref dot_row bit-exact, linearity and one-hot columns.
 *   gelu_tanh: closed forms (gelu(0)=0, large |g| -> relu, odd part identity).
 *   round_f16p: equals numpy float16 rounding over the fp16 normal range.
 *   FP16 mode (nso_f16_tile_row, nso_gemm acc_mode=1): the tile formula against
 *     closed forms (power-of-two blocks whose tiles are exact, hand-computed
 *     roundings of A, B and F, subnormal B, the row scale's ceil(log2 M) at and
 *     just past powers of two, M = 0) and the output schedule against known
 *     answers (integer sums 2049 -> 2048 in one block, 2049 + 1 over two blocks
 *     -> 2050: one rounding at the end, none per block).  These functions restate
 *     this build's own FP16-mode tiles and rounding, so a kernel checked against
 *     them is checked for self-consistency, not against the reference.  Parity
 *     unpinned: the reference's own FP16 arithmetic on Apple simdgroup_half8x8
 *     hardware, which runs nowhere here (it accumulates in half and has no single
 *     final rounding).  The FP16 mode's parity evidence is its 1e-2 bound against
 *     the FP32 path (acc_mode 0, the reference's CPU arithmetic).
 */
#ifndef NS_ORACLE_H
#define NS_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { NSO_Q4_K = 12, NSO_Q6_K = 14 };
enum { NSO_ROW_MAJOR = 0, NSO_NSMFFN = 1, NSO_CDNA4 = 2 };

float nso_f16_to_f32(uint16_t h);
uint16_t nso_f32_to_f16(float f);
/* Round to 11 significant bits (RNE), fp32 exponent range: the FP16 mode's rounding. */
float nso_round_f16p(float v);

float nso_q4k_value(const uint8_t *block, uint32_t i);
float nso_q6k_value(const uint8_t *block, uint32_t i);

/* Byte offset of element-0 block (row, kblock) for the ROW_MAJOR / NSMFFN layouts. */
uint64_t nso_block_index(int layout, uint64_t row, uint64_t kblock, uint64_t nb);

/* Dequantise one row (cols values) of a ROW_MAJOR or NSMFFN tensor to fp32. */
int nso_dequant_row(int type, int layout, const uint8_t *w, uint64_t cols, uint64_t rows,
                    uint64_t row, float *out);

/* quant.cpp:21 -- sequential fp32 sum over k of dequant * x. */
float nso_dot_row(int type, int layout, const uint8_t *w, uint64_t cols, uint64_t rows,
                  uint64_t row, const float *x);

/* y[r] = dot_row(r) for every row, threaded over rows (results identical to the
 * scalar dot_row: each row is dequantised once, then summed in k order). */
int nso_gemv(int type, int layout, const uint8_t *w, uint64_t cols, uint64_t rows,
             const float *x, float *y, int nthreads);

float nso_gelu_tanh(float g);

/* The RMSNorm family (metal:509-529): y = [residual +] (x*r)*w [* *scale], and with
 * next_w also next = (y*r2)*next_w; r = 1/sqrtf(mean(x^2) + eps), r2 likewise over y.
 * residual, scale, next_w (with next) may be NULL.  x, y: [rows][width]. */
int nso_rmsnorm(const float *x, const float *w, const float *residual, const float *scale, const float *next_w,
                uint64_t rows, uint64_t width, float eps, float *y, float *next);

/* h = gelu_tanh(Wg x) * (Wu x), fp32 (decode regime, always FP32). */
int nso_gate_up_geglu(int layout, const uint8_t *wg, const uint8_t *wu, uint64_t cols,
                      uint64_t rows, const float *x, float *h, int nthreads);

/* FP16-mode tile of one row (cols values): F = RNE16(q*2^-24*A + B) with the row
 * scale c folded into A and B (formulas in ns_oracle.c), and 1/c.  F*(1/c) is the
 * reference's half(d*sc*q - dmin*m) / half(d*sc*(v-32)) up to the order of its
 * roundings (metal:229-232, :415-419). */
int nso_f16_tile_row(int type, int layout, const uint8_t *w, uint64_t cols, uint64_t rows, uint64_t row,
                     float *tile, float *inv_c);

/* Prefill contraction: out[t][r] = sum_k W[r][k] * x[t][k] for t < batch.
 * x is fp16 bits [batch][cols].  acc_mode 0 = FP32 (quant.cpp values, sequential
 * fp32 sum, fp32 out); acc_mode 1 = FP16 mode: the tiles of nso_f16_tile_row,
 * a sequential fp32 sum, times 1/c, rounded once to fp16 precision
 * (nso_round_f16p: 11 significant bits, fp32 exponent range). */
int nso_gemm(int type, int layout, const uint8_t *w, uint64_t cols, uint64_t rows,
             uint64_t batch, const uint16_t *x_f16, int acc_mode, float *out, int nthreads);

/* Prefill gate/up + GeGLU: h[t][r] (fp32, not rounded) from fp16 x. */
int nso_gate_up_geglu_prefill(int layout, const uint8_t *wg, const uint8_t *wu, uint64_t cols,
                              uint64_t rows, uint64_t batch, const uint16_t *x_f16,
                              int acc_mode, float *h, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
