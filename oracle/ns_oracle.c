/*
 * ns_oracle.c -- CPU restatement of the reference's quantized FFN arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (the checker and the timed CPU baseline); see
 * ns_oracle.h for the list of reference lines each function follows and for
 * what pins each one.  Built with -ffp-contract=off so that every fp32 sum is
 * the sequential, uncontracted sum that quant.cpp:21 writes.
 */
#include "ns_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---- fp16 <-> fp32 (IEEE binary16, round to nearest even) ---------------- */

float nso_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    const uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        /* zero or subnormal: mant * 2^-24, exact in fp32 */
        float v = (float)mant * 5.9604644775390625e-08f;
        return sign ? -v : v;
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t nso_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u);
    if (ax >= 0x477ff000u) return sign | 0x7c00u; /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                       /* below 2^-14: subnormal half */
        if (ax < 0x33000000u) return sign;        /* <= 2^-25 rounds to zero */
        const uint32_t e = ax >> 23;
        const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e;           /* 14..24 */
        uint32_t r = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return sign | (uint16_t)r;
    }
    const uint32_t e16 = (ax >> 23) - 127u + 15u;
    uint32_t r = (e16 << 10) | ((ax >> 13) & 0x3ffu);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return sign | (uint16_t)r;
}

/* FP16-mode rounding: round to nearest even at 11 significant bits (the fp16
 * significand) while keeping the fp32 exponent range, so values beyond the
 * fp16 maximum do not overflow.  Equals fp16 rounding on the fp16 normal range. */
float nso_round_f16p(float v) {
    uint32_t b;
    memcpy(&b, &v, 4);
    if ((b & 0x7f800000u) == 0x7f800000u) return v;
    b = (b + 0x0fffu + ((b >> 13) & 1u)) & 0xffffe000u;
    memcpy(&v, &b, 4);
    return v;
}

/* ---- element values (quant.cpp:9-18) ------------------------------------ */

static float rd_f16(const uint8_t *p) { return nso_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* quant.cpp:9-12: 8 groups of 32; 6-bit scale/min unpack; w = d*sc*q - dmin*m. */
float nso_q4k_value(const uint8_t *b, uint32_t i) {
    const float d = rd_f16(b), dm = rd_f16(b + 2);
    const uint8_t *s = b + 4, *q = b + 16;
    const uint32_t g = i / 32, l = i % 32;
    uint8_t sc, m;
    if (g < 4) {
        sc = s[g] & 63;
        m = s[g + 4] & 63;
    } else {
        sc = (uint8_t)((s[g + 4] & 15) | ((s[g - 4] >> 6) << 4));
        m = (uint8_t)((s[g + 4] >> 4) | ((s[g] >> 6) << 4));
    }
    const uint8_t v = (g & 1) ? (uint8_t)(q[(g / 2) * 32 + l] >> 4) : (uint8_t)(q[(g / 2) * 32 + l] & 15);
    return d * sc * v - dm * m;
}

/* quant.cpp:13-18: 6-bit value from ql nibble + qh 2 bits; w = d*sc*(v-32). */
float nso_q6k_value(const uint8_t *b, uint32_t i) {
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    const float d = rd_f16(b + 208);
    const uint32_t half = i / 128, p = i % 128, l = p % 32, quarter = p / 32;
    const uint8_t *lo = ql + half * 64, *hi = qh + half * 32;
    int v;
    if (quarter == 0) v = (lo[l] & 15) | (((hi[l] >> 0) & 3) << 4);
    else if (quarter == 1) v = (lo[l + 32] & 15) | (((hi[l] >> 2) & 3) << 4);
    else if (quarter == 2) v = (lo[l] >> 4) | (((hi[l] >> 4) & 3) << 4);
    else v = (lo[l + 32] >> 4) | (((hi[l] >> 6) & 3) << 4);
    return d * sc[half * 8 + (l / 16) + quarter * 2] * (v - 32);
}

/* ---- layouts -------------------------------------------------------------- */

/* ROW_MAJOR: GGUF order (quant.cpp:20 block = e/256).  NSMFFN:
 * metal_ffn.cpp:145-146 target = ((row0/64)*blocks + block)*64 + row. */
uint64_t nso_block_index(int layout, uint64_t row, uint64_t kblock, uint64_t nb) {
    if (layout == NSO_NSMFFN) return ((row / 64) * nb + kblock) * 64 + row % 64;
    return row * nb + kblock;
}

static size_t block_bytes(int type) { return type == NSO_Q4_K ? 144 : 210; }

static int check(int type, int layout, uint64_t cols, uint64_t rows) {
    if (type != NSO_Q4_K && type != NSO_Q6_K) return -1;
    if (layout != NSO_ROW_MAJOR && layout != NSO_NSMFFN) return -1;
    if (cols % 256) return -1;
    if (layout == NSO_NSMFFN && rows % 64) return -1;
    return 0;
}

/* ---- FP16-mode tiles -------------------------------------------------------
 * The FP16 mode multiplies fp16 tiles of the weights, the reference's
 * half(d*sc*q - dmin*m) / half(d*sc*(v-32)) (metal/gemma4.metal:229-232, :415-419),
 * with a per-row power of two c folded in so that the tile is one packed fp16 FMA
 * from the quant bits (this build's kernels, neutron-star_amd/csrc/ns_tile16.hpp):
 *   M = max over the row's blocks of max(|d|, |dmin|) (Q6_K: |d|)
 *   c = 2^(-15 - E), E = ceil(log2 M) (Q6_K: floor(log2 M) + 1, the power of two strictly
 *       above M, so that A = d*sc*2^24*c stays within fp16 for sc = -128), c = 1 when M == 0
 *   A = RNE16(d*sc*2^24*c),  B = RNE16(-dmin*m*c)  (Q6_K: B = RNE16(-32*d*sc*c))
 *   F = RNE16(q*2^-24*A + B)                       (Q6_K: q is the 6-bit v)
 * and the output is RNE11((sum_k F*x) / c).  Every quantity before RNE16 is exact
 * in double, so each RNE16 here is one rounding of the exact value, as the fused
 * fp16 FMA and the fp32 -> fp16 conversions of the kernel are. */

/* Round an exact double to binary16, nearest even, subnormals kept, overflow to inf;
 * returned as the (exact) double of the fp16 value. */
static double rne16(double v) {
    const double a = fabs(v);
    if (a == 0.0) return v;
    int ex;
    frexp(a, &ex);                       /* a = m * 2^ex, m in [0.5, 1) */
    int e = ex - 1;                      /* a in [2^e, 2^(e+1)) */
    if (e < -14) e = -14;                /* subnormal range: ulp 2^-24 */
    const double ulp = ldexp(1.0, e - 10);
    double q = nearbyint(a / ulp);       /* the default mode rounds to nearest even */
    double r = q * ulp;
    if (r > 65504.0) r = INFINITY;
    return v < 0 ? -r : r;
}

static void row_scale(int type, int layout, const uint8_t *w, uint64_t cols, uint64_t row, double *c24,
                      double *inv_c) {
    const uint64_t nb = cols / 256;
    const size_t bs = block_bytes(type);
    double M = 0.0;
    for (uint64_t b = 0; b < nb; ++b) {
        const uint8_t *blk = w + nso_block_index(layout, row, b, nb) * bs;
        if (type == NSO_Q4_K) {
            M = fmax(M, fabs((double)rd_f16(blk)));
            M = fmax(M, fabs((double)rd_f16(blk + 2)));
        } else {
            M = fmax(M, fabs((double)rd_f16(blk + 208)));
        }
    }
    if (!(M > 0.0)) {
        *c24 = 16777216.0;
        *inv_c = 1.0;
        return;
    }
    int ex;
    const double m = frexp(M, &ex);      /* M = m * 2^ex */
    /* ceil(log2 M); Q6_K: floor(log2 M) + 1 = ex */
    const int e = (m == 0.5 && type == NSO_Q4_K) ? ex - 1 : ex;
    *c24 = ldexp(1.0, 9 - e);
    *inv_c = ldexp(1.0, 15 + e);
}

/* F of element i of a block, given the row's c24 = c * 2^24. */
static double f16_tile_value(int type, const uint8_t *b, uint32_t i, double c24) {
    const double c = c24 * 5.9604644775390625e-08;
    if (type == NSO_Q4_K) {
        const double d = rd_f16(b), dm = rd_f16(b + 2);
        const uint8_t *s = b + 4, *q = b + 16;
        const uint32_t g = i / 32, l = i % 32;
        uint8_t sc, m;
        if (g < 4) {
            sc = s[g] & 63;
            m = s[g + 4] & 63;
        } else {
            sc = (uint8_t)((s[g + 4] & 15) | ((s[g - 4] >> 6) << 4));
            m = (uint8_t)((s[g + 4] >> 4) | ((s[g] >> 6) << 4));
        }
        const uint8_t v = (g & 1) ? (uint8_t)(q[(g / 2) * 32 + l] >> 4) : (uint8_t)(q[(g / 2) * 32 + l] & 15);
        const double A = rne16(d * sc * c24), B = rne16(-dm * m * c);
        return rne16((double)v * 5.9604644775390625e-08 * A + B);
    }
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *scs = (const int8_t *)(b + 192);
    const double d = rd_f16(b + 208);
    const uint32_t half = i / 128, p = i % 128, l = p % 32, quarter = p / 32;
    const uint8_t *lo = ql + half * 64, *hi = qh + half * 32;
    int v;
    if (quarter == 0) v = (lo[l] & 15) | (((hi[l] >> 0) & 3) << 4);
    else if (quarter == 1) v = (lo[l + 32] & 15) | (((hi[l] >> 2) & 3) << 4);
    else if (quarter == 2) v = (lo[l] >> 4) | (((hi[l] >> 4) & 3) << 4);
    else v = (lo[l + 32] >> 4) | (((hi[l] >> 6) & 3) << 4);
    const double sc = scs[half * 8 + (l / 16) + quarter * 2];
    const double A = rne16(d * sc * c24), B = rne16(-32.0 * d * sc * c);
    return rne16((double)v * 5.9604644775390625e-08 * A + B);
}

int nso_f16_tile_row(int type, int layout, const uint8_t *w, uint64_t cols, uint64_t rows, uint64_t row,
                     float *tile, float *inv_c) {
    if (check(type, layout, cols, rows) || row >= rows) return -1;
    double c24, ic;
    row_scale(type, layout, w, cols, row, &c24, &ic);
    const uint64_t nb = cols / 256;
    const size_t bs = block_bytes(type);
    for (uint64_t b = 0; b < nb; ++b) {
        const uint8_t *blk = w + nso_block_index(layout, row, b, nb) * bs;
        for (uint32_t i = 0; i < 256; ++i) tile[b * 256 + i] = (float)f16_tile_value(type, blk, i, c24);
    }
    *inv_c = (float)ic;
    return 0;
}

int nso_dequant_row(int type, int layout, const uint8_t *w, uint64_t cols, uint64_t rows,
                    uint64_t row, float *out) {
    if (check(type, layout, cols, rows) || row >= rows) return -1;
    const uint64_t nb = cols / 256;
    const size_t bs = block_bytes(type);
    for (uint64_t b = 0; b < nb; ++b) {
        const uint8_t *blk = w + nso_block_index(layout, row, b, nb) * bs;
        for (uint32_t i = 0; i < 256; ++i)
            out[b * 256 + i] = type == NSO_Q4_K ? nso_q4k_value(blk, i) : nso_q6k_value(blk, i);
    }
    return 0;
}

/* quant.cpp:21: float sum=0; for i<cols: sum += dequant(row*cols+i) * x[i]. */
float nso_dot_row(int type, int layout, const uint8_t *w, uint64_t cols, uint64_t rows,
                  uint64_t row, const float *x) {
    (void)rows;
    const uint64_t nb = cols / 256;
    const size_t bs = block_bytes(type);
    float sum = 0;
    for (uint64_t i = 0; i < cols; ++i) {
        const uint8_t *blk = w + nso_block_index(layout, row, i / 256, nb) * bs;
        const float v = type == NSO_Q4_K ? nso_q4k_value(blk, (uint32_t)(i % 256))
                                         : nso_q6k_value(blk, (uint32_t)(i % 256));
        sum += v * x[i];
    }
    return sum;
}

/* metal/gemma4.metal:78 -- 0.5*g*(1+tanh(0.79788456*g*(1+0.044715*g*g))). */
float nso_gelu_tanh(float g) {
    return 0.5f * g * (1.0f + tanhf(0.7978845608028654f * g * (1.0f + 0.044715f * g * g)));
}

/* metal/gemma4.metal:509-529, the RMSNorm family the engine runs around the FFN block
 * (rms, rms_half, rms_add, rms_add_then_half: metal_engine.mm:291-296).  Per row:
 *   s = sum_k x[k]*x[k] (sequential), r = 1/sqrtf(s/width + eps)          (metal:510, :517)
 *   y[k] = (x[k]*r)*w[k], plus residual[k] first when residual != NULL,
 *          times *scale when scale != NULL                                (metal:511, :517, :520)
 *   with next_w: s2 over y, next[k] = (y[k]*r2)*next_w[k]                  (metal:524-525)
 * The reference sums in 256-thread strides plus simd_sum (metal:510); this is the
 * sequential order, so outputs agree to rounding. */
int nso_rmsnorm(const float *x, const float *w, const float *residual, const float *scale, const float *next_w,
                uint64_t rows, uint64_t width, float eps, float *y, float *next) {
    if (width == 0 || (next_w && !next)) return -1;
    for (uint64_t t = 0; t < rows; ++t) {
        const float *xr = x + t * width;
        float *yr = y + t * width;
        float s = 0.0f;
        for (uint64_t k = 0; k < width; ++k) s += xr[k] * xr[k];
        const float r = 1.0f / sqrtf(s / (float)width + eps);
        float s2 = 0.0f;
        for (uint64_t k = 0; k < width; ++k) {
            float v = (xr[k] * r) * w[k];
            if (residual) {
                v = residual[t * width + k] + v;
                if (scale) v *= *scale;
            }
            yr[k] = v;
            s2 += v * v;
        }
        if (next_w) {
            const float r2 = 1.0f / sqrtf(s2 / (float)width + eps);
            for (uint64_t k = 0; k < width; ++k) next[t * width + k] = (yr[k] * r2) * next_w[k];
        }
    }
    return 0;
}

/* ---- threaded drivers ---------------------------------------------------- */

typedef struct {
    int type, layout, acc_mode;
    const uint8_t *w;
    uint64_t cols, rows, batch;
    const float *x;       /* gemv: fp32 x[cols] */
    const float *xt;      /* gemm: fp32 copy of x transposed [cols][batch] */
    float *out;           /* gemv: [rows]; gemm: [batch][rows] */
    uint64_t r0, r1;
} job_t;

static void *gemv_worker(void *p) {
    job_t *j = (job_t *)p;
    float *row = (float *)malloc(j->cols * sizeof(float));
    for (uint64_t r = j->r0; r < j->r1; ++r) {
        nso_dequant_row(j->type, j->layout, j->w, j->cols, j->rows, r, row);
        float sum = 0;
        for (uint64_t k = 0; k < j->cols; ++k) sum += row[k] * j->x[k];
        j->out[r] = sum;
    }
    free(row);
    return NULL;
}

/* Row dequantised once; the token loop is innermost so each acc[t] is its own
 * sequential k-order sum (vectorised across tokens only). */
static void *gemm_worker(void *p) {
    job_t *j = (job_t *)p;
    const uint64_t B = j->batch;
    float *row = (float *)malloc(j->cols * sizeof(float));
    float *acc = (float *)malloc(B * sizeof(float));
    for (uint64_t r = j->r0; r < j->r1; ++r) {
        float inv_c = 1.0f;
        if (j->acc_mode == 1) nso_f16_tile_row(j->type, j->layout, j->w, j->cols, j->rows, r, row, &inv_c);
        else nso_dequant_row(j->type, j->layout, j->w, j->cols, j->rows, r, row);
        for (uint64_t t = 0; t < B; ++t) acc[t] = 0;
        for (uint64_t k = 0; k < j->cols; ++k) {
            const float wk = row[k];
            const float *xk = j->xt + k * B;
            for (uint64_t t = 0; t < B; ++t) acc[t] += wk * xk[t];
        }
        /* FP16 mode: the sum of the scaled tiles, times 1/c (a power of two: exact),
         * rounded once to fp16 precision (metal:394, :489 write a half tile) */
        for (uint64_t t = 0; t < B; ++t)
            j->out[t * j->rows + r] = j->acc_mode == 1 ? nso_round_f16p(acc[t] * inv_c) : acc[t];
    }
    free(acc);
    free(row);
    return NULL;
}

static int run_rows(job_t *base, uint64_t rows, int nthreads, void *(*fn)(void *)) {
    if (nthreads < 1) nthreads = 1;
    if ((uint64_t)nthreads > rows) nthreads = (int)(rows ? rows : 1);
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nthreads);
    job_t *jobs = (job_t *)malloc(sizeof(job_t) * (size_t)nthreads);
    for (int i = 0; i < nthreads; ++i) {
        jobs[i] = *base;
        jobs[i].r0 = rows * (uint64_t)i / (uint64_t)nthreads;
        jobs[i].r1 = rows * (uint64_t)(i + 1) / (uint64_t)nthreads;
        pthread_create(&th[i], NULL, fn, &jobs[i]);
    }
    for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
    free(jobs);
    free(th);
    return 0;
}

int nso_gemv(int type, int layout, const uint8_t *w, uint64_t cols, uint64_t rows,
             const float *x, float *y, int nthreads) {
    if (check(type, layout, cols, rows)) return -1;
    job_t j;
    memset(&j, 0, sizeof j);
    j.type = type; j.layout = layout; j.w = w; j.cols = cols; j.rows = rows; j.x = x; j.out = y;
    return run_rows(&j, rows, nthreads, gemv_worker);
}

int nso_gate_up_geglu(int layout, const uint8_t *wg, const uint8_t *wu, uint64_t cols,
                      uint64_t rows, const float *x, float *h, int nthreads) {
    float *g = (float *)malloc(rows * sizeof(float));
    float *u = (float *)malloc(rows * sizeof(float));
    int rc = nso_gemv(NSO_Q4_K, layout, wg, cols, rows, x, g, nthreads);
    if (!rc) rc = nso_gemv(NSO_Q4_K, layout, wu, cols, rows, x, u, nthreads);
    if (!rc)
        for (uint64_t r = 0; r < rows; ++r) h[r] = nso_gelu_tanh(g[r]) * u[r];
    free(g);
    free(u);
    return rc;
}

int nso_gemm(int type, int layout, const uint8_t *w, uint64_t cols, uint64_t rows,
             uint64_t batch, const uint16_t *x_f16, int acc_mode, float *out, int nthreads) {
    if (check(type, layout, cols, rows) || (acc_mode != 0 && acc_mode != 1)) return -1;
    float *xt = (float *)malloc(cols * batch * sizeof(float));
    if (!xt) return -1;
    for (uint64_t t = 0; t < batch; ++t)
        for (uint64_t k = 0; k < cols; ++k) xt[k * batch + t] = nso_f16_to_f32(x_f16[t * cols + k]);
    job_t j;
    memset(&j, 0, sizeof j);
    j.type = type; j.layout = layout; j.acc_mode = acc_mode; j.w = w; j.cols = cols;
    j.rows = rows; j.batch = batch; j.xt = xt; j.out = out;
    run_rows(&j, rows, nthreads, gemm_worker);
    free(xt);
    return 0;
}

int nso_gate_up_geglu_prefill(int layout, const uint8_t *wg, const uint8_t *wu, uint64_t cols,
                              uint64_t rows, uint64_t batch, const uint16_t *x_f16,
                              int acc_mode, float *h, int nthreads) {
    float *g = (float *)malloc(rows * batch * sizeof(float));
    float *u = (float *)malloc(rows * batch * sizeof(float));
    int rc = nso_gemm(NSO_Q4_K, layout, wg, cols, rows, batch, x_f16, acc_mode, g, nthreads);
    if (!rc) rc = nso_gemm(NSO_Q4_K, layout, wu, cols, rows, batch, x_f16, acc_mode, u, nthreads);
    if (!rc)
        for (uint64_t i = 0; i < rows * batch; ++i) h[i] = nso_gelu_tanh(g[i]) * u[i];
    free(g);
    free(u);
    return rc;
}
