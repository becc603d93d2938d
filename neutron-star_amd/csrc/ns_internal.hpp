// ns_internal.hpp -- launchers and helpers shared by the C-ABI layer and the kernels.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "ns_common.hpp"

namespace ns {

// Thread-local error text behind ns_last_error().
void set_error(const std::string &msg);

// Kernel-selection overrides of one context (ns_ctx_set_tuning), for tests and
// experiments; the defaults select the measured plans.  Nothing reads the
// environment: an engine process behaves the same whatever it inherits.
struct Tuning {
    int gemv_pf = -1;     // -1: plan; 0 / 1: force the one-unit / the prefetching decode GEMV
    int gemv_waves = 0;   // > 0: the prefetching GEMV's flattened grid with this many waves
    int gemv_whole = 1;   // 0: no whole-slab grid
    int gemv_qslab = 1;   // 0: no k-workgroups-per-slab grid
    int gemm_kparts = 0;  // > 0: the prefill GEMM's split-K parts
    int gemm_q4_reg = 1;  // 0: the LDS-tile Q4_K GEMM instead of the register-fragment one
    int mt_mfma = 1;      // 0: batch 1-4 of the CDNA4 layout on the VALU kernel instead of MFMA
    int mt_parts = 0;     // > 0: the batch 1-4 MFMA kernel's column parts per workgroup
    int mt_slabs = 0;     // > 0: its slabs per workgroup (when the columns are not split)
    int mt_spw = 0;       // > 0: its super-blocks per wave (more workgroups per slab)
    int block_fused = 1;  // 0: the decode FFN block as two launches instead of one
    int block_spin = 0;   // > 0: that launch's bound on a down workgroup's wait (polls)
    int gemm_rs = 1;      // 0: split-K FP16-mode GEMMs finish by the last arrival; > 1: reduce-scatter wait bound
    int wait_free = 0;    // 1 (ns_ctx_set_wait_free): no kernel waits for another workgroup
    int stack_fused = 1;  // 0: the multi-layer decode as one block launch per layer
};

// Whether a launch may use a cross-workgroup wait at all (the GPU is not declared shared).
inline bool waits_allowed(const Tuning &t) { return t.wait_free == 0; }

// Kernels whose workgroups wait for each other (the split-K reduce-scatter of the prefill
// GEMMs, the one-launch decode block, the multi-layer decode launch) bound every wait.  A
// workgroup whose bound runs out ORs its kernel's bit into the caller's sticky status word,
// writes its results as NaN and goes on, so the kernel still ends; the host reports the word
// as an error (ns_ctx_status, ns_noalloc_status).
enum WaitBit : uint32_t { kWaitGemm = 1u, kWaitBlock = 2u, kWaitStack = 4u };

__device__ __forceinline__ void record_wait_timeout(uint32_t *err, uint32_t bit) {
    if (err) __hip_atomic_fetch_or(err, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The error text for a non-zero status word.
std::string wait_status_message(uint32_t v);

// Workspace owned by ns_ctx: fp32 partial sums and per-slab arrival counters
// for reductions that span workgroups, the sticky status word of timed-out waits
// (device-visible; nullptr records nothing), and the context's tuning.  Counters are
// zero between calls (the last workgroup of a slab resets its counter).
struct Workspace {
    float *partial = nullptr;
    size_t partial_floats = 0;
    uint32_t *counters = nullptr;
    size_t counter_count = 0;
    uint32_t *err = nullptr;
    Tuning tune;
};

// The RMSNorm ahead of the FFN (rms: metal:510-511, mm:563), applied by a
// decode GEMV to its input: the dot products take xn = (x * r) * wb with
// r = 1/sqrt(mean(x^2) + eps).
struct NormPrologue {
    const float *x = nullptr, *wb = nullptr;
    float eps = 0.f;
};

// Decode GEMV: out[r] = sum_k W[r,k] x[k] (fp32).  With `up` non-null, the
// gate/up pair with the GeGLU epilogue (out = h).  With `np` non-null (the
// gate/up pair only), x is ignored and the dot products take np's normalised
// vector.  Returns a hipError_t.
hipError_t launch_gemv(int type, int layout, const uint8_t *w, const uint8_t *up,
                       const float *x, float *out, uint32_t cols, uint32_t rows,
                       const Workspace &ws, hipStream_t stream, const NormPrologue *np = nullptr);

// Required workspace for launch_gemv with these shapes.
void gemv_workspace_need(int type, int layout, uint32_t cols, uint32_t rows, bool pair, const Tuning &t,
                         size_t *partial_floats, size_t *counters);

// Batch 2-4 (the reference's mm_fast / gate_up_geglu_mm regime): the weights
// are streamed once for all tokens.  x: [batch][cols], fp16 (xh) or fp32;
// out: [batch][rows], fp32, or fp16 h for the gate/up pair (up non-null, fp16 x).
hipError_t launch_gemv_mt(int type, int layout, const uint8_t *w, const uint8_t *up, const void *x, bool xh,
                          uint32_t batch, void *out, uint32_t cols, uint32_t rows, const Workspace &ws,
                          hipStream_t stream);
// Device buffers of the one-launch decode block and the multi-layer decode launch that outlive
// a call, owned by the context: the epoch (a counter each launch advances, so that values an
// earlier launch left carry no current tag; starts at 1) and the tagged copies of h [ffn] and
// y [cols], and the down projection's tagged column parts [ffn] (64-bit words, zero at
// allocation).
struct StackBuffers {
    uint32_t *epoch = nullptr;
    uint64_t *htag = nullptr, *ytag = nullptr, *ptag = nullptr;
    uint32_t cols = 0, ffn = 0;
};
// The decode FFN block in one launch (gate/up + GeGLU into h, then down into y), CDNA4
// layout, shapes with (ffn/256) a multiple of (cols/256) <= 16.  normw non-null folds the
// RMSNorm of x (weight normw, eps) into the gate/up dot products.  y may alias x; h may not.
bool block_decode_supported(int layout, int down_type, bool norm, uint32_t cols, uint32_t ffn);
void block_decode_workspace_need(uint32_t cols, uint32_t ffn, size_t *partial_floats, size_t *counters);
hipError_t launch_block_decode(int down_type, const uint8_t *wg, const uint8_t *wu, const uint8_t *wd, const float *x,
                               const float *normw, float eps, float *h, float *y, uint32_t cols, uint32_t ffn,
                               const Workspace &ws, const StackBuffers &sb, hipStream_t stream);

// The decode FFN blocks of n_layers consecutive layers in one launch (x_{l+1} = y_l, y updated in
// place), CDNA4 layout, shapes with (ffn/256) a multiple of (cols/256) < 16.  normw non-null:
// layer l folds the RMSNorm of its input (weight normw[l], eps) into its gate/up dot products.
// Host arrays of device pointers; down_types[l] is Q4_K or Q6_K.
bool stack_decode_supported(int layout, bool norm, uint32_t cols, uint32_t ffn);
void stack_decode_workspace_need(uint32_t cols, uint32_t ffn, size_t *partial_floats, size_t *counters);
hipError_t launch_stack_decode(uint32_t n_layers, const uint8_t *const *wg, const uint8_t *const *wu,
                               const uint8_t *const *wd, const int *down_types, const float *x,
                               const float *const *normw, float eps, float *h, float *y, uint32_t cols, uint32_t ffn,
                               const Workspace &ws, const StackBuffers &sb, hipStream_t stream);

// Batch 1-4 on the matrix cores (ns_gemv_mfma.hip), CDNA4 layout; launch_gemv_mt routes there
// when gemv_mfma_eligible.
bool gemv_mfma_eligible(int layout, bool pair, bool xh, uint32_t batch, const Tuning &t);
void gemv_mfma_workspace_need(uint32_t cols, uint32_t rows, bool pair, const Tuning &t, size_t *partial_floats,
                              size_t *counters);
hipError_t launch_gemv_mfma(int type, const uint8_t *w, const uint8_t *up, const void *x, bool xh, uint32_t batch,
                            void *out, uint32_t cols, uint32_t rows, const Workspace &ws, hipStream_t stream);

void gemv_mt_workspace_need(int type, int layout, uint32_t cols, uint32_t rows, bool pair, uint32_t batch, bool xh,
                            const Tuning &t, size_t *partial_floats, size_t *counters);

// Workspace the prefill GEMM needs: Q4_K group sums of x, split-K parts, tile counters.
void gemm_workspace_need(int type, int layout, uint32_t cols, uint32_t rows, uint32_t batch, bool pair,
                         const Tuning &t, size_t *floats, size_t *counters);

// What the FP32-mode Q4_K prefill GEMMs read beside x, written by the group-sums
// kernel, at float offsets from one base (each part starts on a 256-byte boundary):
//   sums   two fp16 planes [batch][cols/32]: hi and lo of the 32-wide group sums of x
//   tfac   [batch] fp32: 2^k_t, token t's sums and copied row being those of x_t * 2^-k_t
//   gflag  [ceil(batch/8)] u32: 1 if any token of that 8-row group has k_t > 0
//   bflag  [ceil(batch/256)] u32: 1 if any 8-row group of that 256-token block is flagged
//   xcopy  [batch][cols] fp16: x_t * 2^-k_t for every token of a flagged 256-token block
// A group sum of 32 fp16 values reaches 32 * 65504; k_t (0 unless token t has a group sum
// beyond 65504) keeps the fp16 hi of every sum finite.  A GEMM token tile lies inside one
// 256-token block; in a flagged block it reads x from xcopy and multiplies its tokens'
// outputs by tfac.
struct XsLayout {
    size_t sums, tfac, gflag, bflag, xcopy, total;
};
__host__ __device__ inline XsLayout xs_layout(uint32_t cols, uint32_t batch) {
    auto up64 = [](size_t n) { return (n + 63) / 64 * 64; };
    XsLayout l;
    l.sums = 0;
    l.tfac = up64(size_t(batch) * (cols / 32));
    l.gflag = l.tfac + up64(batch);
    l.bflag = l.gflag + up64((size_t(batch) + 7) / 8);
    l.xcopy = l.bflag + up64((size_t(batch) + 255) / 256);
    l.total = l.xcopy + up64((size_t(batch) * cols + 1) / 2);
    return l;
}

// The Q4_K CDNA4 prefill GEMM with register-resident weight fragments, FP32 mode
// (ns_gemm_reg.hip): split-K parts it needs, and the launch.  xsums: the base of the
// XsLayout block; partial: the split-K parts.
void gemm_reg_workspace_need(uint32_t cols, uint32_t rows, uint32_t batch, bool pair, const Tuning &t,
                             size_t *part_floats, size_t *counters);
hipError_t launch_gemm_reg(const uint8_t *w, const uint8_t *up, const uint16_t *x, const uint16_t *xsums,
                           void *out, uint32_t cols, uint32_t rows, uint32_t batch, float *partial,
                           uint32_t *counters, uint32_t *err, const Tuning &t, hipStream_t stream);

// The FP16-mode prefill GEMM on the CDNA4 layout (ns_gemm_f16.hip): fp16 weight
// tiles with per-row power-of-two scales (ns_tile16.hpp), no x group sums.
void gemm_f16_workspace_need(uint32_t cols, uint32_t rows, uint32_t batch, bool pair, const Tuning &t,
                             size_t *part_floats, size_t *counters);
hipError_t launch_gemm_f16(int type, const uint8_t *w, const uint8_t *up, const uint16_t *x, void *out, uint32_t cols,
                           uint32_t rows, uint32_t batch, float *partial, uint32_t *counters, uint32_t *err,
                           const Tuning &t, hipStream_t stream);

// Prefill GEMM over fp16 x [batch][cols]: plain (fp32 out [batch][rows]) or the
// gate/up pair with GeGLU (fp16 h [batch][rows]).
hipError_t launch_gemm(int type, int layout, int acc, const uint8_t *w, const uint8_t *up,
                       const uint16_t *x, void *out, uint32_t cols, uint32_t rows,
                       uint32_t batch, const Workspace &ws, hipStream_t stream);

hipError_t launch_dequant(int type, int layout, const uint8_t *w, uint32_t cols, uint32_t rows,
                          uint32_t row0, uint32_t nrows, float *out_f32, uint16_t *out_f16,
                          hipStream_t stream);

// Row-wise RMSNorm family (metal:509-529), one workgroup per row of `width`:
//   y = (x * r) * w                                 (residual == nullptr)
//   y = (residual + (x * r) * w) [* *scale]         (residual != nullptr; fp32 y)
// r = rsqrt(mean(x^2) + eps).  With next_w non-null, also next = (y * r2) * next_w,
// r2 = rsqrt(mean(y^2) + eps) (rms_add_then_f16 and its fp32 form).  half_y / half_next
// select fp16 outputs.
hipError_t launch_rmsnorm(const float *x, const float *w, const float *residual, const float *scale,
                          const float *next_w, uint32_t rows, uint32_t width, float eps, void *y, bool half_y,
                          void *next, bool half_next, hipStream_t stream);

// gemma_geglu[_f16] (metal:530-531): y[i] = gelu_tanh(g[i]) * u[i], fp32 or fp16 y; g and u
// 16-byte aligned.
hipError_t launch_geglu(const float *g, const float *u, uint64_t n, void *y, bool half_out, hipStream_t stream);

// y[i] = fp16(x[i]), round to nearest even; x 16-byte and y 8-byte aligned.
hipError_t launch_f32_to_f16(const float *x, uint16_t *y, size_t n, hipStream_t stream);

// out[t][i] = scale * W[ids[t]][i] (fp32 values as quant.cpp; NaN rows for ids out of range).
hipError_t launch_embedding(int type, int layout, const uint8_t *w, uint32_t cols, uint32_t rows, const int32_t *ids,
                            uint32_t batch, float scale, float *out, hipStream_t stream);

hipError_t launch_retile(int type, const uint8_t *src, uint8_t *dst, uint32_t cols,
                         uint32_t rows, int from_layout, int to_layout, hipStream_t stream);

}  // namespace ns
