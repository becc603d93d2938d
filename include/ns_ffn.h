/*
 * ns_ffn.h -- C ABI of the MI355X-native quantised FFN path (libnsffn.so).
 *
 * Drop-in for the FFN matmul call surface of the reference engine
 * (src/native/metal_engine.mm, "mm" below): the Q4_K/Q6_K dequant-fused GEMV
 * and GEMM behind the Gemma-4 gate/up projections, GeGLU, the down projection
 * and the Q6_K lm-head.  Plain pointers and sizes only.
 *
 * Conventions
 *   - `cols` = K = GGUF shape[0], `rows` = N = GGUF shape[1] (mm:268).
 *   - Inputs are row-major [batch][cols], outputs [batch][rows] (mm:41-42 args).
 *   - Weight pointers point at the first byte of the tensor in device memory
 *     (the reference binds the whole .nsmffn file plus a byte offset, mm:267;
 *     here the caller adds the offset).  Q4_K tensors must be 16-byte aligned,
 *     Q6_K tensors 4-byte aligned.
 *   - Every device entry point is stream-ordered on `stream` (a hipStream_t,
 *     NULL = the null stream) and never synchronises.
 *   - Every function returns NS_OK (0) or an error code; ns_last_error() gives
 *     the message of the last failure on the calling thread.  The C++ wrapper
 *     (neutron-star_amd/host/ffn_path.hpp) rethrows it as std::runtime_error,
 *     which is how the reference reports failures (mm:231-243).
 *   - A context owns the workspace used for split reductions (and the fp16 copy
 *     of an fp32 matmul input above batch 4).  Calls that share
 *     one context must be ordered (one stream, or synchronised); the reference
 *     serialises all GPU work the same way (mm:137).
 *   - Co-residency.  Three kernels let workgroups wait for other workgroups of the same
 *     launch: the split-K reduce-scatter finish of the prefill GEMMs (ns_matmul above batch
 *     4, ns_gate_up_geglu above batch 4, ns_gate_up_geglu_rm32, ns_ffn_down with fp16 input
 *     above batch 4, ns_qkv above batch 4), the one-launch decode block
 *     (ns_ffn_block_decode) and the multi-layer decode launch (ns_ffn_stack_decode).  Each
 *     is launched only when its whole grid fits on the device at once, which guarantees
 *     progress while nothing else occupies the GPU's compute units.  Work of another stream,
 *     context or process that holds CUs (in particular a second such kernel launched at the
 *     same time) can keep part of a grid from being dispatched; every wait is bounded
 *     (seconds), and a wait that runs out writes that call's affected outputs as NaN and sets
 *     the context's status word, which ns_ctx_status reports as NS_ERR_TIMEOUT.  An engine
 *     that shares the GPU calls ns_ctx_set_wait_free(ctx, 1): the same results (bit for bit
 *     in the FP32 mode) from launches that never wait.
 */
#ifndef NS_FFN_H
#define NS_FFN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NS_FFN_ABI_VERSION 1

/* Tensor types: the GGUF ids of include/neutron/native/gguf.hpp:13. */
enum { NS_TYPE_Q4_K = 12, NS_TYPE_Q6_K = 14 };

/* Byte layouts of a quantised [rows][cols] tensor.
 *   ROW_MAJOR  GGUF order (src/native/quant.cpp:20, block = element/256).
 *   NSMFFN     the reference's 64-row slab order (src/native/metal_ffn.cpp:135-149).
 *   CDNA4      NSMFFN re-tiled into 16-byte chunks per row, lossless (ns_retile). */
enum { NS_LAYOUT_ROW_MAJOR = 0, NS_LAYOUT_NSMFFN = 1, NS_LAYOUT_CDNA4 = 2 };

/* Accumulation mode of the prefill GEMMs (mm:565 `fast_swa_ffn`).
 *   FP32  fp32 accumulation of exact products (the 8 global layers, and every
 *         layer with --exact-ffn).
 *   FP16  the local-layer mode: the weights enter as fp16 tiles, the reference's
 *         half(d*sc*q - dmin*m) / half(d*sc*(v-32)) times a power of two per
 *         weight row (which keeps small blocks out of fp16's subnormals); the
 *         products are summed in fp32, and each output is rounded once to fp16
 *         precision (11 significant bits, round to nearest even, fp32 exponent
 *         range), whatever the summation order or split. */
enum { NS_ACC_FP32 = 0, NS_ACC_FP16 = 1 };

enum {
    NS_OK = 0,
    NS_ERR_ARG = 1,
    NS_ERR_SHAPE = 2,
    NS_ERR_HIP = 3,
    NS_ERR_UNSUPPORTED = 4,
    NS_ERR_IO = 5,      /* file create/read/write/mmap failure */
    NS_ERR_FORMAT = 6,  /* .nsmffn file does not validate */
    NS_ERR_TIMEOUT = 7  /* a bounded cross-workgroup wait ran out (ns_ctx_status) */
};

typedef struct ns_ctx ns_ctx;

const char *ns_last_error(void);
int ns_abi_version(void);

/* Context on HIP device `device`: owns the split-reduction workspace
 * (the engine's workspaces, mm:100-101).  No counterpart function in the
 * reference (the engine constructor does this, mm:90-133).  The workspace is
 * sized at creation for every FFN shape of the reference model (model.cpp:14-19)
 * in every layout up to batch 2048 (config.cpp:124), so those calls never
 * allocate.  Another shape that needs more grows it: new buffers are
 * allocated and the old ones kept until ns_ctx_destroy (queued work and
 * captured graphs may still use them); growth never synchronises and fails
 * with NS_ERR_UNSUPPORTED while the call's stream is capturing a graph. */
int ns_ctx_create(int device, ns_ctx **out);
int ns_ctx_destroy(ns_ctx *ctx);
/* finish_command (mm:231-243: wait for the command buffer, throw if it failed): waits for
 * `stream`, then reports whether any work of this context ran a bounded cross-workgroup
 * wait out since the last report (NS_ERR_TIMEOUT, with the kernel named in ns_last_error();
 * the word is cleared).  Synchronises; not for use under graph capture. */
int ns_ctx_status(ns_ctx *ctx, void *stream);
/* No counterpart in the reference (its GPU is never shared): wait_free != 0 makes every later
 * call of this context use launches in which no workgroup waits for another (the split-K
 * GEMMs finish by the last part to arrive; the decode block and the multi-layer decode run
 * as separate launches), for engines that share the GPU with other work.  Results are
 * unchanged (the same per-row arithmetic and order). */
int ns_ctx_set_wait_free(ns_ctx *ctx, int wait_free);
/* Bytes of device workspace the context holds now. */
int ns_ctx_workspace_bytes(const ns_ctx *ctx, uint64_t *bytes);
/* Test and experiment hook, no counterpart in the reference: overrides one
 * kernel-selection choice of this context.  Keys: "gemv_pf" (-1 plan, 0 / 1
 * force the one-unit / prefetching decode GEMV), "gemv_waves" (> 0: the
 * prefetching GEMV's flattened grid), "gemv_whole" / "gemv_qslab" (0 disables
 * that decode grid), "gemm_kparts" (> 0: split-K parts of the prefill GEMM),
 * "gemm_q4_reg" (0: the LDS-tile Q4_K GEMM), "mt_mfma" (0: batch 1-4 of the
 * CDNA4 layout on the VALU kernel instead of the matrix cores), "mt_parts" /
 * "mt_slabs" / "mt_spw" (> 0: that MFMA kernel's column parts per workgroup,
 * slabs per workgroup, super-blocks per wave), "block_fused" (0: the decode
 * FFN block as two launches), "block_spin" (> 0: the one-launch block's bound on
 * a wait, in polls; tests shorten it to exercise the bound), "gemm_rs" (0: split-K
 * FP16-mode prefill GEMMs finish by the last part to arrive instead of the
 * reduce-scatter; > 1: the reduce-scatter's bound on its wait).  Results stay within
 * the same tolerances; engines leave the defaults. */
int ns_ctx_set_tuning(ns_ctx *ctx, const char *key, int value);

/* NativeMetalEngine::matmul (mm:269-275): out = in . W^T for `batch` tokens.
 *   batch == 1, fp32 input      -> dequant-fused GEMV (decode; lm-head with ROW_MAJOR or CDNA4).
 *   batch 2-4, fp32 or fp16     -> small-batch GEMV streaming the weights once for all tokens
 *                                  (gemma_q4k/q6k_mm_fast[_f16][_metal], metal:125-177, mm:273);
 *                                  on the matrix cores for the CDNA4 layout, FP32 accumulation.
 *   batch  > 4, half_input != 0 -> dequant-into-LDS MFMA GEMM, FP32 accumulation (any layout:
 *                                  the reference's swizzled row-major kernels, metal:263-301,
 *                                  432-478, serve attention tensors that stay row-major).
 *   batch  > 4, fp32 input      -> the same GEMM on x rounded to fp16 (round to nearest even),
 *                                  as the reference's tile loader converts fp32 x to half
 *                                  (metal:235, gemma_q{4,6}k_mma_swizzled, mm:274); the fp16
 *                                  copy lives in the context (grown like the workspace, refused
 *                                  under stream capture); fp32 input must be 16-byte aligned.
 * `in` is fp32 [batch][cols] or, with half_input, fp16 bits [batch][cols]; out fp32 [batch][rows]. */
int ns_matmul(ns_ctx *ctx, const void *w, int type, int layout, uint32_t cols, uint32_t rows,
              uint32_t batch, const void *in, int half_input, float *out, void *stream);

/* No counterpart in the reference: ns_matmul for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops and harnesses that forbid hipMalloc).  The same
 * regimes and kernels as ns_matmul with the default tuning, without a context: the split
 * reductions use a static device scratch array of 16 MiB of parts and 65,536 counters that
 * each GPU holds until the process ends (whether or not it ever calls this function).  A
 * prefill GEMM (batch > 4) whose default split-K plan needs more parts than the array holds
 * runs with one K part (the gemm_kparts 1 tuning of ns_matmul: same kernels, one part per
 * tile, each output within the FP32 tolerance of ns_matmul's); a shape that still needs more
 * fails with NS_ERR_UNSUPPORTED (a Q4_K GEMM needs ~0.53 floats of scratch per input value:
 * up to ~2,000 tokens of the 3840-wide gate/up input, ~500 of the 15360-wide down input; Q6_K
 * none).  fp32 input above batch 4 is refused (its fp16 copy would need a buffer).  Calls
 * that overlap on one GPU share the array and race: order them (one stream).  Allocates
 * nothing, never synchronises, and may be captured into a graph. */
int ns_matmul_noalloc(const void *w, int type, int layout, uint32_t cols, uint32_t rows, uint32_t batch,
                      const void *in, int half_input, float *out, void *stream);
/* ns_ctx_status for ns_matmul_noalloc on the current device: waits for `stream`, then reports
 * (NS_ERR_TIMEOUT) and clears a bounded cross-workgroup wait that ran out in the static
 * scratch's calls since the last report.  Allocates nothing; synchronises. */
int ns_noalloc_status(void *stream);

/* gate_up_geglu_decode (mm:290): h[r] = gelu_tanh(Wg[r].x) * (Wu[r].x), fp32, Q4_K gate/up. */
int ns_gate_up_geglu_decode(ns_ctx *ctx, const void *wg, const void *wu, int layout,
                            uint32_t cols, uint32_t rows, const float *x, float *h,
                            void *stream);

/* gate_up_geglu (mm:281-286): H = gelu_tanh(X.Wg^T) * (X.Wu^T), x and h fp16 bits
 * ([batch][cols], [batch][rows]).  batch <= 4 (MTP verification): the small-batch pair kernel,
 * weights streamed once for all tokens (gemma_q4k_gate_up_geglu_mm_f16[_metal], metal:102-112,
 * mm:282); larger batches: the prefill GEMM in the FP32 mode. */
int ns_gate_up_geglu(ns_ctx *ctx, const void *wg, const void *wu, int layout, uint32_t cols, uint32_t rows,
                     uint32_t batch, const uint16_t *x, uint16_t *h, void *stream);

/* gate_up_geglu_rm32 (mm:288): prefill H = gelu_tanh(X.Wg^T) * (X.Wu^T).
 * x fp16 bits [batch][cols], h fp16 bits [batch][rows]; fast_swa != 0 selects
 * NS_ACC_FP16 (metal:379), 0 selects NS_ACC_FP32 (metal:373). */
int ns_gate_up_geglu_rm32(ns_ctx *ctx, const void *wg, const void *wu, int layout,
                          uint32_t cols, uint32_t rows, uint32_t batch, const uint16_t *x,
                          uint16_t *h, int fast_swa, void *stream);

/* ffn_down (mm:289): with half_input and batch > 4 the prefill GEMM in the mode
 * fast_swa selects (metal:480/486 Q6_K, :385/:391 Q4_K); otherwise ns_matmul. */
int ns_ffn_down(ns_ctx *ctx, const void *w, int type, int layout, uint32_t cols, uint32_t rows,
                uint32_t batch, const void *in, int half_input, int fast_swa, float *out,
                void *stream);

/* Bit-exact check hook: dequantise rows [row0, row0+nrows) to fp32 (quant.cpp:20
 * values) and/or fp16 (RNE of that fp32).
 * Either output may be NULL.  Outputs are [nrows][cols]. */
int ns_dequant(ns_ctx *ctx, const void *w, int type, int layout, uint32_t cols, uint32_t rows,
               uint32_t row0, uint32_t nrows, float *out_f32, uint16_t *out_f16, void *stream);

/* The engine's RMSNorm family around the FFN block (metal:509-529; rms, rms_half, rms_add,
 * rms_add_then_half at mm:291-296, called at mm:563, mm:574, mm:576).  Per row of `width`
 * (`rows` rows), r = 1/sqrt(mean(x^2) + eps):
 *   ns_rmsnorm:          y = (x*r)*weight, fp32 or fp16 bits (half_out): rms / rms_half.
 *   ns_rmsnorm_add:      y = residual + (x*r)*weight, times *scale when scale is non-NULL:
 *                        rms_add (gemma_rmsnorm_add[_scale]).
 *   ns_rmsnorm_add_then: y as ns_rmsnorm_add, then next = (y*r2)*next_weight with r2 taken
 *                        over y, as fp16 bits (half_next: rms_add_then_half) or fp32 (rms_add
 *                        followed by rms, the decode order at mm:563).
 * Device pointers; scale points at one fp32 (a layer's out_scale tensor).  An fp32 y may
 * alias x or residual of the same shape (every element is read before it is written, by the
 * thread that writes it); fp16 outputs and `next` must not overlap any input. */
int ns_rmsnorm(ns_ctx *ctx, const float *x, const float *weight, uint32_t rows, uint32_t width, float eps,
               void *y, int half_out, void *stream);
int ns_rmsnorm_add(ns_ctx *ctx, const float *x, const float *weight, const float *residual, const float *scale,
                   uint32_t rows, uint32_t width, float eps, float *y, void *stream);
int ns_rmsnorm_add_then(ns_ctx *ctx, const float *x, const float *weight, const float *residual,
                        const float *scale, const float *next_weight, uint32_t rows, uint32_t width, float eps,
                        float *y, void *next, int half_next, void *stream);

/* gemma_geglu / gemma_geglu_f16 (metal:530-531; dispatched at mm:568 and mm:570 after two
 * separate gate and up matmuls): out[i] = gelu_tanh(gate[i]) * up[i] for i < count, fp32 out
 * or, with half_out, fp16 bits (round to nearest even).  gate and up 16-byte aligned. */
int ns_geglu(ns_ctx *ctx, const float *gate, const float *up, uint64_t count, void *out, int half_out, void *stream);

/* rms (mm:563, the decode branch) fused into gate_up_geglu_decode (mm:571), one launch:
 * h[r] = gelu_tanh(Wg[r].n) * (Wu[r].n) with n = (x*r)*norm_weight, r = 1/sqrt(mean(x^2) + eps).
 * Q4_K gate/up; cols <= 16384; x and norm_weight 16-byte aligned; fp32 x, h. */
int ns_rms_gate_up_geglu_decode(ns_ctx *ctx, const void *wg, const void *wu, int layout, uint32_t cols,
                                uint32_t rows, const float *x, const float *norm_weight, float eps, float *h,
                                void *stream);

/* The decode FFN block (mm:571-573: gate_up_geglu_decode, then ffn_down) in one launch
 * where the shapes allow it (CDNA4 layout, (ffn/256) a multiple of (cols/256) <= 16, as
 * the model's 3840 / 15360 are), else as those two launches.  No single counterpart in
 * the reference: it is the engine's pair of calls.  h = gelu(Wg.n) * (Wu.n), y = Wd.h,
 * with n = x, or with norm_weight non-null n = (x * r) * norm_weight, r = 1/sqrt(mean(x^2)
 * + eps) (the rms ahead of the FFN, mm:563, as ns_rms_gate_up_geglu_decode).  x fp32
 * [cols], h fp32 [ffn] (written), y fp32 [cols].  At the model's shape the results equal
 * the two launches bit for bit (the same per-row order), elsewhere within their FP32
 * tolerance.  y may alias x; h may not overlap either.  x, norm_weight and h 16-byte
 * aligned.  Calls that overlap on one context race (the launch counts its workgroups in
 * the context's workspace).  The one launch's down workgroups wait for the gate/up rows
 * they read, with a bound of seconds: rows of y whose wait ran out are NaN and the
 * context's status records it (ns_ctx_status; see Co-residency above). */
int ns_ffn_block_decode(ns_ctx *ctx, const void *wg, const void *wu, const void *wd, int down_type, int layout,
                        uint32_t cols, uint32_t ffn, const float *x, const float *norm_weight, float eps, float *h,
                        float *y, void *stream);

/* The decode FFN blocks of n_layers consecutive layers with nothing between them (the engine's
 * per-layer decode FFN, mm:563-573, repeated; BASELINE's 48-layer FFN stack), in one launch where
 * the shapes allow it (as ns_ffn_block_decode, with cols/256 < 16), else one ns_ffn_block_decode
 * per layer.  No single counterpart in the reference.  x_0 = x; for layer l, with n_l = x_l or,
 * when norm_weights is non-null, (x_l * r) * norm_weights[l] (r = 1/sqrt(mean(x_l^2) + eps)):
 * h = gelu(Wg[l].n_l) * (Wu[l].n_l), x_{l+1} = Wd[l].h; y = x_{n_layers}.  wg, wu, wd, down_types
 * and norm_weights are host arrays of n_layers entries (device pointers, NS_TYPE_Q4_K /
 * NS_TYPE_Q6_K); the table is copied at the call.  Results equal n_layers calls of
 * ns_ffn_block_decode bit for bit.  h fp32 [ffn] holds the last layer's h; y may alias x; h may
 * not overlap either.  x, h, y and every norm weight 16-byte aligned.  The launch's workgroups
 * wait for each other within and across layers (see Co-residency): calls that overlap on one
 * context race, and a wait that runs out makes y NaN and sets the context's status. */
int ns_ffn_stack_decode(ns_ctx *ctx, uint32_t n_layers, const void *const *wg, const void *const *wu,
                        const void *const *wd, const int *down_types, int layout, uint32_t cols, uint32_t ffn,
                        const float *x, const float *const *norm_weights, float eps, float *h, float *y,
                        void *stream);

/* gemma_q6k_embedding (metal:503-505; the token embedding at mm:310, scale = sqrt(3840)):
 * out[t][i] = scale * W[ids[t]][i], fp32 [batch][cols], each value as quant.cpp computes it.
 * Q4_K or Q6_K in any layout (the engine may re-tile the embedding for the lm-head GEMV).  An id
 * outside [0, rows) yields a row of NaN (the reference does not check). */
int ns_embedding(ns_ctx *ctx, const void *w, int type, int layout, uint32_t cols, uint32_t rows,
                 const int32_t *ids, uint32_t batch, float scale, float *out, void *stream);

/* qkv (mm:311; gemma_qkv_q4_f16 / _q6v_f16 / _tied_v_f16, metal:442-454): the attention
 * projections of one layer in prefill.  x fp16 bits [batch][cols]; q fp32 [batch][q_rows];
 * k, v fp32 [batch][kv_rows].  wq, wk Q4_K; wv of v_type (Q4_K or Q6_K), or NULL for tied V
 * (V = K).  FP32 accumulation.  batch >= 2 (batch 2-4: the small-batch kernels; larger: the
 * prefill GEMM); any layout, ROW_MAJOR being the reference's (attention weights are not
 * re-laid by .nsmffn). */
int ns_qkv(ns_ctx *ctx, const void *wq, const void *wk, const void *wv, int v_type, int layout, uint32_t cols,
           uint32_t q_rows, uint32_t kv_rows, uint32_t batch, const uint16_t *x, float *q, float *k, float *v,
           void *stream);

/* ---- host-side (CPU) utilities; no GPU needed ------------------------------ */

/* Convert a host tensor between layouts (a14; the conversion step of
 * tools/convert_metal_ffn.cpp).  src and dst must not overlap.  NSMFFN and
 * CDNA4 need rows % 64 == 0. */
int ns_retile(const void *src, void *dst, int type, uint32_t cols, uint32_t rows,
              int from_layout, int to_layout);

/* Same conversion on device memory, stream-ordered. */
int ns_retile_device(const void *src, void *dst, int type, uint32_t cols, uint32_t rows,
                     int from_layout, int to_layout, void *stream);

/* Seeded synthetic data (this build's generator; configs of BASELINE.json).
 * Blocks [first, first+count) of a tensor with seed `seed`, ROW_MAJOR block
 * order, written contiguously to out (count * 144 or 210 bytes).
 *   Q4_K: d, dmin = fp16(|N(0,1)| * 1e-3); scales[12], qs[128] uniform bytes.
 *   Q6_K: ql[128], qh[64] uniform bytes; scales int8 uniform in -32..31;
 *         d = fp16(|N(0,1)| * 1e-3). */
int ns_synth_blocks(int type, uint64_t seed, uint64_t first, uint64_t count, void *out,
                    int nthreads);
/* N(0,1) values [first, first+count) of stream `seed`, fp32 or fp16 (RNE of the fp32). */
int ns_synth_normal_f32(uint64_t seed, uint64_t first, uint64_t count, float *out, int nthreads);
int ns_synth_normal_f16(uint64_t seed, uint64_t first, uint64_t count, uint16_t *out,
                        int nthreads);
/* Per-layer seed: seed ^ (layer * 0x9E3779B97F4A7C15). */
uint64_t ns_layer_seed(uint64_t seed, uint32_t layer);

/* ---- the .nsmffn v3 weight file (host-side; no GPU needed) -------------------
 *
 * Byte-compatible with the reference's format (include/neutron/native/metal_ffn.hpp:13-40,
 * src/native/metal_ffn.cpp): a 64 KiB header page (72-byte header + one 48-byte entry per
 * GGUF tensor) and every tensor at its GGUF position, FFN tensors re-laid into 64-row slabs. */

/* MetalFfnKind (metal_ffn.hpp:13); NS_FFN_NONE marks a tensor that is not an FFN matrix. */
enum { NS_FFN_GATE = 0, NS_FFN_UP = 1, NS_FFN_DOWN = 2 };
#define NS_FFN_NONE 0xFFFFFFFFu

/* One GGUF tensor, in GGUF tensor-table order (gguf.hpp:20-27 plus the layer/kind
 * that ffn_tensors() assigns from the model, metal_ffn.cpp:63-71). */
typedef struct ns_tensor_desc {
    uint64_t source_offset; /* Tensor::offset: byte offset inside the GGUF data section */
    uint64_t bytes;         /* Tensor::bytes */
    uint32_t type;          /* GGUF type id (NS_TYPE_Q4_K, NS_TYPE_Q6_K, 0 = F32, 1 = F16, ...) */
    uint32_t cols, rows;    /* shape[0], shape[1] (1 for vectors) */
    uint32_t layer;         /* FFN layer index, or NS_FFN_NONE */
    uint32_t kind;          /* NS_FFN_GATE / _UP / _DOWN, or NS_FFN_NONE */
    uint32_t reserved;      /* padding to 40 bytes; ignored */
} ns_tensor_desc;

/* metal_ffn_fingerprint (metal_ffn.cpp:81-90): the FNV-1a 64 loop (prime 1099511628211) from
 * the reference's start value 1469598103934665603 over version 3 (u32 LE), the GGUF file size
 * (u64 LE) and the first min(head_bytes, 16 MiB) bytes of the GGUF, where head_bytes is the
 * GGUF data offset. */
uint64_t ns_nsmffn_fingerprint(const void *gguf_head, uint64_t head_bytes, uint64_t gguf_file_size);

/* convert_metal_ffn (metal_ffn.cpp:92-165): write out_path (via out_path.tmp, fsync, rename)
 * from the GGUF image `gguf` (gguf_size bytes, data section at data_offset). */
int ns_nsmffn_convert(const char *out_path, const void *gguf, uint64_t gguf_size, uint64_t data_offset,
                      const ns_tensor_desc *tensors, uint32_t count);

/* convert_metal_ffn_in_place (metal_ffn.cpp:167-251): re-lay the FFN tensors of the GGUF file
 * model_path slab by slab, save its metadata area as a sparse GGUF at metadata_path, then write
 * the header page over the start of model_path.  Needs data_offset >= 64 KiB. */
int ns_nsmffn_convert_in_place(const char *model_path, const char *metadata_path, uint64_t data_offset,
                               const ns_tensor_desc *tensors, uint32_t count);

/* MetalFfnFile (metal_ffn.cpp:253-311): mmap `path` read-only and validate it against the GGUF
 * it was made from (its size and ns_nsmffn_fingerprint) and its tensor table; NS_ERR_FORMAT
 * with the reference's messages when it does not match. */
typedef struct ns_nsmffn ns_nsmffn;
int ns_nsmffn_open(const char *path, uint64_t gguf_size, uint64_t gguf_fingerprint,
                   const ns_tensor_desc *expected, uint32_t count, ns_nsmffn **out);
int ns_nsmffn_close(ns_nsmffn *f);
const void *ns_nsmffn_data(const ns_nsmffn *f); /* MetalFfnFile::mapped_data */
uint64_t ns_nsmffn_size(const ns_nsmffn *f);    /* MetalFfnFile::file_size */
/* MetalFfnFile::offset and ::reordered of the tensor whose GGUF offset is source_offset. */
int ns_nsmffn_lookup(const ns_nsmffn *f, uint64_t source_offset, uint64_t *offset, int *reordered);

/* ---- GGUF v3 reader (host side; no GPU needed) ----------------------------------------------
 * The engine's GGUF class (gguf.cpp:71-129, gguf.hpp:29-60): ns_gguf_open mmaps `path`
 * read-only and parses the header, metadata and tensor table with the reference's checks and
 * messages (NS_ERR_FORMAT: "bad GGUF magic", "only GGUF v3 is supported", "truncated GGUF
 * header", "invalid GGUF counts", "invalid tensor rank", "invalid quantized tensor shape: <name>",
 * "unsupported tensor type <id>: <name>", "tensor outside GGUF mapping: <name>", ...).  The data
 * section starts at the header's end rounded up to general.alignment (default 32).  prefetch != 0
 * asks the kernel to page the file in (skipped when NEUTRON_NO_SSD_PREFETCH is set). */
typedef struct ns_gguf ns_gguf;
typedef struct ns_gguf_tensor_info {
    const char *name; /* owned by the ns_gguf */
    uint32_t type;    /* GGUF type id: 0 F32, 1 F16, 12 Q4_K, 14 Q6_K */
    uint32_t n_dims;
    uint64_t shape[4];
    uint64_t offset; /* Tensor::offset, from the data section */
    uint64_t bytes;  /* Tensor::bytes */
} ns_gguf_tensor_info;

int ns_gguf_open(const char *path, int prefetch, ns_gguf **out);
int ns_gguf_close(ns_gguf *g);
uint64_t ns_gguf_data_offset(const ns_gguf *g);   /* GGUF::data_offset */
uint64_t ns_gguf_file_size(const ns_gguf *g);     /* GGUF::file_size */
const void *ns_gguf_mapped_data(const ns_gguf *g); /* GGUF::mapped_data */
uint32_t ns_gguf_tensor_count(const ns_gguf *g);  /* GGUF::tensors().size() */
int ns_gguf_tensor(const ns_gguf *g, uint32_t index, ns_gguf_tensor_info *out);
/* GGUF::tensor(name) / has_tensor: "missing tensor: <name>" when absent. */
int ns_gguf_find_tensor(const ns_gguf *g, const char *name, uint32_t *index);
/* GGUF::has, meta_u64 (integers of any width and sign), meta_number (integers or floats),
 * meta<std::string>, and typed arrays (element type as the GGUF value type; data is NULL for
 * string arrays).  "missing GGUF metadata: <key>" / "metadata is not integer: <key>". */
int ns_gguf_has_meta(const ns_gguf *g, const char *key);
int ns_gguf_meta_u64(const ns_gguf *g, const char *key, uint64_t *out);
int ns_gguf_meta_number(const ns_gguf *g, const char *key, double *out);
int ns_gguf_meta_string(const ns_gguf *g, const char *key, const char **out);
int ns_gguf_meta_array(const ns_gguf *g, const char *key, uint32_t *elem_type, uint64_t *count,
                       const void **data);
/* The tensor table for the .nsmffn functions, in GGUF order: each FFN matrix
 * (blk.<i>.ffn_gate / ffn_up / ffn_down.weight, the Gemma4Model names at model.cpp:17) gets its
 * layer and kind, as ffn_tensors() assigns them (metal_ffn.cpp:63-71); every other tensor
 * NS_FFN_NONE.  With out == NULL only *count is set. */
int ns_gguf_ffn_table(const ns_gguf *g, ns_tensor_desc *out, uint32_t capacity, uint32_t *count);

#ifdef __cplusplus
}
#endif
#endif /* NS_FFN_H */
