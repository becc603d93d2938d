// ns_capi.cpp -- the extern "C" boundary (include/ns_ffn.h): argument
// validation, the context/workspace, and regime dispatch mirroring the
// reference engine's helpers (src/native/metal_engine.mm:269-290).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <string>

#include "ns_ffn.h"
#include "ns_internal.hpp"

#include <vector>

struct ns_ctx {
    int device = 0;
    ns::Workspace ws;
    // fp16 copy of an fp32 input for the GEMM (matmul above batch 4 with fp32 input)
    uint16_t *xh = nullptr;
    size_t xh_count = 0;
    // Buffers replaced by workspace growth.  Work queued earlier, or a graph
    // captured earlier, may still use them, so they live until ns_ctx_destroy.
    std::vector<void *> retired;
    // Device word the kernels OR a WaitBit into when a bounded cross-workgroup wait runs out
    // (ws.err points here); read and cleared by ns_ctx_status.
    uint32_t *err = nullptr;
    // The decode block's and the multi-layer decode launch's epoch and tagged h / y (one
    // allocation).
    ns::StackBuffers stack;
    void *stack_mem = nullptr;
};

namespace {
using namespace ns;

int fail(int code, const std::string &msg) {
    set_error(msg);
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(NS_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// The reference accepts cols % 256 == 0 and rows % 64 == 0 (metal_ffn.cpp:74).
int check_tensor(const char *fn, const void *w, int type, int layout, uint32_t cols, uint32_t rows) {
    if (!w) return fail(NS_ERR_ARG, std::string(fn) + ": null weight pointer");
    if (type != Q4_K && type != Q6_K) return fail(NS_ERR_ARG, std::string(fn) + ": type must be Q4_K or Q6_K");
    if (layout != ROW_MAJOR && layout != NSMFFN && layout != CDNA4)
        return fail(NS_ERR_ARG, std::string(fn) + ": unknown layout");
    if (cols == 0 || cols % kQK) return fail(NS_ERR_SHAPE, std::string(fn) + ": cols must be a positive multiple of 256");
    if (rows == 0 || (layout != ROW_MAJOR && rows % kRowTile))
        return fail(NS_ERR_SHAPE, std::string(fn) + ": rows must be a positive multiple of 64 for slab layouts");
    const uintptr_t a = reinterpret_cast<uintptr_t>(w);
    if ((type == Q4_K && a % 16) || (type == Q6_K && a % 4))
        return fail(NS_ERR_ARG, std::string(fn) + ": weight pointer misaligned");
    // The kernels address a tensor through buffer descriptors with a 32-bit byte range.
    if (uint64_t(rows) * (cols / kQK) * block_bytes(type) >= (uint64_t(1) << 31))
        return fail(NS_ERR_SHAPE, std::string(fn) + ": tensor of 2 GiB or more");
    return NS_OK;
}

// Makes the context workspace hold at least this much.  ns_ctx_create sizes it
// for every FFN shape of the reference model up to batch 2048, so growth is for
// other shapes only.  Growth allocates new buffers and retires the old ones
// without freeing them (queued work and captured graphs may still use them), so
// it never synchronises; it is refused while `s` is capturing a graph, where an
// allocation cannot be recorded.
int ensure_ws(ns_ctx *ctx, size_t partial_floats, size_t counters, hipStream_t s) {
    if (partial_floats <= ctx->ws.partial_floats && counters <= ctx->ws.counter_count) return NS_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (s && hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
        return fail(NS_ERR_UNSUPPORTED, "workspace growth during stream capture: run the shape once before capturing");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return hip_fail(e, "workspace growth");
    if (partial_floats > ctx->ws.partial_floats) {
        float *p = nullptr;
        e = hipMalloc(reinterpret_cast<void **>(&p), partial_floats * sizeof(float));
        if (e != hipSuccess) return hip_fail(e, "workspace allocation");
        if (ctx->ws.partial) ctx->retired.push_back(ctx->ws.partial);
        ctx->ws.partial = p;
        ctx->ws.partial_floats = partial_floats;
    }
    if (counters > ctx->ws.counter_count) {
        uint32_t *c = nullptr;
        e = hipMalloc(reinterpret_cast<void **>(&c), counters * sizeof(uint32_t));
        if (e != hipSuccess) return hip_fail(e, "workspace allocation");
        // stream-ordered before the first kernel that counts in it
        e = hipMemsetAsync(c, 0, counters * sizeof(uint32_t), s);
        if (e != hipSuccess) {
            (void)hipFree(c);
            return hip_fail(e, "workspace allocation");
        }
        if (ctx->ws.counters) ctx->retired.push_back(ctx->ws.counters);
        ctx->ws.counters = c;
        ctx->ws.counter_count = counters;
    }
    return NS_OK;
}

// Makes the context's multi-layer decode buffers fit cols x ffn, on the same terms as ensure_ws
// (growth retires the old allocation and is refused during stream capture).  A new allocation is
// zeroed and its epoch set to 1, synchronously: no tag of zeroed memory is ever current.
int ensure_stack(ns_ctx *ctx, uint32_t cols, uint32_t ffn, hipStream_t s) {
    StackBuffers &sb = ctx->stack;
    if (sb.epoch && cols <= sb.cols && ffn <= sb.ffn) return NS_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (s && hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
        return fail(NS_ERR_UNSUPPORTED, "decode buffer growth during stream capture: run the shape once before capturing");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return hip_fail(e, "decode buffer growth");
    const uint32_t c = std::max(cols, sb.cols), f = std::max(ffn, sb.ffn);
    const size_t bytes = 256 + (2 * size_t(f) + c) * sizeof(uint64_t);
    void *p = nullptr;
    e = hipMalloc(&p, bytes);
    if (e == hipSuccess) e = hipMemset(p, 0, bytes);
    const uint32_t one = 1;
    if (e == hipSuccess) e = hipMemcpy(p, &one, sizeof one, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        if (p) (void)hipFree(p);
        return hip_fail(e, "decode buffer allocation");
    }
    if (ctx->stack_mem) ctx->retired.push_back(ctx->stack_mem);
    ctx->stack_mem = p;
    sb.epoch = static_cast<uint32_t *>(p);
    sb.htag = reinterpret_cast<uint64_t *>(static_cast<char *>(p) + 256);
    sb.ytag = sb.htag + f;
    sb.ptag = sb.ytag + c;
    sb.cols = c;
    sb.ffn = f;
    return NS_OK;
}

// Makes the context's fp16 input buffer hold at least n values, on the same terms as
// ensure_ws (growth retires the old buffer and is refused during stream capture).
int ensure_xh(ns_ctx *ctx, size_t n, hipStream_t s) {
    if (n <= ctx->xh_count) return NS_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (s && hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
        return fail(NS_ERR_UNSUPPORTED, "input buffer growth during stream capture: run the shape once before capturing");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return hip_fail(e, "input buffer growth");
    uint16_t *p = nullptr;
    e = hipMalloc(reinterpret_cast<void **>(&p), n * sizeof(uint16_t));
    if (e != hipSuccess) return hip_fail(e, "input buffer allocation");
    if (ctx->xh) ctx->retired.push_back(ctx->xh);
    ctx->xh = p;
    ctx->xh_count = n;
    return NS_OK;
}

// Workspace every FFN call of the reference model needs (model.cpp:14-19: gate/up
// 15360 x 3840 Q4_K, down 3840 x 15360 Q4_K or Q6_K, lm-head 262144 x 3840 Q6_K) in
// every layout, for every batch the engine allows (1..2048, config.cpp:124).
void model_workspace_need(const Tuning &t, size_t *floats, size_t *counters) {
    size_t pf = 0, nc = 0;
    auto take = [&](size_t f, size_t c) {
        pf = std::max(pf, f);
        nc = std::max(nc, c);
    };
    struct Shape {
        int type;
        uint32_t cols, rows;
        bool pair;
    };
    const Shape shapes[] = {{Q4_K, 3840, 15360, true}, {Q4_K, 3840, 15360, false}, {Q4_K, 15360, 3840, false},
                            {Q6_K, 15360, 3840, false}, {Q6_K, 3840, 262144, false}};
    for (int layout : {ROW_MAJOR, NSMFFN, CDNA4})
        for (const Shape &sh : shapes) {
            size_t f = 0, c = 0;
            gemv_workspace_need(sh.type, layout, sh.cols, sh.rows, sh.pair, t, &f, &c);
            take(f, c);
            for (uint32_t b = 2; b <= 4; ++b)
                for (bool xh : {false, true}) {
                    if (sh.pair && !xh) continue;
                    gemv_mt_workspace_need(sh.type, layout, sh.cols, sh.rows, sh.pair, b, xh, t, &f, &c);
                    take(f, c);
                }
            if (sh.rows > 16384) continue;  // the lm-head is a decode GEMV
            for (uint32_t b = 5; b <= 2048; ++b) {
                gemm_workspace_need(sh.type, layout, sh.cols, sh.rows, b, sh.pair, t, &f, &c);
                take(f, c);
            }
        }
    size_t f = 0, c = 0;
    block_decode_workspace_need(3840, 15360, &f, &c);
    take(f, c);
    stack_decode_workspace_need(3840, 15360, &f, &c);
    take(f, c);
    *floats = pf;
    *counters = nc;
}

int gemv(ns_ctx *ctx, const char *fn, int type, int layout, const void *w, const void *up, const float *x,
         float *out, uint32_t cols, uint32_t rows, hipStream_t s) {
    size_t pf = 0, nc = 0;
    gemv_workspace_need(type, layout, cols, rows, up != nullptr, ctx->ws.tune, &pf, &nc);
    if (int rc = ensure_ws(ctx, pf, nc, s)) return rc;
    const hipError_t e = launch_gemv(type, layout, static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(up),
                                     x, out, cols, rows, ctx->ws, s);
    return e == hipSuccess ? NS_OK : hip_fail(e, fn);
}

// Batch 2-4: the weights stream once for every token (mm:273, mm:282).
int gemv_mt(ns_ctx *ctx, const char *fn, int type, int layout, const void *w, const void *up, const void *x,
            bool xh, uint32_t batch, void *out, uint32_t cols, uint32_t rows, hipStream_t s) {
    size_t pf = 0, nc = 0;
    gemv_mt_workspace_need(type, layout, cols, rows, up != nullptr, batch, xh, ctx->ws.tune, &pf, &nc);
    if (int rc = ensure_ws(ctx, pf, nc, s)) return rc;
    const hipError_t e = launch_gemv_mt(type, layout, static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(up),
                                        x, xh, batch, out, cols, rows, ctx->ws, s);
    return e == hipSuccess ? NS_OK : hip_fail(e, fn);
}

int gemm(ns_ctx *ctx, const char *fn, int type, int layout, int acc, const void *w, const void *up,
         const uint16_t *x, void *out, uint32_t cols, uint32_t rows, uint32_t batch, hipStream_t s) {
    size_t wf = 0, wc = 0;
    gemm_workspace_need(type, layout, cols, rows, batch, up != nullptr, ctx->ws.tune, &wf, &wc);
    if (int rc = ensure_ws(ctx, wf, wc, s)) return rc;
    const hipError_t e = launch_gemm(type, layout, acc, static_cast<const uint8_t *>(w),
                                     static_cast<const uint8_t *>(up), x, out, cols, rows, batch, ctx->ws, s);
    return e == hipSuccess ? NS_OK : hip_fail(e, fn);
}

}  // namespace

extern "C" int ns_ctx_create(int device, ns_ctx **out) {
    if (!out) return fail(NS_ERR_ARG, "ns_ctx_create: null output");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) return hip_fail(e, "ns_ctx_create");
    if (device < 0 || device >= n) return fail(NS_ERR_ARG, "ns_ctx_create: no such device");
    e = hipSetDevice(device);
    if (e != hipSuccess) return hip_fail(e, "ns_ctx_create");
    auto *ctx = new ns_ctx;
    ctx->device = device;
    // Enough for every FFN shape of the reference model without growth.
    size_t pf = 0, nc = 0;
    model_workspace_need(ctx->ws.tune, &pf, &nc);
    if (int rc = ensure_ws(ctx, pf, std::max(nc, size_t(1) << 16), nullptr)) {
        ns_ctx_destroy(ctx);
        return rc;
    }
    e = hipMalloc(reinterpret_cast<void **>(&ctx->err), 256);
    if (e == hipSuccess) e = hipMemset(ctx->err, 0, 256);
    if (e != hipSuccess) {
        ns_ctx_destroy(ctx);
        return hip_fail(e, "ns_ctx_create: status word");
    }
    ctx->ws.err = ctx->err;
    // the multi-layer decode buffers for the reference model's shape (model.cpp:14-19)
    if (int rc = ensure_stack(ctx, 3840, 15360, nullptr)) {
        ns_ctx_destroy(ctx);
        return rc;
    }
    e = hipDeviceSynchronize();  // the counters' clear has finished before any stream uses them
    if (e != hipSuccess) {
        ns_ctx_destroy(ctx);
        return hip_fail(e, "ns_ctx_create");
    }
    *out = ctx;
    return NS_OK;
}

extern "C" int ns_ctx_workspace_bytes(const ns_ctx *ctx, uint64_t *bytes) {
    if (!ctx || !bytes) return fail(NS_ERR_ARG, "ns_ctx_workspace_bytes: null argument");
    *bytes = uint64_t(ctx->ws.partial_floats) * sizeof(float) + uint64_t(ctx->ws.counter_count) * sizeof(uint32_t);
    return NS_OK;
}

extern "C" int ns_ctx_set_tuning(ns_ctx *ctx, const char *key, int value) {
    if (!ctx || !key) return fail(NS_ERR_ARG, "ns_ctx_set_tuning: null argument");
    Tuning &t = ctx->ws.tune;
    const std::string k(key);
    if (k == "gemv_pf") t.gemv_pf = value;
    else if (k == "gemv_waves") t.gemv_waves = value;
    else if (k == "gemv_whole") t.gemv_whole = value;
    else if (k == "gemv_qslab") t.gemv_qslab = value;
    else if (k == "gemm_kparts") t.gemm_kparts = value;
    else if (k == "gemm_q4_reg") t.gemm_q4_reg = value;
    else if (k == "mt_mfma") t.mt_mfma = value;
    else if (k == "mt_parts") t.mt_parts = value;
    else if (k == "mt_slabs") t.mt_slabs = value;
    else if (k == "mt_spw") t.mt_spw = value;
    else if (k == "block_fused") t.block_fused = value;
    else if (k == "block_spin") t.block_spin = value;
    else if (k == "gemm_rs") t.gemm_rs = value;
    else if (k == "stack_fused") t.stack_fused = value;
    else return fail(NS_ERR_ARG, "ns_ctx_set_tuning: unknown key " + k);
    return NS_OK;
}

extern "C" int ns_ctx_destroy(ns_ctx *ctx) {
    if (!ctx) return NS_OK;
    (void)hipSetDevice(ctx->device);
    (void)hipDeviceSynchronize();
    if (ctx->ws.partial) (void)hipFree(ctx->ws.partial);
    if (ctx->ws.counters) (void)hipFree(ctx->ws.counters);
    if (ctx->xh) (void)hipFree(ctx->xh);
    if (ctx->err) (void)hipFree(ctx->err);
    if (ctx->stack_mem) (void)hipFree(ctx->stack_mem);
    for (void *p : ctx->retired) (void)hipFree(p);
    delete ctx;
    return NS_OK;
}

namespace ns {
// Text of a non-zero status word (WaitBit flags).
std::string wait_status_message(uint32_t v) {
    std::string which;
    const auto add = [&](uint32_t bit, const char *name) {
        if (!(v & bit)) return;
        if (!which.empty()) which += ", ";
        which += name;
    };
    add(kWaitGemm, "a prefill GEMM's split-K reduce-scatter");
    add(kWaitBlock, "the one-launch decode FFN block");
    add(kWaitStack, "the multi-layer decode launch");
    return "a cross-workgroup wait ran out in " + which +
           ": some outputs of that call are NaN (its workgroups were not all resident at once; run with "
           "ns_ctx_set_wait_free when other work shares the GPU)";
}
}  // namespace ns

extern "C" int ns_ctx_status(ns_ctx *ctx, void *stream) {
    if (!ctx) return fail(NS_ERR_ARG, "ns_ctx_status: null context");
    hipError_t e = hipSetDevice(ctx->device);
    uint32_t v = 0;
    if (e == hipSuccess) e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (e == hipSuccess) e = hipMemcpy(&v, ctx->err, sizeof v, hipMemcpyDeviceToHost);
    if (e == hipSuccess && v != 0) e = hipMemset(ctx->err, 0, sizeof v);
    if (e != hipSuccess) return hip_fail(e, "ns_ctx_status");
    return v == 0 ? NS_OK : fail(NS_ERR_TIMEOUT, "ns_ctx_status: " + ns::wait_status_message(v));
}

extern "C" int ns_ctx_set_wait_free(ns_ctx *ctx, int wait_free) {
    if (!ctx) return fail(NS_ERR_ARG, "ns_ctx_set_wait_free: null context");
    ctx->ws.tune.wait_free = wait_free != 0 ? 1 : 0;
    return NS_OK;
}

extern "C" int ns_matmul(ns_ctx *ctx, const void *w, int type, int layout, uint32_t cols, uint32_t rows,
                         uint32_t batch, const void *in, int half_input, float *out, void *stream) {
    if (!ctx) return fail(NS_ERR_ARG, "ns_matmul: null context");
    if (int rc = check_tensor("ns_matmul", w, type, layout, cols, rows)) return rc;
    if (!in || !out || batch == 0) return fail(NS_ERR_ARG, "ns_matmul: null input/output or zero batch");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // mm:269-275: batch 2-4 -> the small-batch kernels (fp32 or fp16 input); batch > 4 -> the
    // MMA (prefill) GEMM
    if (batch >= 2 && batch <= 4)
        return gemv_mt(ctx, "ns_matmul", type, layout, w, nullptr, in, half_input != 0, batch, out, cols, rows, s);
    if (half_input && batch > 1)
        return gemm(ctx, "ns_matmul", type, layout, ACC_FP32, w, nullptr, static_cast<const uint16_t *>(in), out,
                    cols, rows, batch, s);
    if (half_input) return fail(NS_ERR_UNSUPPORTED, "ns_matmul: fp16 input at batch 1 is not a reference regime");
    const auto *x = static_cast<const float *>(in);
    if (batch == 1) return gemv(ctx, "ns_matmul", type, layout, w, nullptr, x, out, cols, rows, s);
    // mm:274: fp32 input above batch 4 takes the MMA GEMM too, whose tile loader rounds each x
    // value to half (metal:235): x to fp16 (round to nearest even), then the prefill GEMM in
    // the FP32 mode
    if (reinterpret_cast<uintptr_t>(x) % 16) return fail(NS_ERR_ARG, "ns_matmul: fp32 input must be 16-byte aligned");
    const size_t n = size_t(batch) * cols;
    if (int rc = ensure_xh(ctx, n, s)) return rc;
    const hipError_t e = launch_f32_to_f16(x, ctx->xh, n, s);
    if (e != hipSuccess) return hip_fail(e, "ns_matmul");
    return gemm(ctx, "ns_matmul", type, layout, ACC_FP32, w, nullptr, ctx->xh, out, cols, rows, batch, s);
}

extern "C" int ns_gate_up_geglu_decode(ns_ctx *ctx, const void *wg, const void *wu, int layout, uint32_t cols,
                                       uint32_t rows, const float *x, float *h, void *stream) {
    if (!ctx) return fail(NS_ERR_ARG, "ns_gate_up_geglu_decode: null context");
    if (int rc = check_tensor("ns_gate_up_geglu_decode", wg, Q4_K, layout, cols, rows)) return rc;
    if (int rc = check_tensor("ns_gate_up_geglu_decode", wu, Q4_K, layout, cols, rows)) return rc;
    if (!x || !h) return fail(NS_ERR_ARG, "ns_gate_up_geglu_decode: null input/output");
    return gemv(ctx, "ns_gate_up_geglu_decode", Q4_K, layout, wg, wu, x, h, cols, rows,
                static_cast<hipStream_t>(stream));
}

extern "C" int ns_gate_up_geglu(ns_ctx *ctx, const void *wg, const void *wu, int layout, uint32_t cols,
                                uint32_t rows, uint32_t batch, const uint16_t *x, uint16_t *h, void *stream) {
    if (!ctx) return fail(NS_ERR_ARG, "ns_gate_up_geglu: null context");
    if (int rc = check_tensor("ns_gate_up_geglu", wg, Q4_K, layout, cols, rows)) return rc;
    if (int rc = check_tensor("ns_gate_up_geglu", wu, Q4_K, layout, cols, rows)) return rc;
    if (!x || !h || batch == 0) return fail(NS_ERR_ARG, "ns_gate_up_geglu: null input/output or zero batch");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // mm:282: batch <= 4 -> the small-batch pair kernel; larger batches -> the prefill GEMM (FP32 mode)
    if (batch <= 4) return gemv_mt(ctx, "ns_gate_up_geglu", Q4_K, layout, wg, wu, x, true, batch, h, cols, rows, s);
    return gemm(ctx, "ns_gate_up_geglu", Q4_K, layout, ACC_FP32, wg, wu, x, h, cols, rows, batch, s);
}

extern "C" int ns_gate_up_geglu_rm32(ns_ctx *ctx, const void *wg, const void *wu, int layout, uint32_t cols,
                                     uint32_t rows, uint32_t batch, const uint16_t *x, uint16_t *h, int fast_swa,
                                     void *stream) {
    if (!ctx) return fail(NS_ERR_ARG, "ns_gate_up_geglu_rm32: null context");
    if (int rc = check_tensor("ns_gate_up_geglu_rm32", wg, Q4_K, layout, cols, rows)) return rc;
    if (int rc = check_tensor("ns_gate_up_geglu_rm32", wu, Q4_K, layout, cols, rows)) return rc;
    if (!x || !h || batch == 0) return fail(NS_ERR_ARG, "ns_gate_up_geglu_rm32: null input/output or zero batch");
    return gemm(ctx, "ns_gate_up_geglu_rm32", Q4_K, layout, fast_swa ? ACC_FP16 : ACC_FP32, wg, wu, x, h, cols,
                rows, batch, static_cast<hipStream_t>(stream));
}

extern "C" int ns_ffn_down(ns_ctx *ctx, const void *w, int type, int layout, uint32_t cols, uint32_t rows,
                           uint32_t batch, const void *in, int half_input, int fast_swa, float *out, void *stream) {
    if (!ctx) return fail(NS_ERR_ARG, "ns_ffn_down: null context");
    if (half_input && batch > 4) {  // mm:289; batches up to 4 take matmul's small-batch kernels
        if (int rc = check_tensor("ns_ffn_down", w, type, layout, cols, rows)) return rc;
        if (!in || !out) return fail(NS_ERR_ARG, "ns_ffn_down: null input/output");
        return gemm(ctx, "ns_ffn_down", type, layout, fast_swa ? ACC_FP16 : ACC_FP32, w, nullptr,
                    static_cast<const uint16_t *>(in), out, cols, rows, batch, static_cast<hipStream_t>(stream));
    }
    return ns_matmul(ctx, w, type, layout, cols, rows, batch, in, half_input, out, stream);
}

extern "C" int ns_dequant(ns_ctx *ctx, const void *w, int type, int layout, uint32_t cols, uint32_t rows,
                          uint32_t row0, uint32_t nrows, float *out_f32, uint16_t *out_f16, void *stream) {
    if (!ctx) return fail(NS_ERR_ARG, "ns_dequant: null context");
    if (int rc = check_tensor("ns_dequant", w, type, layout, cols, rows)) return rc;
    if (uint64_t(row0) + nrows > rows) return fail(NS_ERR_SHAPE, "ns_dequant: row range out of bounds");
    const hipError_t e = launch_dequant(type, layout, static_cast<const uint8_t *>(w), cols, rows, row0, nrows,
                                        out_f32, out_f16, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? NS_OK : hip_fail(e, "ns_dequant");
}

extern "C" int ns_retile_device(const void *src, void *dst, int type, uint32_t cols, uint32_t rows, int from_layout,
                                int to_layout, void *stream) {
    if (int rc = check_tensor("ns_retile_device", src, type, from_layout, cols, rows)) return rc;
    if (int rc = check_tensor("ns_retile_device", dst, type, to_layout, cols, rows)) return rc;
    if (src == dst) return fail(NS_ERR_ARG, "ns_retile_device: in-place conversion is not supported");
    const hipError_t e = launch_retile(type, static_cast<const uint8_t *>(src), static_cast<uint8_t *>(dst), cols,
                                       rows, from_layout, to_layout, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? NS_OK : hip_fail(e, "ns_retile_device");
}

extern "C" int ns_rmsnorm(ns_ctx *ctx, const float *x, const float *weight, uint32_t rows, uint32_t width, float eps,
                          void *y, int half_out, void *stream) {
    if (!ctx) return fail(NS_ERR_ARG, "ns_rmsnorm: null context");
    if (!x || !weight || !y || rows == 0 || width == 0) return fail(NS_ERR_ARG, "ns_rmsnorm: null buffer or empty shape");
    const hipError_t e = launch_rmsnorm(x, weight, nullptr, nullptr, nullptr, rows, width, eps, y, half_out != 0,
                                        nullptr, false, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? NS_OK : hip_fail(e, "ns_rmsnorm");
}

extern "C" int ns_rmsnorm_add(ns_ctx *ctx, const float *x, const float *weight, const float *residual,
                              const float *scale, uint32_t rows, uint32_t width, float eps, float *y, void *stream) {
    if (!ctx) return fail(NS_ERR_ARG, "ns_rmsnorm_add: null context");
    if (!x || !weight || !residual || !y || rows == 0 || width == 0)
        return fail(NS_ERR_ARG, "ns_rmsnorm_add: null buffer or empty shape");
    const hipError_t e = launch_rmsnorm(x, weight, residual, scale, nullptr, rows, width, eps, y, false, nullptr,
                                        false, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? NS_OK : hip_fail(e, "ns_rmsnorm_add");
}

extern "C" int ns_rmsnorm_add_then(ns_ctx *ctx, const float *x, const float *weight, const float *residual,
                                   const float *scale, const float *next_weight, uint32_t rows, uint32_t width,
                                   float eps, float *y, void *next, int half_next, void *stream) {
    if (!ctx) return fail(NS_ERR_ARG, "ns_rmsnorm_add_then: null context");
    if (!x || !weight || !residual || !next_weight || !y || !next || rows == 0 || width == 0)
        return fail(NS_ERR_ARG, "ns_rmsnorm_add_then: null buffer or empty shape");
    const hipError_t e = launch_rmsnorm(x, weight, residual, scale, next_weight, rows, width, eps, y, false, next,
                                        half_next != 0, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? NS_OK : hip_fail(e, "ns_rmsnorm_add_then");
}

extern "C" int ns_geglu(ns_ctx *ctx, const float *gate, const float *up, uint64_t count, void *out, int half_out,
                        void *stream) {
    if (!ctx) return fail(NS_ERR_ARG, "ns_geglu: null context");
    if (!gate || !up || !out) return fail(NS_ERR_ARG, "ns_geglu: null buffer");
    if ((reinterpret_cast<uintptr_t>(gate) | reinterpret_cast<uintptr_t>(up)) % 16)
        return fail(NS_ERR_ARG, "ns_geglu: gate and up must be 16-byte aligned");
    const hipError_t e = launch_geglu(gate, up, count, out, half_out != 0, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? NS_OK : hip_fail(e, "ns_geglu");
}

namespace {
int rms_gate_up(ns_ctx *ctx, const char *fn, const void *wg, const void *wu, int layout, uint32_t cols,
                uint32_t rows, const NormPrologue &np, float *h, void *stream) {
    if (!ctx) return fail(NS_ERR_ARG, std::string(fn) + ": null context");
    if (int rc = check_tensor(fn, wg, Q4_K, layout, cols, rows)) return rc;
    if (int rc = check_tensor(fn, wu, Q4_K, layout, cols, rows)) return rc;
    if (!np.x || !np.wb || !h) return fail(NS_ERR_ARG, std::string(fn) + ": null input/output");
    if (cols > 16384) return fail(NS_ERR_SHAPE, std::string(fn) + ": cols above 16384 (the LDS copy of x)");
    if ((reinterpret_cast<uintptr_t>(np.x) | reinterpret_cast<uintptr_t>(np.wb)) % 16)
        return fail(NS_ERR_ARG, std::string(fn) + ": x and norm_weight must be 16-byte aligned");
    size_t pf = 0, nc = 0;
    gemv_workspace_need(Q4_K, layout, cols, rows, true, ctx->ws.tune, &pf, &nc);
    if (int rc = ensure_ws(ctx, pf, nc, static_cast<hipStream_t>(stream))) return rc;
    const hipError_t e = launch_gemv(Q4_K, layout, static_cast<const uint8_t *>(wg), static_cast<const uint8_t *>(wu),
                                     nullptr, h, cols, rows, ctx->ws, static_cast<hipStream_t>(stream), &np);
    return e == hipSuccess ? NS_OK : hip_fail(e, fn);
}
}  // namespace

extern "C" int ns_rms_gate_up_geglu_decode(ns_ctx *ctx, const void *wg, const void *wu, int layout, uint32_t cols,
                                           uint32_t rows, const float *x, const float *norm_weight, float eps,
                                           float *h, void *stream) {
    NormPrologue np;
    np.x = x;
    np.wb = norm_weight;
    np.eps = eps;
    return rms_gate_up(ctx, "ns_rms_gate_up_geglu_decode", wg, wu, layout, cols, rows, np, h, stream);
}

extern "C" int ns_ffn_block_decode(ns_ctx *ctx, const void *wg, const void *wu, const void *wd, int down_type,
                                   int layout, uint32_t cols, uint32_t ffn, const float *x, const float *norm_weight,
                                   float eps, float *h, float *y, void *stream) {
    const char *fn = "ns_ffn_block_decode";
    if (!ctx) return fail(NS_ERR_ARG, "ns_ffn_block_decode: null context");
    if (int rc = check_tensor(fn, wg, Q4_K, layout, cols, ffn)) return rc;
    if (int rc = check_tensor(fn, wu, Q4_K, layout, cols, ffn)) return rc;
    if (int rc = check_tensor(fn, wd, down_type, layout, ffn, cols)) return rc;
    if (!x || !h || !y) return fail(NS_ERR_ARG, "ns_ffn_block_decode: null input/output");
    const auto overlap = [](const void *a, size_t na, const void *b, size_t nb) {
        const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
        return pa < pb + nb && pb < pa + na;
    };
    if (overlap(h, ffn * 4, x, cols * 4)) return fail(NS_ERR_ARG, "ns_ffn_block_decode: h overlaps x");
    if (overlap(h, ffn * 4, y, cols * 4)) return fail(NS_ERR_ARG, "ns_ffn_block_decode: h overlaps y");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(norm_weight) | reinterpret_cast<uintptr_t>(h)) % 16)
        return fail(NS_ERR_ARG, "ns_ffn_block_decode: x, norm_weight and h must be 16-byte aligned");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (ctx->ws.tune.block_fused != 0 && waits_allowed(ctx->ws.tune) &&
        block_decode_supported(layout, down_type, norm_weight != nullptr, cols, ffn)) {
        size_t pf = 0, nc = 0;
        block_decode_workspace_need(cols, ffn, &pf, &nc);
        if (int rc = ensure_ws(ctx, pf, nc, s)) return rc;
        if (int rc = ensure_stack(ctx, cols, ffn, s)) return rc;
        const hipError_t e = launch_block_decode(down_type, static_cast<const uint8_t *>(wg),
                                                 static_cast<const uint8_t *>(wu), static_cast<const uint8_t *>(wd), x,
                                                 norm_weight, eps, h, y, cols, ffn, ctx->ws, ctx->stack, s);
        return e == hipSuccess ? NS_OK : hip_fail(e, fn);
    }
    // two launches (mm:571-573): gate/up + GeGLU (with the norm when given), then down
    if (norm_weight) {
        if (int rc = ns_rms_gate_up_geglu_decode(ctx, wg, wu, layout, cols, ffn, x, norm_weight, eps, h, stream)) return rc;
    } else if (int rc = ns_gate_up_geglu_decode(ctx, wg, wu, layout, cols, ffn, x, h, stream)) {
        return rc;
    }
    return ns_matmul(ctx, wd, down_type, layout, ffn, cols, 1, h, 0, y, stream);
}

extern "C" int ns_ffn_stack_decode(ns_ctx *ctx, uint32_t n_layers, const void *const *wg, const void *const *wu,
                                   const void *const *wd, const int *down_types, int layout, uint32_t cols,
                                   uint32_t ffn, const float *x, const float *const *norm_weights, float eps, float *h,
                                   float *y, void *stream) {
    const char *fn = "ns_ffn_stack_decode";
    if (!ctx) return fail(NS_ERR_ARG, "ns_ffn_stack_decode: null context");
    if (n_layers == 0 || !wg || !wu || !wd || !down_types)
        return fail(NS_ERR_ARG, "ns_ffn_stack_decode: no layers or a null weight table");
    if (!x || !h || !y) return fail(NS_ERR_ARG, "ns_ffn_stack_decode: null input/output");
    for (uint32_t l = 0; l < n_layers; ++l) {
        if (int rc = check_tensor(fn, wg[l], Q4_K, layout, cols, ffn)) return rc;
        if (int rc = check_tensor(fn, wu[l], Q4_K, layout, cols, ffn)) return rc;
        if (int rc = check_tensor(fn, wd[l], down_types[l], layout, ffn, cols)) return rc;
        if (norm_weights && (!norm_weights[l] || reinterpret_cast<uintptr_t>(norm_weights[l]) % 16))
            return fail(NS_ERR_ARG, "ns_ffn_stack_decode: each norm weight must be non-null and 16-byte aligned");
    }
    const auto overlap = [](const void *a, size_t na, const void *b, size_t nb) {
        const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
        return pa < pb + nb && pb < pa + na;
    };
    if (overlap(h, ffn * 4, x, cols * 4)) return fail(NS_ERR_ARG, "ns_ffn_stack_decode: h overlaps x");
    if (overlap(h, ffn * 4, y, cols * 4)) return fail(NS_ERR_ARG, "ns_ffn_stack_decode: h overlaps y");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(h)) % 16)
        return fail(NS_ERR_ARG, "ns_ffn_stack_decode: x, h and y must be 16-byte aligned");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (ctx->ws.tune.stack_fused != 0 && waits_allowed(ctx->ws.tune) &&
        stack_decode_supported(layout, norm_weights != nullptr, cols, ffn)) {
        size_t pf = 0, nc = 0;
        stack_decode_workspace_need(cols, ffn, &pf, &nc);
        if (int rc = ensure_ws(ctx, pf, nc, s)) return rc;
        if (int rc = ensure_stack(ctx, cols, ffn, s)) return rc;
        const hipError_t e = launch_stack_decode(n_layers, reinterpret_cast<const uint8_t *const *>(wg),
                                                 reinterpret_cast<const uint8_t *const *>(wu),
                                                 reinterpret_cast<const uint8_t *const *>(wd), down_types, x,
                                                 norm_weights, eps, h, y, cols, ffn, ctx->ws, ctx->stack, s);
        return e == hipSuccess ? NS_OK : hip_fail(e, fn);
    }
    // one block per layer, each continuing from the previous one's y in place
    for (uint32_t l = 0; l < n_layers; ++l)
        if (int rc = ns_ffn_block_decode(ctx, wg[l], wu[l], wd[l], down_types[l], layout, cols, ffn, l == 0 ? x : y,
                                         norm_weights ? norm_weights[l] : nullptr, eps, h, y, stream))
            return rc;
    return NS_OK;
}

extern "C" int ns_embedding(ns_ctx *ctx, const void *w, int type, int layout, uint32_t cols, uint32_t rows,
                            const int32_t *ids, uint32_t batch, float scale, float *out, void *stream) {
    if (!ctx) return fail(NS_ERR_ARG, "ns_embedding: null context");
    if (int rc = check_tensor("ns_embedding", w, type, layout, cols, rows)) return rc;
    if (!ids || !out || batch == 0) return fail(NS_ERR_ARG, "ns_embedding: null ids/output or zero batch");
    const hipError_t e = launch_embedding(type, layout, static_cast<const uint8_t *>(w), cols, rows, ids, batch, scale,
                                          out, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? NS_OK : hip_fail(e, "ns_embedding");
}

extern "C" int ns_qkv(ns_ctx *ctx, const void *wq, const void *wk, const void *wv, int v_type, int layout,
                      uint32_t cols, uint32_t q_rows, uint32_t kv_rows, uint32_t batch, const uint16_t *x, float *q,
                      float *k, float *v, void *stream) {
    const char *fn = "ns_qkv";
    if (!ctx) return fail(NS_ERR_ARG, "ns_qkv: null context");
    if (int rc = check_tensor(fn, wq, Q4_K, layout, cols, q_rows)) return rc;
    if (int rc = check_tensor(fn, wk, Q4_K, layout, cols, kv_rows)) return rc;
    if (wv)
        if (int rc = check_tensor(fn, wv, v_type, layout, cols, kv_rows)) return rc;
    if (!x || !q || !k || !v) return fail(NS_ERR_ARG, "ns_qkv: null input/output");
    if (batch < 2) return fail(NS_ERR_UNSUPPORTED, "ns_qkv: the fused projection is the prefill path (batch >= 2)");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // Q, K and V each stream their own weights once; x (fp16 [batch][cols]) is re-read
    // from the caches.  Batch 2-4 takes the small-batch kernels, larger batches the GEMM.
    auto proj = [&](const void *w, int type, uint32_t rows, float *out) {
        if (batch <= 4) return gemv_mt(ctx, fn, type, layout, w, nullptr, x, true, batch, out, cols, rows, s);
        return gemm(ctx, fn, type, layout, ACC_FP32, w, nullptr, x, out, cols, rows, batch, s);
    };
    if (int rc = proj(wq, Q4_K, q_rows, q)) return rc;
    if (int rc = proj(wk, Q4_K, kv_rows, k)) return rc;
    if (wv) return proj(wv, v_type, kv_rows, v);
    // tied V (gemma_qkv_tied_v_f16, metal:454): V is K
    const hipError_t e = hipMemcpyAsync(v, k, size_t(batch) * kv_rows * sizeof(float), hipMemcpyDeviceToDevice, s);
    return e == hipSuccess ? NS_OK : hip_fail(e, fn);
}
