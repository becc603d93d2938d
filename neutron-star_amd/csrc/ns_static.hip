// ns_static.hip -- ns_matmul_noalloc: ns_matmul without a context, on a static
// device scratch array, for callers that cannot allocate device memory (code
// under HIP graph capture, serving loops that forbid hipMalloc).
//
// The kernels are ns_matmul's own (launch_gemv, launch_gemv_mt, launch_gemm with
// the default tuning); only their workspace differs.  It is `scratch`, a
// file-scope __device__ array of kScratchFloats fp32 parts followed by
// kScratchCounters arrival counters (16 MiB + 256 KiB), which every GPU the
// library runs on holds until the process ends.  Host code never passes the
// array's name to a kernel: on first use on a device, with that device current,
// hipGetSymbolAddress gives the device address, kept per device.  Every call
// on one GPU shares that GPU's array, so calls that overlap on one GPU (two
// streams, or two threads) race; callers order them.  The counters must start
// at zero: each call clears the ones it uses with a small kernel before the
// matmul (stream-ordered, no hipMemsetAsync, so the call can be captured).
// A prefill GEMM whose default plan (split-K parts padded to whole tiles) does not
// fit runs with one K part instead (no parts; only the Q4_K group sums of x), as
// ns_matmul does with the gemm_kparts 1 tuning.  The array also holds a status
// word for bounded cross-workgroup waits that ran out, read by ns_noalloc_status.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "ns_ffn.h"
#include "ns_internal.hpp"

namespace ns {
namespace {

constexpr size_t kScratchFloats = size_t(4) << 20;  // 16 MiB of fp32 parts
constexpr size_t kScratchCounters = size_t(1) << 16;

struct ScratchMem {
    float parts[kScratchFloats];
    uint32_t counters[kScratchCounters];
    uint32_t err[64];  // err[0]: the WaitBit flags of timed-out waits since the last report
};
static __device__ __align__(256) ScratchMem scratch;

constexpr int kMaxDevices = 64;

// Device address of `scratch` per device, looked up once (under a mutex) with that
// device current.
int scratch_address(ScratchMem **out) {
    static std::mutex mu;
    static ScratchMem *addr[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        set_error(std::string("ns_matmul_noalloc: hipGetDevice: ") + hipGetErrorString(e));
        return NS_ERR_HIP;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        set_error("ns_matmul_noalloc: device index above 63");
        return NS_ERR_UNSUPPORTED;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            set_error(std::string("ns_matmul_noalloc: hipGetSymbolAddress: ") + hipGetErrorString(e));
            return NS_ERR_HIP;
        }
        addr[dev] = static_cast<ScratchMem *>(p);
    }
    *out = addr[dev];
    return NS_OK;
}

__global__ void clear_counters(uint32_t *c, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) c[i] = 0u;
}

int fail(int code, const std::string &msg) {
    set_error(msg);
    return code;
}

}  // namespace
}  // namespace ns

extern "C" int ns_matmul_noalloc(const void *w, int type, int layout, uint32_t cols, uint32_t rows, uint32_t batch,
                                 const void *in, int half_input, float *out, void *stream) {
    using namespace ns;
    const char *fn = "ns_matmul_noalloc";
    if (!w || !in || !out || batch == 0) return fail(NS_ERR_ARG, std::string(fn) + ": null argument or zero batch");
    if (type != Q4_K && type != Q6_K) return fail(NS_ERR_ARG, std::string(fn) + ": type must be Q4_K or Q6_K");
    if (layout != ROW_MAJOR && layout != NSMFFN && layout != CDNA4) return fail(NS_ERR_ARG, std::string(fn) + ": unknown layout");
    if (cols == 0 || cols % kQK) return fail(NS_ERR_SHAPE, std::string(fn) + ": cols must be a positive multiple of 256");
    if (rows == 0 || (layout != ROW_MAJOR && rows % kRowTile))
        return fail(NS_ERR_SHAPE, std::string(fn) + ": rows must be a positive multiple of 64 for slab layouts");
    const uintptr_t a = reinterpret_cast<uintptr_t>(w);
    if ((type == Q4_K && a % 16) || (type == Q6_K && a % 4)) return fail(NS_ERR_ARG, std::string(fn) + ": weight pointer misaligned");
    if (uint64_t(rows) * (cols / kQK) * block_bytes(type) >= (uint64_t(1) << 31))
        return fail(NS_ERR_SHAPE, std::string(fn) + ": tensor of 2 GiB or more");
    if (half_input && batch == 1) return fail(NS_ERR_UNSUPPORTED, std::string(fn) + ": fp16 input at batch 1 is not a reference regime");
    if (!half_input && batch > 4) return fail(NS_ERR_UNSUPPORTED, std::string(fn) + ": fp32 input above batch 4 (converted to an fp16 copy before the GEMM, a buffer this entry point does not hold) is not offered");

    // the same regime split and kernels as ns_matmul (mm:269-275)
    Tuning t;
    size_t need_f = 0, need_c = 0;
    const auto fits = [&] { return need_f <= kScratchFloats && need_c <= kScratchCounters; };
    if (batch == 1) gemv_workspace_need(type, layout, cols, rows, false, t, &need_f, &need_c);
    else if (batch <= 4) gemv_mt_workspace_need(type, layout, cols, rows, false, batch, half_input != 0, t, &need_f, &need_c);
    else {
        gemm_workspace_need(type, layout, cols, rows, batch, false, t, &need_f, &need_c);
        if (!fits()) {  // no split-K parts: the GEMM keeps its whole K range per tile
            t.gemm_kparts = 1;
            gemm_workspace_need(type, layout, cols, rows, batch, false, t, &need_f, &need_c);
        }
    }
    if (!fits())
        return fail(NS_ERR_UNSUPPORTED, std::string(fn) + ": this shape needs " + std::to_string(need_f * 4) + " B of parts and " +
                                            std::to_string(need_c) + " counters, above the static scratch (" +
                                            std::to_string(kScratchFloats * 4) + " B, " + std::to_string(kScratchCounters) + ")");
    ScratchMem *sm = nullptr;
    if (int rc = scratch_address(&sm)) return rc;
    Workspace ws;
    ws.partial = sm->parts;
    ws.partial_floats = kScratchFloats;
    ws.counters = sm->counters;
    ws.counter_count = kScratchCounters;
    ws.err = sm->err;
    ws.tune = t;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (need_c) {
        clear_counters<<<dim3(uint32_t((need_c + 255) / 256)), dim3(256), 0, s>>>(ws.counters, uint32_t(need_c));
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return fail(NS_ERR_HIP, std::string(fn) + ": " + hipGetErrorString(e));
    }
    hipError_t e;
    const auto *wb = static_cast<const uint8_t *>(w);
    if (batch == 1) e = launch_gemv(type, layout, wb, nullptr, static_cast<const float *>(in), out, cols, rows, ws, s);
    else if (batch <= 4) e = launch_gemv_mt(type, layout, wb, nullptr, in, half_input != 0, batch, out, cols, rows, ws, s);
    else e = launch_gemm(type, layout, ACC_FP32, wb, nullptr, static_cast<const uint16_t *>(in), out, cols, rows, batch, ws, s);
    return e == hipSuccess ? NS_OK : fail(NS_ERR_HIP, std::string(fn) + ": " + hipGetErrorString(e));
}

extern "C" int ns_noalloc_status(void *stream) {
    using namespace ns;
    ScratchMem *sm = nullptr;
    if (int rc = scratch_address(&sm)) return rc;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    uint32_t v = 0;
    hipError_t e = hipStreamSynchronize(s);
    if (e == hipSuccess) e = hipMemcpy(&v, sm->err, sizeof v, hipMemcpyDeviceToHost);
    if (e == hipSuccess && v != 0) {
        clear_counters<<<dim3(1), dim3(64), 0, s>>>(sm->err, 1u);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipStreamSynchronize(s);
    }
    if (e != hipSuccess) return fail(NS_ERR_HIP, std::string("ns_noalloc_status: ") + hipGetErrorString(e));
    return v == 0 ? NS_OK : fail(NS_ERR_TIMEOUT, "ns_noalloc_status: " + wait_status_message(v));
}
