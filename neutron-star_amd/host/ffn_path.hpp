// ffn_path.hpp -- C++ host layer over the C ABI (include/ns_ffn.h) that keeps
// the reference engine's FFN call surface (src/native/metal_engine.mm):
//
//   matmul(e, w, in, out, batch, half_input)          mm:269-275
//   gate_up_geglu_rm32(e, gate, up, in, out, batch, fast_swa)   mm:288
//   gate_up_geglu_decode(e, gate, up, in, out)        mm:290
//   ffn_down(e, w, in, out, batch, half_input, fast_swa)        mm:289
//
// The reference passes an id<MTLComputeCommandEncoder>; here the first
// argument is the hipStream_t the work is ordered on.  Weights are addressed
// the way the reference addresses them: one device image of the weight file
// plus a per-tensor byte offset and layout (MetalFfnFile::offset / reordered,
// src/native/metal_ffn.cpp:300-311).  Failures throw std::runtime_error with
// the C ABI's message, the reference's error convention (mm:231-243).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "ns_ffn.h"

namespace neutron::amd {

// GGUF tensor types used on this path (include/neutron/native/gguf.hpp:13).
enum class TensorType : uint32_t { F32 = 0, F16 = 1, Q4_K = 12, Q6_K = 14 };

// Descriptor of one weight tensor, as in gguf.hpp:20-27: shape[0] = cols (K),
// shape[1] = rows (N); `offset` identifies the tensor (the GGUF data offset).
struct Tensor {
    std::string name;
    std::vector<uint64_t> shape;
    TensorType type{};
    uint64_t offset = 0;
    uint64_t bytes = 0;
};

enum class Layout : int { RowMajor = NS_LAYOUT_ROW_MAJOR, Nsmffn = NS_LAYOUT_NSMFFN, Cdna4 = NS_LAYOUT_CDNA4 };

inline void check(int rc) {
    if (rc != NS_OK) throw std::runtime_error(std::string("neutron-star-amd: ") + ns_last_error());
}

// A device image of the weights: one allocation, each tensor at a byte offset
// in a given layout (the role MetalFfnFile plays for the Metal engine).
class WeightImage {
public:
    WeightImage() = default;
    WeightImage(const WeightImage &) = delete;
    WeightImage &operator=(const WeightImage &) = delete;
    ~WeightImage() {
        if (base_) (void)hipFree(base_);
    }

    // Allocate `bytes` of device memory for the image.
    void allocate(size_t bytes) {
        if (base_) throw std::runtime_error("weight image already allocated");
        if (hipMalloc(&base_, bytes) != hipSuccess) throw std::runtime_error("weight image allocation failed");
        size_ = bytes;
    }
    // Copy host bytes of one tensor into the image at `image_offset` and
    // register it; with `retile_to_cdna4`, NSMFFN / ROW_MAJOR input is converted
    // on the device into the CDNA4 layout (the conversion step at load time).
    void upload(const Tensor &t, const void *host, uint64_t image_offset, Layout layout, bool retile_to_cdna4,
                hipStream_t stream) {
        if (!base_ || image_offset + t.bytes > size_) throw std::runtime_error("tensor outside the weight image: " + t.name);
        uint8_t *dst = static_cast<uint8_t *>(base_) + image_offset;
        if (!retile_to_cdna4 || layout == Layout::Cdna4 || t.type == TensorType::F32 || t.type == TensorType::F16) {
            if (hipMemcpyAsync(dst, host, t.bytes, hipMemcpyHostToDevice, stream) != hipSuccess)
                throw std::runtime_error("weight upload failed: " + t.name);
            entries_[t.offset] = {image_offset, layout};
            return;
        }
        void *tmp = nullptr;
        if (hipMalloc(&tmp, t.bytes) != hipSuccess) throw std::runtime_error("staging allocation failed");
        bool ok = hipMemcpyAsync(tmp, host, t.bytes, hipMemcpyHostToDevice, stream) == hipSuccess;
        int rc = ok ? ns_retile_device(tmp, dst, int(t.type), uint32_t(t.shape.at(0)), uint32_t(t.shape.at(1)),
                                       int(layout), NS_LAYOUT_CDNA4, stream)
                    : NS_ERR_HIP;
        ok = ok && rc == NS_OK && hipStreamSynchronize(stream) == hipSuccess;
        (void)hipFree(tmp);
        if (!ok) throw std::runtime_error("weight conversion failed: " + t.name + ": " + ns_last_error());
        entries_[t.offset] = {image_offset, Layout::Cdna4};
    }
    // MetalFfnFile::offset (metal_ffn.cpp:300-305): byte offset of a tensor.
    uint64_t offset(const Tensor &t) const { return entry(t).first; }
    Layout layout(const Tensor &t) const { return entry(t).second; }
    const void *data(const Tensor &t) const { return static_cast<const uint8_t *>(base_) + offset(t); }

private:
    const std::pair<uint64_t, Layout> &entry(const Tensor &t) const {
        const auto it = entries_.find(t.offset);
        if (it == entries_.end()) throw std::runtime_error("tensor missing from weight image: " + t.name);
        return it->second;
    }
    void *base_ = nullptr;
    size_t size_ = 0;
    std::unordered_map<uint64_t, std::pair<uint64_t, Layout>> entries_;
};

// The FFN dispatch helpers of the reference engine over one device context.
class FfnPath {
public:
    explicit FfnPath(const WeightImage &weights, int device = 0) : w_(weights) { check(ns_ctx_create(device, &ctx_)); }
    ~FfnPath() { ns_ctx_destroy(ctx_); }
    FfnPath(const FfnPath &) = delete;
    FfnPath &operator=(const FfnPath &) = delete;

    // mm:269-275: batch 1 -> dequant-fused GEMV; batch 2-4 -> the small-batch kernels (the
    // weights streamed once for every token, fp32 or fp16 input); batch > 4 -> MFMA GEMM (FP32
    // accumulation; fp32 input rounded to fp16 first, as the reference's tile loader does).
    void matmul(hipStream_t e, const Tensor &w, const void *in, float *out, uint32_t batch,
                bool half_input = false) const {
        check(ns_matmul(ctx_, w_.data(w), int(w.type), int(w_.layout(w)), cols(w), rows(w), batch, in,
                        half_input ? 1 : 0, out, e));
    }
    // mm:281: gate/up + GeGLU, fp16 in, fp16 out; batch <= 4 (MTP verification) streams
    // the weights once for every token.
    void gate_up_geglu(hipStream_t e, const Tensor &gate, const Tensor &up, const uint16_t *in, uint16_t *out,
                       uint32_t batch) const {
        same_shape(gate, up);
        check(ns_gate_up_geglu(ctx_, w_.data(gate), w_.data(up), int(w_.layout(gate)), cols(gate), rows(gate), batch,
                               in, out, e));
    }
    // mm:288: prefill gate/up + GeGLU, fp16 in, fp16 out; fast_swa selects the FP16 mode.
    void gate_up_geglu_rm32(hipStream_t e, const Tensor &gate, const Tensor &up, const uint16_t *in, uint16_t *out,
                            uint32_t batch, bool fast_swa) const {
        same_shape(gate, up);
        check(ns_gate_up_geglu_rm32(ctx_, w_.data(gate), w_.data(up), int(w_.layout(gate)), cols(gate), rows(gate),
                                    batch, in, out, fast_swa ? 1 : 0, e));
    }
    // mm:290: decode gate/up + GeGLU, fp32 in and out.
    void gate_up_geglu_decode(hipStream_t e, const Tensor &gate, const Tensor &up, const float *in, float *out) const {
        same_shape(gate, up);
        check(ns_gate_up_geglu_decode(ctx_, w_.data(gate), w_.data(up), int(w_.layout(gate)), cols(gate), rows(gate),
                                      in, out, e));
    }
    // mm:289: the down projection; prefill GEMM when half_input and batch > 1.
    void ffn_down(hipStream_t e, const Tensor &w, const void *in, float *out, uint32_t batch, bool half_input,
                  bool fast_swa = false) const {
        check(ns_ffn_down(ctx_, w_.data(w), int(w.type), int(w_.layout(w)), cols(w), rows(w), batch, in,
                          half_input ? 1 : 0, fast_swa ? 1 : 0, out, e));
    }

    // The FFN part of the engine's per-layer loop (mm:564-573): gate/up + GeGLU
    // into `mid`, then the down projection into `out`, in the accumulation mode
    // fast_swa_ffn = prefill && swa && !exact_ffn (mm:565).  Prefill: `in` is fp16
    // [batch][cols] (halfbuf) and `mid` fp16 [batch][ffn]; decode: both fp32.
    void ffn_block(hipStream_t e, const Tensor &gate, const Tensor &up, const Tensor &down, const void *in, void *mid,
                   float *out, uint32_t batch, bool prefill, bool swa, bool exact_ffn) const {
        const bool fast_swa = prefill && swa && !exact_ffn;
        if (prefill && batch > 4) {
            gate_up_geglu_rm32(e, gate, up, static_cast<const uint16_t *>(in), static_cast<uint16_t *>(mid), batch,
                               fast_swa);
        } else if (prefill) {
            // mm:569: a prefill of 2-4 tokens (MTP verification) takes gate_up_geglu, the
            // small-batch kernel, in FP32 accumulation whatever the layer's mode
            gate_up_geglu(e, gate, up, static_cast<const uint16_t *>(in), static_cast<uint16_t *>(mid), batch);
        } else if (batch == 1) {
            // mm:571-573: gate/up + GeGLU, then down, in one launch where the shapes allow it
            ffn_block_decode(e, gate, up, down, static_cast<const float *>(in), nullptr, 0.f,
                             static_cast<float *>(mid), out);
            return;
        } else {
            // mm:570: a decode of 2-4 fp32 tokens takes matmul(gate), matmul(up) (the small-batch
            // kernels, each streaming its weights once for every token) and gemma_geglu into mid
            same_shape(gate, up);
            const size_t n = size_t(batch) * rows(gate);
            float *g = scratch_.gate(n), *u = scratch_.up(n);
            matmul(e, gate, in, g, batch, false);
            matmul(e, up, in, u, batch, false);
            check(ns_geglu(ctx_, g, u, n, mid, 0, e));
        }
        ffn_down(e, down, mid, out, batch, prefill, fast_swa);
    }

    // finish_command (mm:231-243): waits for the work queued on `e` and throws if any call of
    // this path ran a bounded cross-workgroup wait out (its outputs then hold NaN).
    void finish(hipStream_t e) const { check(ns_ctx_status(ctx_, e)); }
    // For engines that share the GPU with other work: launches in which no workgroup waits
    // for another (ns_ctx_set_wait_free); results are unchanged.
    void set_wait_free(bool on) { check(ns_ctx_set_wait_free(ctx_, on ? 1 : 0)); }

    // The decode block (mm:563 rms when norm_w is given, mm:571-573) in one launch:
    // mid = GeGLU(gate.n, up.n), out = down.mid, n = in or its RMSNorm (norm_w, eps).
    // out may alias in.
    void ffn_block_decode(hipStream_t e, const Tensor &gate, const Tensor &up, const Tensor &down, const float *in,
                          const float *norm_w, float eps, float *mid, float *out) const {
        same_shape(gate, up);
        if (down.shape.at(0) != gate.shape.at(1) || down.shape.at(1) != gate.shape.at(0) ||
            w_.layout(down) != w_.layout(gate))
            throw std::runtime_error("down tensor does not match gate/up: " + down.name);
        check(ns_ffn_block_decode(ctx_, w_.data(gate), w_.data(up), w_.data(down), int(down.type),
                                  int(w_.layout(gate)), cols(gate), rows(gate), in, norm_w, eps, mid, out, e));
    }

    // qkv (mm:311): Q, K and V projections of fp16 `in` ([batch][cols]) into fp32 q, k, v;
    // wv == nullptr is the tied-V model (V = K).  batch >= 2.
    void qkv(hipStream_t e, const Tensor &wq, const Tensor &wk, const Tensor *wv, const uint16_t *in, float *q,
             float *k, float *v, uint32_t batch) const {
        if (wq.shape.at(0) != wk.shape.at(0) || w_.layout(wq) != w_.layout(wk) ||
            (wv && (wv->shape != wk.shape || w_.layout(*wv) != w_.layout(wk))))
            throw std::runtime_error("qkv tensors differ in input width, kv shape or layout: " + wq.name);
        check(ns_qkv(ctx_, w_.data(wq), w_.data(wk), wv ? w_.data(*wv) : nullptr, wv ? int(wv->type) : int(wk.type),
                     int(w_.layout(wq)), cols(wq), rows(wq), rows(wk), batch, in, q, k, v, e));
    }
    // The token embedding (mm:310, gemma_q6k_embedding): out[t] = scale * embedding[ids[t]].
    void embedding(hipStream_t e, const Tensor &emb, const int32_t *ids, uint32_t batch, float scale,
                   float *out) const {
        check(ns_embedding(ctx_, w_.data(emb), int(emb.type), int(w_.layout(emb)), cols(emb), rows(emb), ids, batch,
                           scale, out, e));
    }

    // The RMSNorm helpers around the FFN block (mm:291-296; metal:509-529).  Norm
    // weights are fp32 device vectors of `width`; eps is the model's epsilon.
    // rms (mm:291): out = (in * r) * w per row, r = 1/sqrt(mean(in^2) + eps).
    void rms(hipStream_t e, const float *in, float *out, const float *w, uint32_t width, uint32_t rows,
             float eps) const {
        check(ns_rmsnorm(ctx_, in, w, rows, width, eps, out, 0, e));
    }
    // rms_half (mm:292): the same into fp16 (the engine's halfbuf).
    void rms_half(hipStream_t e, const float *in, const float *w, uint32_t width, uint32_t rows, float eps,
                  uint16_t *half_out) const {
        check(ns_rmsnorm(ctx_, in, w, rows, width, eps, half_out, 1, e));
    }
    // rms_add (mm:295): out = residual + (in * r) * w, times *scale when given.
    void rms_add(hipStream_t e, const float *in, const float *residual, float *out, const float *w, uint32_t width,
                 uint32_t rows, float eps, const float *scale = nullptr) const {
        check(ns_rmsnorm_add(ctx_, in, w, residual, scale, rows, width, eps, out, e));
    }
    // rms_add_then_half (mm:296): rms_add into `out`, then half((out * r2) * next_w).
    void rms_add_then_half(hipStream_t e, const float *in, const float *residual, float *out, const float *w,
                           const float *next_w, uint32_t width, uint32_t rows, float eps, uint16_t *half_out,
                           const float *scale = nullptr) const {
        check(ns_rmsnorm_add_then(ctx_, in, w, residual, scale, next_w, rows, width, eps, out, half_out, 1, e));
    }
    // rms (mm:563, decode) fused into gate_up_geglu_decode (mm:571): one launch.
    void rms_gate_up_geglu_decode(hipStream_t e, const Tensor &gate, const Tensor &up, const float *in,
                                  const float *norm_w, float eps, float *out) const {
        same_shape(gate, up);
        check(ns_rms_gate_up_geglu_decode(ctx_, w_.data(gate), w_.data(up), int(w_.layout(gate)), cols(gate),
                                          rows(gate), in, norm_w, eps, out, e));
    }

private:
    static uint32_t cols(const Tensor &t) { return uint32_t(t.shape.at(0)); }
    static uint32_t rows(const Tensor &t) { return t.shape.size() > 1 ? uint32_t(t.shape[1]) : 1u; }
    void same_shape(const Tensor &a, const Tensor &b) const {
        if (a.shape != b.shape || w_.layout(a) != w_.layout(b))
            throw std::runtime_error("gate and up tensors differ in shape or layout: " + a.name + ", " + b.name);
    }
    // The engine's separate `gate` and `up` activation buffers (mm:100-101), used by the decode
    // of 2-4 tokens (mm:570); grown on first use of a larger batch and kept until the path is
    // destroyed (queued work may still read them).  The first call of a batch size allocates,
    // so it must not be the one captured into a graph.
    class Scratch {
    public:
        ~Scratch() {
            for (void *p : bufs_) (void)hipFree(p);
        }
        float *gate(size_t n) { return grow(gate_, gate_n_, n); }
        float *up(size_t n) { return grow(up_, up_n_, n); }

    private:
        float *grow(float *&p, size_t &have, size_t n) {
            if (n <= have) return p;
            void *q = nullptr;
            if (hipMalloc(&q, n * sizeof(float)) != hipSuccess) throw std::runtime_error("activation buffer allocation failed");
            bufs_.push_back(q);
            p = static_cast<float *>(q);
            have = n;
            return p;
        }
        float *gate_ = nullptr, *up_ = nullptr;
        size_t gate_n_ = 0, up_n_ = 0;
        std::vector<void *> bufs_;
    };

    const WeightImage &w_;
    ns_ctx *ctx_ = nullptr;
    mutable Scratch scratch_;
};

}  // namespace neutron::amd
