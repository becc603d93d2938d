// ns_norm.hip -- standardisation of FFN outputs between layers of the stack.
//
// BASELINE config 4 keeps the hidden state of the 48-layer FFN stack an N(0,1)
// vector at unit RMS between layers: x_t = (y_t - mean(y_t)) / rms(y_t - mean(y_t))
// per token, as fp16 for the prefill GEMMs (the engine's halfbuf,
// metal_engine.mm:563) or fp32 for the decode GEMVs (its `norm` buffer).  It
// stands in for the engine's residual-add + RMSNorm between FFN blocks
// (rms_add_then_half, metal:523-529), which is outside this path.
//
// The mean is removed because BASELINE's synthetic weights are not centred:
// a Q4_K weight d*sc*q - dmin*m with d, dmin = |N|*1e-3 and uniform sc, m, q
// has mean ~0.16, so every output of a layer carries a common component
// proportional to sum(x).  A chain that only rescales drifts towards a constant
// vector within a few layers; once that constant is negative every gate output
// is far below zero, GeGLU returns exactly 0, and the next rescale is 0/0.
// A row whose values are all equal maps to zeros.
//
// One workgroup per token; both sums are taken in fp32 in a fixed order
// (deterministic), the second about the mean so the common component does not
// cancel precision away.  The output row must not alias the input row.
#include "ns_internal.hpp"
#include "ns_quant.hpp"

namespace ns {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float block_sum(float s, float *part) {
    for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m);
    __syncthreads();  // `part` may still be read from the previous sum
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) tot += part[w];
    return tot;
}

// Rows of up to kThreads * 4 * kMaxVec values are read once into registers
// (float4 per thread, coalesced); longer or unaligned rows take the looped path.
constexpr int kMaxVec = 8;  // float4 loads per thread: rows of up to 8192 values

template <bool HALF>
__global__ __launch_bounds__(kThreads) void standardize_kernel(const float *__restrict__ y, uint32_t cols,
                                                             void *__restrict__ out, bool vec_ok) {
    __shared__ float part[kThreads / 64];
    const uint32_t t = blockIdx.x, tid = threadIdx.x;
    const float *row = y + size_t(t) * cols;
    const uint32_t n4 = cols / 4;
    if (vec_ok && cols % 4 == 0 && n4 <= uint32_t(kThreads * kMaxVec)) {
        float4 v[kMaxVec];
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < kMaxVec; ++i) {
            const uint32_t j = tid + uint32_t(i) * kThreads;
            v[i] = j < n4 ? reinterpret_cast<const float4 *>(row)[j] : float4{0.f, 0.f, 0.f, 0.f};
            s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
        }
        const float mean = block_sum(s, part) / float(cols);
        float q = 0.f;
#pragma unroll
        for (int i = 0; i < kMaxVec; ++i) {
            if (tid + uint32_t(i) * kThreads >= n4) continue;
            v[i].x -= mean;
            v[i].y -= mean;
            v[i].z -= mean;
            v[i].w -= mean;
            q = __builtin_fmaf(v[i].x, v[i].x, q);
            q = __builtin_fmaf(v[i].y, v[i].y, q);
            q = __builtin_fmaf(v[i].z, v[i].z, q);
            q = __builtin_fmaf(v[i].w, v[i].w, q);
        }
        const float var = block_sum(q, part) / float(cols);
        const float inv = var > 0.f ? 1.0f / __builtin_sqrtf(var) : 0.f;
#pragma unroll
        for (int i = 0; i < kMaxVec; ++i) {
            const uint32_t j = tid + uint32_t(i) * kThreads;
            if (j >= n4) continue;
            const float a = v[i].x * inv, b = v[i].y * inv, c = v[i].z * inv, d = v[i].w * inv;
            if constexpr (HALF) {
                typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
                reinterpret_cast<half4_t *>(out)[size_t(t) * n4 + j] = half4_t{_Float16(a), _Float16(b), _Float16(c), _Float16(d)};
            } else {
                reinterpret_cast<float4 *>(out)[size_t(t) * n4 + j] = float4{a, b, c, d};
            }
        }
        return;
    }
    float s = 0.f;
    for (uint32_t k = tid; k < cols; k += kThreads) s += row[k];
    const float mean = block_sum(s, part) / float(cols);
    float q = 0.f;
    for (uint32_t k = tid; k < cols; k += kThreads) {
        const float c = row[k] - mean;
        q = __builtin_fmaf(c, c, q);
    }
    const float var = block_sum(q, part) / float(cols);
    const float inv = var > 0.f ? 1.0f / __builtin_sqrtf(var) : 0.f;
    for (uint32_t k = tid; k < cols; k += kThreads) {
        const float v = (row[k] - mean) * inv;
        if constexpr (HALF) reinterpret_cast<_Float16 *>(out)[size_t(t) * cols + k] = _Float16(v);
        else reinterpret_cast<float *>(out)[size_t(t) * cols + k] = v;
    }
}

}  // namespace

hipError_t launch_standardize(const float *y, uint32_t batch, uint32_t cols, void *out, bool half,
                              hipStream_t stream) {
    // float4 / half4 accesses need 16-byte aligned input and output rows
    const bool vec_ok = (reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(out)) % 16 == 0;
    if (half) standardize_kernel<true><<<dim3(batch), dim3(kThreads), 0, stream>>>(y, cols, out, vec_ok);
    else standardize_kernel<false><<<dim3(batch), dim3(kThreads), 0, stream>>>(y, cols, out, vec_ok);
    return hipGetLastError();
}

}  // namespace ns
