// ns_norm.hip -- the engine's elementwise steps around the FFN matmuls: the RMSNorm
// family (metal:509-529: rms / rms_half, rms_add, rms_add_then_half and its fp32 form,
// one workgroup per row) and the standalone GeGLU (metal:530-531) that follows two
// separate gate/up matmuls.
#include <algorithm>

#include "ns_internal.hpp"
#include "ns_quant.hpp"
#include "ns_rms.hpp"

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

// The engine's RMSNorm family around the FFN block (metal:509-529; rms, rms_half,
// rms_add, rms_add_then_half at mm:291-296, called at mm:563, :574, :576):
//   y = (x * r) * w                                   gemma_rmsnorm[_f16]
//   y = residual + (x * r) * w  [then * scale]        gemma_rmsnorm_add[_scale]
//   next = (y * r2) * next_w                          ..._then_f16 (and its fp32 form)
// with r = 1/sqrt(sum(x^2)/width + eps) per row, r2 the same over y.  One
// workgroup per row; each thread owns the elements k = tid + j*256.  The second
// pass re-reads y where this thread stored it, as the reference does.
template <bool HY, bool ADD, bool THEN, bool HN>
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const float *x, const float *__restrict__ w,
                                                         const float *residual,
                                                         const float *__restrict__ scale,
                                                         const float *__restrict__ next_w, uint32_t width, float eps,
                                                         void *y, void *__restrict__ next) {
    __shared__ float part[kThreads / 64];
    const size_t base = size_t(blockIdx.x) * width;
    const uint32_t tid = threadIdx.x;
    const float *xr = x + base;
    float s = 0.f;
    for (uint32_t k = tid; k < width; k += kThreads) s = __builtin_fmaf(xr[k], xr[k], s);
    const float r = 1.0f / __builtin_sqrtf(block_sum(s, part) / float(width) + eps);
    const float sc = (ADD && scale) ? *scale : 1.0f;
    float s2 = 0.f;
    for (uint32_t k = tid; k < width; k += kThreads) {
        float v = (xr[k] * r) * w[k];
        if constexpr (ADD) {
            v = residual[base + k] + v;
            if (scale) v *= sc;
        }
        if constexpr (HY) static_cast<_Float16 *>(y)[base + k] = _Float16(v);
        else static_cast<float *>(y)[base + k] = v;
        if constexpr (THEN) s2 = __builtin_fmaf(v, v, s2);
    }
    if constexpr (THEN) {
        const float r2 = 1.0f / __builtin_sqrtf(block_sum(s2, part) / float(width) + eps);
        const float *yr = static_cast<const float *>(y) + base;
        for (uint32_t k = tid; k < width; k += kThreads) {
            const float v = (yr[k] * r2) * next_w[k];
            if constexpr (HN) static_cast<_Float16 *>(next)[base + k] = _Float16(v);
            else static_cast<float *>(next)[base + k] = v;
        }
    }
}

// The same family with the row held in registers (ns::rms_row): one memory round
// trip per row.  HY: fp16 y (rms_half, no residual); HZ: fp16 next.
template <bool HY, bool HZ>
// x, residual and y are not restrict: an fp32 y may alias x or residual (every
// thread loads its whole row share before it stores).
__global__ __launch_bounds__(1024) void rmsnorm_vec_kernel(const float *x, const float *__restrict__ w,
                                                          const float *residual,
                                                          const float *__restrict__ scale,
                                                          const float *__restrict__ next_w, uint32_t width, float eps,
                                                          void *y, void *__restrict__ next) {
    __shared__ float part[16];
    typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
    const size_t base4 = size_t(blockIdx.x) * (width / 4);
    auto h4 = [](const float4 &v) { return half4_t{_Float16(v.x), _Float16(v.y), _Float16(v.z), _Float16(v.w)}; };
    rms_row<4>(reinterpret_cast<const float4 *>(x) + base4, reinterpret_cast<const float4 *>(w),
               residual ? reinterpret_cast<const float4 *>(residual) + base4 : nullptr, scale,
               reinterpret_cast<const float4 *>(next_w), width / 4, eps, part,
               [&](uint32_t j, const float4 &v) {
                   if constexpr (HY) static_cast<half4_t *>(y)[base4 + j] = h4(v);
                   else static_cast<float4 *>(y)[base4 + j] = v;
               },
               [&](uint32_t j, const float4 &z) {
                   if constexpr (HZ) static_cast<half4_t *>(next)[base4 + j] = h4(z);
                   else static_cast<float4 *>(next)[base4 + j] = z;
               });
}

// y = fp16(x), round to nearest even (the conversion of the reference's tile loader,
// metal:235), four values per thread; n need not be a multiple of four.
__global__ __launch_bounds__(256) void f32_to_f16_kernel(const float *__restrict__ x, _Float16 *__restrict__ y,
                                                          size_t n) {
    const size_t i = (size_t(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
    if (i + 4 <= n) {
        const float4 v = *reinterpret_cast<const float4 *>(x + i);
        typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
        *reinterpret_cast<half4_t *>(y + i) = half4_t{_Float16(v.x), _Float16(v.y), _Float16(v.z), _Float16(v.w)};
    } else {
        for (size_t k = i; k < n; ++k) y[k] = _Float16(x[k]);
    }
}

}  // namespace

hipError_t launch_f32_to_f16(const float *x, uint16_t *y, size_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    // the vector path needs 16-byte x and 8-byte y: otherwise one value per thread
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(y) % 8) return hipErrorInvalidValue;
    const size_t threads = (n + 3) / 4;
    f32_to_f16_kernel<<<dim3(uint32_t((threads + 255) / 256)), dim3(256), 0, stream>>>(
        x, reinterpret_cast<_Float16 *>(y), n);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const float *x, const float *w, const float *residual, const float *scale,
                          const float *next_w, uint32_t rows, uint32_t width, float eps, void *y, bool half_y,
                          void *next, bool half_next, hipStream_t stream) {
    if (next_w && !residual) return hipErrorInvalidValue;  // the second norm follows rms_add only
    if (residual && half_y) return hipErrorInvalidValue;   // rms_add writes the fp32 residual stream
    const dim3 g(rows);
    // The register form: rows of up to 4 float4 per thread at up to 1024 threads, 16-byte
    // aligned (fp16 outputs 8-byte aligned).
    auto al = [](const void *p, uintptr_t a) { return !p || reinterpret_cast<uintptr_t>(p) % a == 0; };
    const uint32_t n4 = width / 4;
    const bool vec = width % 4 == 0 && n4 <= 4096 && al(x, 16) && al(w, 16) && al(residual, 16) &&
                     al(next_w, 16) && al(y, half_y ? 8 : 16) && al(next, half_next ? 8 : 16);
    if (vec) {
        const uint32_t nt = std::min(1024u, std::max(64u, ((n4 + 3) / 4 + 63) / 64 * 64));
        const dim3 b(nt);
        if (half_y) rmsnorm_vec_kernel<true, false><<<g, b, 0, stream>>>(x, w, nullptr, nullptr, nullptr, width, eps, y, nullptr);
        else if (half_next) rmsnorm_vec_kernel<false, true><<<g, b, 0, stream>>>(x, w, residual, scale, next_w, width, eps, y, next);
        else rmsnorm_vec_kernel<false, false><<<g, b, 0, stream>>>(x, w, residual, scale, next_w, width, eps, y, next);
        return hipGetLastError();
    }
    const dim3 b(kThreads);
    if (!residual) {
        if (half_y) rmsnorm_kernel<true, false, false, false><<<g, b, 0, stream>>>(x, w, nullptr, nullptr, nullptr, width, eps, y, nullptr);
        else rmsnorm_kernel<false, false, false, false><<<g, b, 0, stream>>>(x, w, nullptr, nullptr, nullptr, width, eps, y, nullptr);
    } else if (!next_w) {
        rmsnorm_kernel<false, true, false, false><<<g, b, 0, stream>>>(x, w, residual, scale, nullptr, width, eps, y, nullptr);
    } else if (half_next) {
        rmsnorm_kernel<false, true, true, true><<<g, b, 0, stream>>>(x, w, residual, scale, next_w, width, eps, y, next);
    } else {
        rmsnorm_kernel<false, true, true, false><<<g, b, 0, stream>>>(x, w, residual, scale, next_w, width, eps, y, next);
    }
    return hipGetLastError();
}

namespace {
// gemma_geglu / gemma_geglu_f16 (metal:530-531): y[i] = gelu_tanh(g[i]) * u[i], fp32 or fp16
// (round to nearest even) out.  Four values per thread where the pointers allow it.
template <bool HALF>
__global__ __launch_bounds__(kThreads) void geglu_kernel(const float *__restrict__ g, const float *__restrict__ u,
                                                         uint64_t n, void *__restrict__ y) {
    const uint64_t i = (uint64_t(blockIdx.x) * kThreads + threadIdx.x) * 4;
    if (i >= n) return;
    float v[4];
    if (i + 4 <= n) {
        const float4 a = *reinterpret_cast<const float4 *>(g + i), b = *reinterpret_cast<const float4 *>(u + i);
        v[0] = gelu_tanh(a.x) * b.x;
        v[1] = gelu_tanh(a.y) * b.y;
        v[2] = gelu_tanh(a.z) * b.z;
        v[3] = gelu_tanh(a.w) * b.w;
    } else {
        for (uint64_t k = 0; k < 4; ++k) v[k] = i + k < n ? gelu_tanh(g[i + k]) * u[i + k] : 0.f;
    }
    for (uint64_t k = 0; k < 4 && i + k < n; ++k) {
        if constexpr (HALF) reinterpret_cast<_Float16 *>(y)[i + k] = _Float16(v[k]);
        else reinterpret_cast<float *>(y)[i + k] = v[k];
    }
}
}  // namespace

hipError_t launch_geglu(const float *g, const float *u, uint64_t n, void *y, bool half_out, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    if ((reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(u)) % 16) return hipErrorInvalidValue;
    const uint64_t blocks = (n + 4 * kThreads - 1) / (4 * kThreads);
    if (blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
    if (half_out) geglu_kernel<true><<<dim3(uint32_t(blocks)), dim3(kThreads), 0, stream>>>(g, u, n, y);
    else geglu_kernel<false><<<dim3(uint32_t(blocks)), dim3(kThreads), 0, stream>>>(g, u, n, y);
    return hipGetLastError();
}

}  // namespace ns
