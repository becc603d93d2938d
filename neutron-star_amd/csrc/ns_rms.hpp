// ns_rms.hpp -- one row of the RMSNorm family (metal:509-529) computed by one
// workgroup, shared by the standalone kernels (ns_norm.hip) and the decode
// GEMV prologue (ns_gemv.hip).
//
// The row is 4*n4 fp32 values.  Thread tid owns the float4 chunks
// j = tid + i*nt (i < KV), so KV*nt >= n4 must hold; every global load of the
// row is issued before the first use, so the row costs one memory round trip.
//   res == nullptr: y = (x*r)*w                       r = 1/sqrt(sum(x^2)/n + eps)
//   res != nullptr: y = (res + (x*r)*w) [* *scale]
//   next_w:         z = (y*r2)*next_w                 r2 likewise over y
// out_y(j, y) and out_z(j, z) receive the chunks.  Sums are fp32 FMAs in a
// fixed order (the same in every workgroup with the same nt).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace ns {

// Sum of one value per thread over the workgroup; `part` holds one float per wave.
__device__ __forceinline__ float wg_sum(float s, float *part, uint32_t nw) {
    for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m);
    __syncthreads();  // `part` may still be read from the previous sum
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    float tot = 0.f;
    for (uint32_t w = 0; w < nw; ++w) tot += part[w];
    return tot;
}

__device__ __forceinline__ float rms_factor(float sumsq, uint32_t n, float eps) {
    return 1.0f / __builtin_sqrtf(sumsq / float(n) + eps);
}

__device__ __forceinline__ float sumsq4(const float4 &v, float s) {
    s = __builtin_fmaf(v.x, v.x, s);
    s = __builtin_fmaf(v.y, v.y, s);
    s = __builtin_fmaf(v.z, v.z, s);
    return __builtin_fmaf(v.w, v.w, s);
}

__device__ __forceinline__ float4 mul4(const float4 &a, float r, const float4 &w) {
    return float4{(a.x * r) * w.x, (a.y * r) * w.y, (a.z * r) * w.z, (a.w * r) * w.w};
}

// The row's registers between the two phases.  Splitting the loads from the
// arithmetic lets a caller issue other loads in between: vector loads complete
// in order, so the arithmetic then waits only for the row.
template <int KV>
struct RmsRow {
    float4 X[KV], W[KV], R[KV], Z[KV];
    float sc;
};

template <int KV>
__device__ __forceinline__ void rms_row_load(RmsRow<KV> &rr, const float4 *x,
                                             const float4 *__restrict__ w, const float4 *res,
                                             const float *__restrict__ scale, const float4 *__restrict__ next_w,
                                             uint32_t n4) {
    const uint32_t nt = blockDim.x, tid = threadIdx.x;
    rr.sc = (res && scale) ? *scale : 1.0f;
#pragma unroll
    for (int i = 0; i < KV; ++i) {
        const uint32_t j = tid + uint32_t(i) * nt;
        if (j < n4) {
            rr.X[i] = x[j];
            rr.W[i] = w[j];
            if (res) rr.R[i] = res[j];
            if (next_w) rr.Z[i] = next_w[j];
        }
    }
}

template <int KV, class OutY, class OutZ>
__device__ __forceinline__ void rms_row_finish(RmsRow<KV> &rr, bool has_res, bool has_scale, bool has_next,
                                               uint32_t n4, float eps, float *part, OutY &&out_y, OutZ &&out_z) {
    const uint32_t nt = blockDim.x, tid = threadIdx.x, nw = (nt + 63) >> 6;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < KV; ++i)
        if (tid + uint32_t(i) * nt < n4) s = sumsq4(rr.X[i], s);
    const float r = rms_factor(wg_sum(s, part, nw), 4 * n4, eps);
    float s2 = 0.f;
#pragma unroll
    for (int i = 0; i < KV; ++i) {
        const uint32_t j = tid + uint32_t(i) * nt;
        if (j >= n4) continue;
        float4 v = mul4(rr.X[i], r, rr.W[i]);
        if (has_res) {
            v = float4{rr.R[i].x + v.x, rr.R[i].y + v.y, rr.R[i].z + v.z, rr.R[i].w + v.w};
            if (has_scale) v = float4{v.x * rr.sc, v.y * rr.sc, v.z * rr.sc, v.w * rr.sc};
        }
        out_y(j, v);
        rr.X[i] = v;
        if (has_next) s2 = sumsq4(v, s2);
    }
    if (!has_next) return;
    const float r2 = rms_factor(wg_sum(s2, part, nw), 4 * n4, eps);
#pragma unroll
    for (int i = 0; i < KV; ++i) {
        const uint32_t j = tid + uint32_t(i) * nt;
        if (j < n4) out_z(j, mul4(rr.X[i], r2, rr.Z[i]));
    }
}

template <int KV, class OutY, class OutZ>
__device__ __forceinline__ void rms_row(const float4 *x, const float4 *__restrict__ w,
                                        const float4 *res, const float *__restrict__ scale,
                                        const float4 *__restrict__ next_w, uint32_t n4, float eps, float *part,
                                        OutY &&out_y, OutZ &&out_z) {
    RmsRow<KV> rr;
    rms_row_load<KV>(rr, x, w, res, scale, next_w, n4);
    rms_row_finish<KV>(rr, res != nullptr, scale != nullptr, next_w != nullptr, n4, eps, part, out_y, out_z);
}

}  // namespace ns
