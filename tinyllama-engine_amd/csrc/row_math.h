// Sums over rows of floats in one fixed order, shared by every kernel that
// must agree bit for bit: the rmsnorm kernels (one row, a batch of rows) and
// the matrix-vector kernel's fused rmsnorm and block-format run sums.  A
// prompt run as one batch and the same prompt run token by token then give
// identical layer-0 results.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tla {

// Pairwise: (x + y) + (z + w).
__device__ __forceinline__ float sum4(float4 v)
{
    return (v.x + v.y) + (v.z + v.w);
}

// ((x^2 + y^2) + z^2) + w^2 with explicit fused multiply-adds, so that no
// kernel's contraction choices change the rounding.
__device__ __forceinline__ float sum_sq4(float4 v)
{
    return fmaf(v.w, v.w, fmaf(v.z, v.z, fmaf(v.y, v.y, v.x * v.x)));
}

__device__ __forceinline__ bool aligned16(const void* p)
{
    return (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

// Wave tree (xor 32 .. 1), then the waves' sums in order; one barrier.
template <int kThreads>
__device__ __forceinline__ float block_sum(float v, float* s_red)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kThreads / 64; ++i) t += s_red[i];
    return t;
}

// Sum of squares of one row, by a workgroup of kThreads: thread t takes the
// 16-byte pieces t, t + kThreads, ... (when the row is 16-byte aligned and
// size a multiple of 4; else the columns t, t + kThreads, ...), then a wave
// tree and the waves in order.  s_red holds kThreads / 64 floats; the call
// contains one barrier.
template <int kThreads>
__device__ __forceinline__ float row_sum_squares(const float* x, int size, float* s_red)
{
    float ss = 0.f;
    if (aligned16(x) && (size & 3) == 0) {
        for (int c4 = threadIdx.x; c4 < size / 4; c4 += kThreads)
            ss += sum_sq4(*reinterpret_cast<const float4*>(x + 4 * c4));
    } else {
        for (int c = threadIdx.x; c < size; c += kThreads) ss = fmaf(x[c], x[c], ss);
    }
    return block_sum<kThreads>(ss, s_red);
}

}  // namespace tla
