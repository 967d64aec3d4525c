// Device-side rotation helpers shared by the decode and prefill kernels.
//
// RoPE rotates adjacent pairs (2i, 2i+1) of each head (the reference's
// layout, src/ops.cpp:1252-1262):
//     x0' = x0*cos - x1*sin,   x1' = x0*sin + x1*cos
// Each product and each sum is rounded on its own (contraction off), so the
// result is bit-identical to the reference's x86-64 build, which has no FMA.
// cos/sin come from a table computed on the host with the reference's own
// float expressions (engine.hip), so the device never evaluates sin/cos.
#pragma once

#include <hip/hip_runtime.h>

namespace tla {

__device__ __forceinline__ float rot_lo(float x0, float x1, float c, float s)
{
#pragma clang fp contract(off)
    return x0 * c - x1 * s;
}

__device__ __forceinline__ float rot_hi(float x0, float x1, float c, float s)
{
#pragma clang fp contract(off)
    return x0 * s + x1 * c;
}

// x holds dims d..d+3 (d even): pairs (d, d+1) and (d+2, d+3).
// cs = (cos_a, sin_a, cos_b, sin_b) for those two pairs.
__device__ __forceinline__ float4 rotate4(float4 x, float4 cs)
{
    float4 r;
    r.x = rot_lo(x.x, x.y, cs.x, cs.y);
    r.y = rot_hi(x.x, x.y, cs.x, cs.y);
    r.z = rot_lo(x.z, x.w, cs.z, cs.w);
    r.w = rot_hi(x.z, x.w, cs.z, cs.w);
    return r;
}

__device__ __forceinline__ float4 ldg4(const float* p)
{
    return *reinterpret_cast<const float4*>(p);
}

// 16-byte load at a 32-bit byte offset from a (wave-uniform) base: lets the
// compiler use the scalar-base + 32-bit-offset addressing form.
__device__ __forceinline__ float4 ldg4_at(const float* base, unsigned byte_off)
{
    return *reinterpret_cast<const float4*>(reinterpret_cast<const char*>(base) + byte_off);
}

__device__ __forceinline__ float2 ldg2_at(const float* base, unsigned byte_off)
{
    return *reinterpret_cast<const float2*>(reinterpret_cast<const char*>(base) + byte_off);
}

__device__ __forceinline__ void stg4(float* p, float4 v)
{
    *reinterpret_cast<float4*>(p) = v;
}

}  // namespace tla
