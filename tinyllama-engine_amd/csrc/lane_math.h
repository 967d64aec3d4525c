// Exchanges between the lanes of one wave in registers, with gfx950's
// permlane swaps instead of cross-lane shuffles (ds_bpermute, an LDS round
// trip).  Given x and a copy of x:
//   v_permlane32_swap leaves [x lanes 0-31 | x lanes 0-31] in the first and
//     [x lanes 32-63 | x lanes 32-63] in the second register;
//   v_permlane16_swap does the same for each pair of 16-lane rows, so the
//     first holds rows (0, 0, 2, 2) and the second rows (1, 1, 3, 3).
// Every lane then holds its own value and its partner's (lane l ^ 32, or
// l ^ 16) one in each register, and max / sum of the two are the same in
// every lane as with a shuffle (both operations commute).
//
// Register-only inline asm: through the compiler's builtins the two results
// of a swap were folded into one register (ROCm 7.2), so that a sum of both
// read one of them twice.  The s_nop pairs cover the swaps' VALU read / write
// hazards, which the compiler does not track inside asm.
#pragma once

#include <hip/hip_runtime.h>

namespace tla {

__device__ __forceinline__ void swap_halves32(float x, float& a, float& b)
{
    unsigned u = __builtin_bit_cast(unsigned, x), v = u;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(u), "+v"(v));
    a = __builtin_bit_cast(float, u);
    b = __builtin_bit_cast(float, v);
}

__device__ __forceinline__ void swap_rows16(float x, float& a, float& b)
{
    unsigned u = __builtin_bit_cast(unsigned, x), v = u;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(u), "+v"(v));
    a = __builtin_bit_cast(float, u);
    b = __builtin_bit_cast(float, v);
}

// x combined with lane l ^ 32's x / lane l ^ 16's x.
__device__ __forceinline__ float max_xor32(float x)
{
    float a, b;
    swap_halves32(x, a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float sum_xor32(float x)
{
    float a, b;
    swap_halves32(x, a, b);
    return a + b;
}
__device__ __forceinline__ float max_xor16(float x)
{
    float a, b;
    swap_rows16(x, a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float sum_xor16(float x)
{
    float a, b;
    swap_rows16(x, a, b);
    return a + b;
}

}  // namespace tla
