// fp32 values as sums of bf16 pieces, for products on the bf16 matrix cores
// that keep fp32 accuracy: a product of two bf16 pieces (8 significant bits
// each) is exact in an fp32 accumulator, so sum_k a b over split operands is
// an fp32 sum of exact products.
#pragma once

#include <hip/hip_runtime.h>

namespace tla {

// v = v0 + v1 + v2 exactly, each a bf16 (round to nearest even at each
// step; v - v0 has at most 16 significant bits, v - v0 - v1 at most 8).
__device__ __forceinline__ void split3(float v, __bf16& v0, __bf16& v1, __bf16& v2)
{
    v0 = static_cast<__bf16>(v);
    const float r1 = v - static_cast<float>(v0);
    v1 = static_cast<__bf16>(r1);
    v2 = static_cast<__bf16>(r1 - static_cast<float>(v1));
}

// The three planes of eight values, as split3 per value but two values per
// conversion (v_cvt_pk_bf16_f32), each rounded pair widened back to floats
// from the packed word by a shift and a mask: 5.5 operations per value.
typedef float split_f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 split_bf16x8 __attribute__((ext_vector_type(8)));
typedef float split_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 split_bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned split_u32x4 __attribute__((ext_vector_type(4)));

// (a, b) rounded to bf16 and packed (a in the low half); a0, b0 the rounded
// values as floats.
__device__ __forceinline__ unsigned round_pair(float a, float b, float& a0, float& b0)
{
    const unsigned pk = __builtin_bit_cast(unsigned, __builtin_convertvector(split_f32x2{a, b}, split_bf16x2));
    a0 = __builtin_bit_cast(float, pk << 16);
    b0 = __builtin_bit_cast(float, pk & 0xffff0000u);
    return pk;
}

__device__ __forceinline__ void split3x8(split_f32x8 v, split_bf16x8& v0, split_bf16x8& v1, split_bf16x8& v2)
{
    split_u32x4 w0, w1, w2;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float a0, b0, a1, b1, a2, b2;
        w0[i] = round_pair(v[2 * i], v[2 * i + 1], a0, b0);
        const float ra = v[2 * i] - a0, rb = v[2 * i + 1] - b0;
        w1[i] = round_pair(ra, rb, a1, b1);
        w2[i] = round_pair(ra - a1, rb - b1, a2, b2);
    }
    v0 = __builtin_bit_cast(split_bf16x8, w0);
    v1 = __builtin_bit_cast(split_bf16x8, w1);
    v2 = __builtin_bit_cast(split_bf16x8, w2);
}

// v = v0 + v1 exactly for v of at most 16 significant bits.
__device__ __forceinline__ void split2(float v, __bf16& v0, __bf16& v1)
{
    v0 = static_cast<__bf16>(v);
    v1 = static_cast<__bf16>(v - static_cast<float>(v0));
}

}  // namespace tla
