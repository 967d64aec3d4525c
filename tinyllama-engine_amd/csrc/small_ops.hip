// Stand-alone device ops: rope (src/ops.cpp:1223-1281), softmax
// (src/ops.cpp:1072-1091) and a vectorised device copy.
#include "rope_math.h"
#include "tla_internal.h"

namespace tla {
namespace {

// One thread per rotated pair; q heads first, then k heads, as the
// reference's two loops (src/ops.cpp:1229-1280).  cos/sin for this position
// arrive in the kernel arguments, computed on the host (engine.hip).
__global__ __launch_bounds__(256) void rope_kernel(const RopeParams p)
{
    const int pairs = p.head_dim / 2;
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= (p.n_head + p.n_head_kv) * pairs) return;
    const int h = idx / pairs;
    const int i = idx - h * pairs;
    float* row = (h < p.n_head) ? p.q + (long long)h * p.head_dim
                                : p.k + (long long)(h - p.n_head) * p.head_dim;
    const float2 cs = p.cs[i];
    const float x0 = row[2 * i];
    const float x1 = row[2 * i + 1];
    row[2 * i] = rot_lo(x0, x1, cs.x, cs.y);
    row[2 * i + 1] = rot_hi(x0, x1, cs.x, cs.y);
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
    return v;
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

// softmax in place: max, exp(x - max), sum, multiply by 1/sum (the same
// three steps and the same final multiply as src/ops.cpp:1072-1091).
__global__ __launch_bounds__(1024) void softmax_kernel(float* x, int n)
{
    __shared__ float red[16];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;

    float m = -INFINITY;
    for (int i = tid; i < n; i += 1024) m = fmaxf(m, x[i]);
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = red[0];
    for (int w = 1; w < 16; ++w) m = fmaxf(m, red[w]);
    __syncthreads();

    float s = 0.f;
    for (int i = tid; i < n; i += 1024) {
        const float e = expf(x[i] - m);
        x[i] = e;
        s += e;
    }
    s = wave_sum(s);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    s = 0.f;
    for (int w = 0; w < 16; ++w) s += red[w];
    const float inv = 1.0f / s;
    for (int i = tid; i < n; i += 1024) x[i] *= inv;
}

__global__ __launch_bounds__(256) void copy16_kernel(float4* __restrict__ dst,
                                                     const float4* __restrict__ src, long long n16)
{
    const long long stride = (long long)gridDim.x * 256;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

__global__ __launch_bounds__(256) void copy1_kernel(unsigned char* __restrict__ dst,
                                                    const unsigned char* __restrict__ src, long long n)
{
    const long long stride = (long long)gridDim.x * 256;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

__global__ __launch_bounds__(256) void zero16_kernel(float4* __restrict__ dst, long long n16)
{
    const long long stride = (long long)gridDim.x * 256;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride)
        dst[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}

__global__ __launch_bounds__(256) void zero1_kernel(unsigned char* __restrict__ dst, long long n)
{
    const long long stride = (long long)gridDim.x * 256;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) dst[i] = 0;
}

// Streaming read floor: workgroup w sums the 16-byte words [w * per_wg,
// (w + 1) * per_wg) of src, each thread kDepth 16-byte loads in flight
// (unrolled), and writes its sum only if it equals a value no sum of these
// inputs takes, so that the loads stay but nothing is written.  The fastest
// a single launch can move a given number of bytes from HBM, over the load
// forms a kernel can use:
//   kKind 0  global_load_dwordx4
//   kKind 1  global_load_dwordx4 nt (__builtin_nontemporal_load)
//   kKind 2  buffer_load_dwordx4 through a resource covering the chunk: the
//            loads past its end return zeros without a request, so every
//            round issues all kDepth loads (no remainder loop)
//   kKind 3  the same with the nt bit
constexpr int kRawBufferWord3 = 0x00020000;  // untyped 32-bit buffer (gfx9 family)
constexpr int kCachePolicyNt = 2;            // buffer cache-policy bit NT (gfx940 family)

typedef float floatx4_t __attribute__((ext_vector_type(4)));

template <int kKind>
__device__ __forceinline__ float4 floor_load(const float4* p)
{
    if constexpr (kKind == 1) {
        const floatx4_t v = __builtin_nontemporal_load(reinterpret_cast<const floatx4_t*>(p));
        return make_float4(v.x, v.y, v.z, v.w);
    } else {
        return *p;
    }
}

template <int kKind, int kDepth>
__global__ __launch_bounds__(256) void read_floor_kernel(const float4* __restrict__ src, long long n16,
                                                         long long per_wg, float* __restrict__ sink)
{
    const long long lo = (long long)blockIdx.x * per_wg;
    const long long hi = lo + per_wg < n16 ? lo + per_wg : n16;
    float acc = 0.f;
    if constexpr (kKind >= 2) {
        // chunk bytes < 2^31 (host check): 32-bit offsets
        const unsigned n = (unsigned)(hi > lo ? hi - lo : 0);
        const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float4*>(src + lo), 0, n * 16u,
                                                          kRawBufferWord3);
        for (unsigned i = threadIdx.x; i < n; i += kDepth * 256) {
            float4 v[kDepth];
#pragma unroll
            for (int u = 0; u < kDepth; ++u)
                v[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      rs, (i + u * 256u) * 16u, 0, kKind == 3 ? kCachePolicyNt : 0));
#pragma unroll
            for (int u = 0; u < kDepth; ++u) acc += (v[u].x + v[u].y) + (v[u].z + v[u].w);
        }
    } else {
        long long i = lo + threadIdx.x;
        for (; i + (kDepth - 1) * 256 < hi; i += kDepth * 256) {
            float4 v[kDepth];
#pragma unroll
            for (int u = 0; u < kDepth; ++u)
                v[u] = floor_load<kKind>(&src[i + u * 256]);
#pragma unroll
            for (int u = 0; u < kDepth; ++u) acc += (v[u].x + v[u].y) + (v[u].z + v[u].w);
        }
        for (; i < hi; i += 256) {
            const float4 v = floor_load<kKind>(&src[i]);
            acc += (v.x + v.y) + (v.z + v.w);
        }
    }
    if (acc == -1234.5f) sink[blockIdx.x] = acc;
}

// MFMA floor: each wave runs `iters` rounds of 16 v_mfma_f32_32x32x16_bf16
// on two independent accumulators, operands pseudo-random per lane (so the
// matrix cores see real bit patterns), and writes its sum only if it equals a
// value no sum of these operands takes, so that the work stays but nothing is
// written.  The fastest a single launch can execute a given number of bf16
// MFMA flops: 2 x 32 x 32 x 16 per instruction, the instruction the prefill
// attention kernel's products run on.
typedef float floatx16_t __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

__global__ __launch_bounds__(256) void mfma_floor_kernel(int iters, float* __restrict__ sink)
{
    floatx16_t c0 = {}, c1 = {};
    bf16x8_t r[4];
    unsigned h = threadIdx.x * 2654435761u + blockIdx.x * 40503u + 12345u;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            h ^= h << 13;
            h ^= h >> 17;
            h ^= h << 5;
            r[i][e] = static_cast<__bf16>((float)(int)(h & 0xffffff) * (1.0f / 8388608.0f) - 1.0f);
        }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(r[u & 3], r[(u + 1) & 3], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(r[(u + 2) & 3], r[(u + 3) & 3], c1, 0, 0, 0);
        }
    }
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc += c0[i] + c1[i];
    if (acc == -1234.5f) sink[blockIdx.x] = acc;
}

}  // namespace

hipError_t load_small_ops_code()
{
    hipFuncAttributes a;
    return hipFuncGetAttributes(&a, reinterpret_cast<const void*>(&copy16_kernel));
}

hipError_t launch_mfma_floor(int n_wg, int iters, float* sink, hipStream_t s)
{
    if (n_wg < 1 || iters < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mfma_floor_kernel, dim3((unsigned)n_wg), dim3(256), 0, s, iters, sink);
    return hipGetLastError();
}

hipError_t launch_read_floor(const void* src, size_t bytes, int n_wg, int kind, int depth, float* sink,
                             hipStream_t s)
{
    const long long n16 = (long long)(bytes / 16);
    if (n16 == 0 || n_wg < 1 || kind < 0 || kind > 3 || (depth != 8 && depth != 16 && depth != 32))
        return hipErrorInvalidValue;
    const long long per_wg = (n16 + n_wg - 1) / n_wg;
    if (kind >= 2 && (per_wg + 32 * 256) * 16 >= (1ll << 31)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)n_wg), block(256);
    const float4* p = static_cast<const float4*>(src);
    auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, block, 0, s, p, n16, per_wg, sink); };
#define TLA_READ_FLOOR_DEPTHS(K)                        \
    if (depth == 8) go(read_floor_kernel<K, 8>);        \
    else if (depth == 16) go(read_floor_kernel<K, 16>); \
    else go(read_floor_kernel<K, 32>);
    if (kind == 0) { TLA_READ_FLOOR_DEPTHS(0) }
    else if (kind == 1) { TLA_READ_FLOOR_DEPTHS(1) }
    else if (kind == 2) { TLA_READ_FLOOR_DEPTHS(2) }
    else { TLA_READ_FLOOR_DEPTHS(3) }
#undef TLA_READ_FLOOR_DEPTHS
    return hipGetLastError();
}

hipError_t launch_zero(void* dst, size_t bytes, hipStream_t s)
{
    if (bytes == 0) return hipSuccess;
    const bool aligned = (reinterpret_cast<uintptr_t>(dst) & 15) == 0;
    const long long n16 = aligned ? (long long)(bytes / 16) : 0;
    if (n16 > 0) {
        long long blocks = (n16 + 255) / 256;
        if (blocks > 256 * 64) blocks = 256 * 64;
        hipLaunchKernelGGL(zero16_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                           static_cast<float4*>(dst), n16);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    const size_t done = (size_t)n16 * 16;
    if (done < bytes) {
        const long long rest = (long long)(bytes - done);
        long long blocks = (rest + 255) / 256;
        if (blocks > 4096) blocks = 4096;
        hipLaunchKernelGGL(zero1_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                           static_cast<unsigned char*>(dst) + done, rest);
        return hipGetLastError();
    }
    return hipSuccess;
}

hipError_t launch_rope(const RopeParams& p, hipStream_t s)
{
    const int total = (p.n_head + p.n_head_kv) * (p.head_dim / 2);
    hipLaunchKernelGGL(rope_kernel, dim3((total + 255) / 256), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_softmax(float* x, int size, hipStream_t s)
{
    hipLaunchKernelGGL(softmax_kernel, dim3(1), dim3(1024), 0, s, x, size);
    return hipGetLastError();
}

hipError_t launch_copy(void* dst, const void* src, size_t bytes, hipStream_t s)
{
    if (bytes == 0) return hipSuccess;
    const bool aligned = ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15) == 0;
    const long long n16 = aligned ? (long long)(bytes / 16) : 0;
    if (n16 > 0) {
        long long blocks = (n16 + 255) / 256;
        if (blocks > 256 * 64) blocks = 256 * 64;
        hipLaunchKernelGGL(copy16_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                           static_cast<float4*>(dst), static_cast<const float4*>(src), n16);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    const size_t done = (size_t)n16 * 16;
    if (done < bytes) {
        const long long rest = (long long)(bytes - done);
        long long blocks = (rest + 255) / 256;
        if (blocks > 4096) blocks = 4096;
        hipLaunchKernelGGL(copy1_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                           static_cast<unsigned char*>(dst) + done,
                           static_cast<const unsigned char*>(src) + done, rest);
        return hipGetLastError();
    }
    return hipSuccess;
}

}  // namespace tla
