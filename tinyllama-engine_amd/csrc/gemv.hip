// Matrix-vector products for the projections either side of the attention
// block, in the reference's weight formats (matmul(), src/ops.cpp:959-983,
// block layouts src/gguf.h:56-135), plus rmsnorm and vec_add.
//
// y[v][r] = sum_c W[r][c] * x[v][c] for up to 8 vectors v at once; W is read
// from HBM once per launch, so the kernel is HBM-bound (about 0.56 B of
// weights per multiply-add at Q4_0, 2 B at F16).  Optional fusions:
//   - rmsnorm prologue (src/ops.cpp:1003-1055): each workgroup normalises x
//     into LDS, so the input half of the attention block (rmsnorm, Wq, Wk,
//     Wv; src/forward.cpp:180-190) is one launch with three segments;
//   - residual epilogue: y += W.x, the output half (Wo then vec_add,
//     src/forward.cpp:210-213).
//
// Work decomposition: the weights of a row are cut into units of 64 (two
// Q8_0/Q4_0 blocks, 128 B of F16, 256 B of F32, a quarter of a Q6_K
// super-block).  With cols a multiple of 64 every Q8_0/Q4_0 unit starts on a
// 4-byte boundary, so it is read with aligned dword loads; Q6_K super-blocks
// (210 B) are 2-byte aligned and read with 16-bit loads.  32 lanes serve a
// row when it has at most 32 units (cols <= 2048), else 64; the lanes' dot
// products meet in a shuffle reduction.  x sits in LDS, read as float4.
//
// Products and sums are fp32 but grouped differently from the reference's
// sequential loops, so results match it to fp32 rounding, not bit for bit.
#include "rope_math.h"
#include "tla_internal.h"

namespace tla {
namespace {

constexpr int kThreads = 256;
constexpr int kUnit = 64;  // weights per lane step

__device__ __forceinline__ float half_bits_to_float(unsigned h)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h)));
}

// x[c0 .. c0+15] of vector v from LDS (16 floats).
__device__ __forceinline__ void lds16(const float* xs, int c0, float (&o)[16])
{
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 t = *reinterpret_cast<const float4*>(xs + c0 + 4 * i);
        o[4 * i + 0] = t.x;
        o[4 * i + 1] = t.y;
        o[4 * i + 2] = t.z;
        o[4 * i + 3] = t.w;
    }
}

// ---- one 64-weight unit of a row, dotted with each vector ----------------

template <int kType>
struct Unit;

template <>
struct Unit<kF32> {
    float w[64];
    __device__ void load(const unsigned char* row, int u)
    {
        const float4* p = reinterpret_cast<const float4*>(row + u * 256);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float4 t = p[i];
            w[4 * i] = t.x;
            w[4 * i + 1] = t.y;
            w[4 * i + 2] = t.z;
            w[4 * i + 3] = t.w;
        }
    }
    __device__ float dot(const float* xs, int u) const
    {
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float xv[16];
            lds16(xs, u * 64 + 16 * q, xv);
#pragma unroll
            for (int i = 0; i < 16; ++i) s += w[16 * q + i] * xv[i];
        }
        return s;
    }
};

template <>
struct Unit<kF16> {
    uint4 raw[8];  // 64 halves
    __device__ void load(const unsigned char* row, int u)
    {
        const uint4* p = reinterpret_cast<const uint4*>(row + u * 128);
#pragma unroll
        for (int i = 0; i < 8; ++i) raw[i] = p[i];
    }
    __device__ float dot(const float* xs, int u) const
    {
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float xv[16];
            lds16(xs, u * 64 + 16 * q, xv);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint4 r = raw[2 * q + i];
                const unsigned wd[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    s += half_bits_to_float(wd[j] & 0xFFFFu) * xv[8 * i + 2 * j];
                    s += half_bits_to_float(wd[j] >> 16) * xv[8 * i + 2 * j + 1];
                }
            }
        }
        return s;
    }
};

// Two Q8_0 blocks (68 bytes, 17 dwords): d0 | qs0[32] | d1 | qs1[32].
template <>
struct Unit<kQ8_0> {
    unsigned dw[17];
    __device__ void load(const unsigned char* row, int u)
    {
        const unsigned* p = reinterpret_cast<const unsigned*>(row + u * 68);
#pragma unroll
        for (int i = 0; i < 17; ++i) dw[i] = p[i];
    }
    // byte b (0..67) of the pair, as a signed value
    __device__ int sbyte(int b) const
    {
        return static_cast<int>(static_cast<signed char>((dw[b >> 2] >> (8 * (b & 3))) & 0xFFu));
    }
    __device__ float dot(const float* xs, int u) const
    {
        float s = 0.f;
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            const int base = 34 * blk;  // byte offset of the block
            const float d = half_bits_to_float(blk == 0 ? (dw[0] & 0xFFFFu) : (dw[8] >> 16));
            float bs = 0.f;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                float xv[16];
                lds16(xs, u * 64 + 32 * blk + 16 * q, xv);
#pragma unroll
                for (int i = 0; i < 16; ++i) bs += static_cast<float>(sbyte(base + 2 + 16 * q + i)) * xv[i];
            }
            s += d * bs;
        }
        return s;
    }
};

// Two Q4_0 blocks (36 bytes, 9 dwords): d0 | qs0[16] | d1 | qs1[16]; byte j
// of qs holds element j (low nibble) and j + 16 (high nibble), value - 8.
template <>
struct Unit<kQ4_0> {
    unsigned dw[9];
    __device__ void load(const unsigned char* row, int u)
    {
        const unsigned* p = reinterpret_cast<const unsigned*>(row + u * 36);
#pragma unroll
        for (int i = 0; i < 9; ++i) dw[i] = p[i];
    }
    __device__ unsigned ubyte(int b) const { return (dw[b >> 2] >> (8 * (b & 3))) & 0xFFu; }
    __device__ float dot(const float* xs, int u) const
    {
        float s = 0.f;
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            const int base = 18 * blk;
            const float d = half_bits_to_float(blk == 0 ? (dw[0] & 0xFFFFu) : (dw[4] >> 16));
            float lo[16], hi[16];
            lds16(xs, u * 64 + 32 * blk, lo);
            lds16(xs, u * 64 + 32 * blk + 16, hi);
            float bs = 0.f;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const unsigned q = ubyte(base + 2 + j);
                bs += static_cast<float>(static_cast<int>(q & 0xFu) - 8) * lo[j];
                bs += static_cast<float>(static_cast<int>(q >> 4) - 8) * hi[j];
            }
            s += d * bs;
        }
        return s;
    }
};

// A quarter of a Q6_K super-block (ql[128] qh[64] scales[16] d; 210 bytes):
// half h, rows l = 16m .. 16m+15 of that half, i.e. elements
// 128h + l + {0, 32, 64, 96}, the grouping of the reference's loops.
template <>
struct Unit<kQ6_K> {
    unsigned short qla[8], qlb[8], qh[8];  // ql[64h+16m ..], ql[64h+32+16m ..], qh[32h+16m ..]
    int sc[4];
    float d;
    __device__ void load(const unsigned char* row, int u)
    {
        const int b = u >> 2, q = u & 3, h = q >> 1, m = q & 1;
        const unsigned char* sb = row + 210 * b;
        const unsigned short* a = reinterpret_cast<const unsigned short*>(sb + 64 * h + 16 * m);
        const unsigned short* bb = reinterpret_cast<const unsigned short*>(sb + 64 * h + 32 + 16 * m);
        const unsigned short* c = reinterpret_cast<const unsigned short*>(sb + 128 + 32 * h + 16 * m);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            qla[i] = a[i];
            qlb[i] = bb[i];
            qh[i] = c[i];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) sc[k] = static_cast<signed char>(sb[192 + 8 * h + m + 2 * k]);
        d = half_bits_to_float(*reinterpret_cast<const unsigned short*>(sb + 208));
    }
    __device__ float dot(const float* xs, int u) const
    {
        const int b = u >> 2, q = u & 3, h = q >> 1, m = q & 1;
        const int c0 = 256 * b + 128 * h + 16 * m;
        float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float xv[16];
            lds16(xs, c0 + 32 * k, xv);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const unsigned la = (qla[i >> 1] >> (8 * (i & 1))) & 0xFFu;
                const unsigned lb = (qlb[i >> 1] >> (8 * (i & 1))) & 0xFFu;
                const unsigned hb = (qh[i >> 1] >> (8 * (i & 1))) & 0xFFu;
                const unsigned lo4 = (k == 0) ? (la & 0xFu) : (k == 1) ? (lb & 0xFu) : (k == 2) ? (la >> 4) : (lb >> 4);
                const int qv = static_cast<int>(lo4 | (((hb >> (2 * k)) & 3u) << 4)) - 32;
                s4[k] += static_cast<float>(qv) * xv[i];
            }
        }
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) s += d * static_cast<float>(sc[k]) * s4[k];
        return s;
    }
};

// ---- kernel ------------------------------------------------------------------

template <int kType, int kLanesPerRow>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const GemvParams p)
{
    extern __shared__ float xs_all[];  // [n_vec][cols]
    __shared__ float s_red[kThreads / 64][kGemvMaxVec];

    // Stage x (rmsnorm'ed when asked) in LDS.
    for (int v = 0; v < p.n_vec; ++v) {
        const float* xv = p.x + v * p.x_stride;
        float* xs = xs_all + v * p.cols;
        if (p.norm_w) {
            float ss = 0.f;
            for (int c = threadIdx.x; c < p.cols; c += kThreads) ss += xv[c] * xv[c];
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
            if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6][0] = ss;
            __syncthreads();
            ss = 0.f;
#pragma unroll
            for (int w = 0; w < kThreads / 64; ++w) ss += s_red[w][0];
            __syncthreads();
            const float rms = 1.0f / sqrtf(ss / static_cast<float>(p.cols) + p.eps);
            for (int c = threadIdx.x; c < p.cols; c += kThreads) xs[c] = xv[c] * rms * p.norm_w[c];
        } else {
            for (int c = threadIdx.x; c < p.cols; c += kThreads) xs[c] = xv[c];
        }
    }
    __syncthreads();

    constexpr int kRowsPerWave = 64 / kLanesPerRow;
    const int lane = threadIdx.x & 63;
    const int sub = lane / kLanesPerRow;  // which row of the wave's group
    const int l = lane % kLanesPerRow;
    const int wave = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int n_waves = gridDim.x * (kThreads / 64);
    const int units = p.cols / kUnit;

    for (int r0 = wave * kRowsPerWave; r0 < p.total_rows; r0 += n_waves * kRowsPerWave) {
        const int r = r0 + sub;
        // segment of row r (boundaries are per lane group)
        int seg = 0, row = r;
        while (seg + 1 < p.n_seg && row >= p.seg[seg].rows) {
            row -= p.seg[seg].rows;
            ++seg;
        }
        const bool valid = r < p.total_rows;
        const unsigned char* wrow = p.seg[seg].w + static_cast<long long>(valid ? row : 0) * p.row_bytes;
        float acc[kGemvMaxVec];
#pragma unroll
        for (int v = 0; v < kGemvMaxVec; ++v) acc[v] = 0.f;
        if (valid) {
            for (int u = l; u < units; u += kLanesPerRow) {
                Unit<kType> un;
                un.load(wrow, u);
#pragma unroll
                for (int v = 0; v < kGemvMaxVec; ++v)
                    if (v < p.n_vec) acc[v] += un.dot(xs_all + v * p.cols, u);
            }
        }
#pragma unroll
        for (int v = 0; v < kGemvMaxVec; ++v) {
            if (v >= p.n_vec) break;
            float t = acc[v];
#pragma unroll
            for (int o = kLanesPerRow / 2; o >= 1; o >>= 1) t += __shfl_xor(t, o);
            if (valid && l == 0) {
                float* dst = p.seg[seg].out + v * p.seg[seg].out_stride + row;
                *dst = p.add ? *dst + t : t;
            }
        }
    }
}

__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(float* out, const float* x,
                                                           const float* w, int size, float eps)
{
    __shared__ float s_red[kThreads / 64];
    float ss = 0.f;
    for (int c = threadIdx.x; c < size; c += kThreads) ss += x[c] * x[c];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = 0.f;
#pragma unroll
    for (int i = 0; i < kThreads / 64; ++i) ss += s_red[i];
    const float rms = 1.0f / sqrtf(ss / static_cast<float>(size) + eps);
    for (int c = threadIdx.x; c < size; c += kThreads) out[c] = x[c] * rms * w[c];
}

__global__ __launch_bounds__(kThreads) void vec_add_kernel(float* out, const float* x, int size)
{
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i < size) out[i] += x[i];
}

template <int kType>
hipError_t launch_typed(const GemvParams& p, hipStream_t s)
{
    const int units = p.cols / kUnit;
    const size_t lds = static_cast<size_t>(p.n_vec) * p.cols * sizeof(float);
    const int rows_per_wg = (kThreads / 64) * (units <= 32 ? 2 : 1);
    int blocks = (p.total_rows + rows_per_wg - 1) / rows_per_wg;
    if (blocks > 2048) blocks = 2048;
    if (units <= 32)
        hipLaunchKernelGGL((gemv_kernel<kType, 32>), dim3(blocks), dim3(kThreads), lds, s, p);
    else
        hipLaunchKernelGGL((gemv_kernel<kType, 64>), dim3(blocks), dim3(kThreads), lds, s, p);
    return hipGetLastError();
}

}  // namespace

long long weight_row_bytes(int type, int cols)
{
    switch (type) {
    case kF32: return 4LL * cols;
    case kF16: return 2LL * cols;
    case kQ8_0: return 34LL * (cols / 32);
    case kQ4_0: return 18LL * (cols / 32);
    case kQ6_K: return 210LL * (cols / 256);
    default: return 0;
    }
}

hipError_t launch_gemv(int type, const GemvParams& p, hipStream_t s)
{
    switch (type) {
    case kF32: return launch_typed<kF32>(p, s);
    case kF16: return launch_typed<kF16>(p, s);
    case kQ8_0: return launch_typed<kQ8_0>(p, s);
    case kQ4_0: return launch_typed<kQ4_0>(p, s);
    case kQ6_K: return launch_typed<kQ6_K>(p, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_rmsnorm(float* out, const float* x, const float* w, int size, float eps,
                          hipStream_t s)
{
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(kThreads), 0, s, out, x, w, size, eps);
    return hipGetLastError();
}

hipError_t launch_vec_add(float* out, const float* x, int size, hipStream_t s)
{
    hipLaunchKernelGGL(vec_add_kernel, dim3((size + kThreads - 1) / kThreads), dim3(kThreads), 0, s,
                       out, x, size);
    return hipGetLastError();
}

}  // namespace tla
