// Matrix products for a batch of tokens (the prompt): Y[t][r] (+)= W[r] . X[t]
// with W in the reference's weight formats (matmul(), src/ops.cpp:959-983,
// block layouts src/gguf.h:56-135) dequantised in registers and multiplied
// on the fp32 matrix cores (v_mfma_f32_32x32x2f32).  This is the batched form
// of the projections forward() makes per token (src/forward.cpp:180-228) when
// the prompt runs through the model at once.
//
// Tiling: a workgroup (4 waves) owns 128 weight rows x 128 tokens; a wave
// owns 32 rows x all 128 tokens (four 32x32 accumulators), so each
// dequantised weight feeds four MFMAs.  The K dimension advances in chunks
// of 32 columns (one Q8_0 / Q4_0 block): the chunk's X tile [128 tokens][32
// columns] is staged once in LDS (row pitch 33 floats: the lanes of an MFMA
// B operand read 32 tokens at one column, which then fall in 32 different
// banks) and read by all four waves; each lane loads its own weight row's
// block and dequantises it into A operands.
//
// The contraction order inside a chunk is (s, s + 16) for s = 0..15: MFMA
// step s takes columns s (A lanes 0-31) and s + 16 (lanes 32-63).  That
// order follows the Q4_0 byte layout (byte s holds elements s and s + 16)
// and is applied to X identically, so the sum is unchanged.
//
// fp32 products and fp32 accumulation in a different order than the
// reference's sequential loops: results agree to fp32 rounding.
#include "launch_extra.h"
#include "row_math.h"
#include "tla_internal.h"

namespace tla {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kTileRows = 128;  // weight rows per workgroup (32 per wave)
constexpr int kTileToks = 128;  // tokens per workgroup
constexpr int kChunk = 32;      // columns per K step
constexpr int kPitch = 33;      // LDS floats per staged token row

__device__ __forceinline__ float half_to_float(unsigned h)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h)));
}

// One lane's view of a weight row's 32-column chunk: the 16 values at
// columns s + 16k (s = 0..15) for the lane's half k.
template <int kType>
struct Chunk;

template <>
struct Chunk<kF32> {
    float4 w[4];
    __device__ void load(const unsigned char* row, int c, int k)
    {
        const float4* p = reinterpret_cast<const float4*>(row + 4 * (kChunk * c + 16 * k));
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = p[i];
    }
    __device__ float value(int s) const
    {
        const float4 v = w[s >> 2];
        const int e = s & 3;
        return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
    }
};

template <>
struct Chunk<kF16> {
    uint4 h[2];
    __device__ void load(const unsigned char* row, int c, int k)
    {
        const uint4* p = reinterpret_cast<const uint4*>(row + 2 * (kChunk * c + 16 * k));
        h[0] = p[0];
        h[1] = p[1];
    }
    __device__ float value(int s) const
    {
        const uint4 v = h[s >> 3];
        const int d = (s >> 1) & 3;
        const unsigned w = d == 0 ? v.x : d == 1 ? v.y : d == 2 ? v.z : v.w;
        return half_to_float((s & 1) ? (w >> 16) : (w & 0xFFFFu));
    }
};

// Q8_0 block: d (fp16) | qs[32] int8; column e is qs[e].
template <>
struct Chunk<kQ8_0> {
    unsigned q[4];
    float d;
    __device__ void load(const unsigned char* row, int c, int k)
    {
        const unsigned char* b = row + 34 * c;
        d = half_to_float(b[0] | (b[1] << 8));
        // 16 bytes at an even address: 16-bit aligned loads, assembled
        const unsigned short* p = reinterpret_cast<const unsigned short*>(b + 2 + 16 * k);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = p[2 * i] | (static_cast<unsigned>(p[2 * i + 1]) << 16);
    }
    __device__ float value(int s) const
    {
        const int v = static_cast<signed char>((q[s >> 2] >> (8 * (s & 3))) & 0xFFu);
        return static_cast<float>(v) * d;
    }
};

// Q4_0 block: d (fp16) | qs[16]; byte j holds column j (low nibble) and
// j + 16 (high nibble), value - 8.  Half k takes the nibble 4k of byte s.
template <>
struct Chunk<kQ4_0> {
    unsigned q[4];
    float d;
    int shift;
    __device__ void load(const unsigned char* row, int c, int k)
    {
        const unsigned char* b = row + 18 * c;
        d = half_to_float(b[0] | (b[1] << 8));
        const unsigned short* p = reinterpret_cast<const unsigned short*>(b + 2);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = p[2 * i] | (static_cast<unsigned>(p[2 * i + 1]) << 16);
        shift = 4 * k;
    }
    __device__ float value(int s) const
    {
        const int v = static_cast<int>((q[s >> 2] >> (8 * (s & 3) + shift)) & 0xFu) - 8;
        return static_cast<float>(v) * d;
    }
};

// Y (+)= W . X for the segments of p (each a multiple of 32 rows, so a
// wave's 32 rows lie in one segment).
template <int kType>
__global__ __launch_bounds__(kThreads) void gemm_kernel(const GemmParams p)
{
    __shared__ float xs[2][kTileToks * kPitch];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int i = lane & 31, k = lane >> 5;
    const int row0 = blockIdx.x * kTileRows + wave * 32;  // the wave's 32 rows
    const int tok0 = blockIdx.y * kTileToks;
    // this workgroup's column chunks [c0, c1): all, or its split's share
    const int n_all = p.cols / kChunk;
    const int c0 = static_cast<int>(static_cast<long long>(n_all) * blockIdx.z / gridDim.z);
    const int c1 = static_cast<int>(static_cast<long long>(n_all) * (blockIdx.z + 1) / gridDim.z);

    // the wave's segment (uniform: segment sizes are multiples of 32)
    int seg = 0, srow = row0;
    while (seg + 1 < p.n_seg && srow >= p.seg[seg].rows) {
        srow -= p.seg[seg].rows;
        ++seg;
    }
    const bool rows_valid = row0 < p.total_rows;
    const GemvSegment S = p.seg[seg];
    const unsigned char* wrow = S.w + static_cast<long long>(rows_valid ? srow + i : 0) * p.row_bytes;

    // X staging: thread tid moves tokens tid/8 + 32m (m = 0..3), columns
    // 4(tid%8) .. +3 of a chunk; rows past n_tok stage zeros.
    const int st = tid >> 3, sc = 4 * (tid & 7);
    float4 xr[4];
    auto load_x = [&](int c) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int t = tok0 + st + 32 * m;
            xr[m] = t < p.n_tok
                        ? *reinterpret_cast<const float4*>(p.x + static_cast<long long>(t) * p.x_stride +
                                                           kChunk * c + sc)
                        : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto store_x = [&](int b) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            float* d = xs[b] + (st + 32 * m) * kPitch + sc;
            d[0] = xr[m].x;
            d[1] = xr[m].y;
            d[2] = xr[m].z;
            d[3] = xr[m].w;
        }
    };

    floatx16 acc[4] = {};
    Chunk<kType> wc, wn;
    wc.load(wrow, c0, k);
    load_x(c0);
    store_x(0);
    __syncthreads();
    for (int c = c0; c < c1; ++c) {
        const bool more = c + 1 < c1;
        if (more) {
            wn.load(wrow, c + 1, k);
            load_x(c + 1);
        }
        const float* xt = xs[(c - c0) & 1] + i * kPitch + 16 * k;  // token 32h + i at h * 32 rows
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const float a = wc.value(s);
#pragma unroll
            for (int h = 0; h < 4; ++h)
                acc[h] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, xt[32 * h * kPitch + s], acc[h], 0, 0, 0);
        }
        if (more) {
            store_x((c + 1 - c0) & 1);
            wc = wn;
        }
        __syncthreads();
    }

    // D[r][t]: lane holds token (lane % 32) of each subtile and rows
    // (v % 4) + 8 (v / 4) + 4 (lane / 32) of the wave's 32.
    if (!rows_valid) return;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        const int t = tok0 + 32 * h + i;
        if (t >= p.n_tok) continue;
        if (gridDim.z > 1) {
            // partial tile: part[split][t][row], dense over all rows
            float* o = p.part + (static_cast<long long>(blockIdx.z) * p.n_tok + t) * p.total_rows + row0;
#pragma unroll
            for (int v = 0; v < 16; ++v) o[(v & 3) + 8 * (v >> 2) + 4 * k] = acc[h][v];
            continue;
        }
        float* o = S.out + static_cast<long long>(t) * S.out_stride + srow;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int r = (v & 3) + 8 * (v >> 2) + 4 * k;
            o[r] = p.add ? o[r] + acc[h][v] : acc[h][v];
        }
    }
}

// out[t][row] (+)= sum over splits of part[split][t][row], splits in order.
__global__ __launch_bounds__(kThreads) void gemm_reduce_kernel(const GemmParams p)
{
    const long long n = static_cast<long long>(p.n_tok) * p.total_rows;
    const long long idx = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (idx >= n) return;
    const int t = static_cast<int>(idx / p.total_rows);
    int r = static_cast<int>(idx - static_cast<long long>(t) * p.total_rows);
    float sum = 0.f;
    for (int sp = 0; sp < p.k_splits; ++sp) sum += p.part[sp * n + idx];
    int seg = 0;
    while (seg + 1 < p.n_seg && r >= p.seg[seg].rows) {
        r -= p.seg[seg].rows;
        ++seg;
    }
    float* o = p.seg[seg].out + static_cast<long long>(t) * p.seg[seg].out_stride + r;
    *o = p.add ? *o + sum : sum;
}

template <int kType>
hipError_t launch_typed(const GemmParams& p, hipStream_t s)
{
    const int splits = p.k_splits > 1 ? p.k_splits : 1;
    const dim3 grid((p.total_rows + kTileRows - 1) / kTileRows, (p.n_tok + kTileToks - 1) / kTileToks, splits);
    hipLaunchKernelGGL(gemm_kernel<kType>, grid, dim3(kThreads), 0, s, p);
    if (splits > 1) {
        const long long n = static_cast<long long>(p.n_tok) * p.total_rows;
        hipLaunchKernelGGL(gemm_reduce_kernel, dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)),
                           dim3(kThreads), 0, s, p);
    }
    return hipGetLastError();
}

// x[t] = x[t] / sqrt(mean(x[t]^2) + eps) * w for each of n_tok rows (one
// workgroup per row), into out.
__global__ __launch_bounds__(kThreads) void rmsnorm_rows_kernel(float* out, const float* x, const float* w,
                                                                int size, float eps)
{
    __shared__ float s_red[kThreads / 64];
    const float* xr = x + static_cast<long long>(blockIdx.x) * size;
    float* o = out + static_cast<long long>(blockIdx.x) * size;
    const float ss = row_sum_squares<kThreads>(xr, size, s_red);
    const float rms = 1.0f / sqrtf(ss / static_cast<float>(size) + eps);
    for (int c = threadIdx.x; c < size; c += kThreads) o[c] = xr[c] * rms * w[c];
}

// h[t][c] = silu(h[t][c]) * h[t][n_ff + c] in place, rows of 2 n_ff floats
// (gate then up), with the reference's operation order (src/ops.cpp:1107-1148).
__global__ __launch_bounds__(kThreads) void swiglu_rows_kernel(float* h, int n_ff)
{
    float* g = h + static_cast<long long>(blockIdx.y) * 2 * n_ff;
    const int c = blockIdx.x * kThreads + threadIdx.x;
    if (c < n_ff) {
        const float v = g[c];
        const float sigmoid = 1.0f / (1.0f + expf(-v));
        g[c] = (v * sigmoid) * g[n_ff + c];
    }
}

// Q6_K super-block (ql[128] qh[64] scales[16] d; 210 bytes, 256 values):
// value r = d * scales[8h + 2k + l / 16] * q with h = r / 128, k = (r % 128)
// / 32, l = r % 32, q = (4 bits of ql[64h + 32(k % 2) + l], low for k < 2)
// | (2 bits 2k of qh[32h + l]) << 4, minus 32 (src/gguf.h layout; the
// reference's embed_token() order of products).
__device__ float q6k_value(const unsigned char* blk, int r)
{
    const int h = r >> 7, k = (r & 127) >> 5, l = r & 31;
    const unsigned char* ql = blk + 64 * h;
    const unsigned char* qh = blk + 128 + 32 * h;
    const signed char* sc = reinterpret_cast<const signed char*>(blk + 192) + 8 * h;
    const float d = half_to_float(blk[208] | (blk[209] << 8));
    const int lo = (k & 1) ? ql[l + 32] : ql[l];
    const int q = ((k < 2 ? (lo & 0x0F) : (lo >> 4)) | (((qh[l] >> (2 * k)) & 3) << 4)) - 32;
    return d * static_cast<float>(sc[(l >> 4) + 2 * k]) * static_cast<float>(q);
}

// out[row][4j .. 4j + 3] = the fp32 values of columns 4j .. 4j + 3 of a
// weight row, one thread per float4 of output, so the threads of a wave
// store 1 KiB contiguously.  The values are the ones gemm_kernel multiplies
// (Chunk<>::value; Q6_K by q6k_value).  Blocks start at even byte offsets,
// so the quantised bytes are read as 16-bit halves.
template <int kType>
__global__ __launch_bounds__(kThreads) void dequant_rows_kernel(const unsigned char* __restrict__ w,
                                                                long long row_bytes, int rows, int cols,
                                                                float* __restrict__ out)
{
    const int n4 = cols / 4;
    const long long g = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (g >= static_cast<long long>(rows) * n4) return;
    const int row = static_cast<int>(g / n4);
    const int col = 4 * static_cast<int>(g - static_cast<long long>(row) * n4);
    const unsigned char* wrow = w + row * row_bytes;
    float4 v;
    if constexpr (kType == kF32) {
        v = *reinterpret_cast<const float4*>(wrow + 4LL * col);
    } else if constexpr (kType == kF16) {
        const uint2 h = *reinterpret_cast<const uint2*>(wrow + 2LL * col);
        v = make_float4(half_to_float(h.x & 0xFFFFu), half_to_float(h.x >> 16), half_to_float(h.y & 0xFFFFu),
                        half_to_float(h.y >> 16));
    } else if constexpr (kType == kQ6_K) {
        const unsigned char* blk = wrow + 210LL * (col >> 8);
        const int r = col & 255;
        v = make_float4(q6k_value(blk, r), q6k_value(blk, r + 1), q6k_value(blk, r + 2), q6k_value(blk, r + 3));
    } else {
        constexpr int kBlock = kType == kQ8_0 ? 34 : 18;
        const unsigned char* blk = wrow + static_cast<long long>(kBlock) * (col >> 5);
        const unsigned short* hw = reinterpret_cast<const unsigned short*>(blk);
        const float d = half_to_float(hw[0]);
        const int cb = col & 31;
        if constexpr (kType == kQ8_0) {
            // columns cb .. cb + 3 are qs[cb .. cb + 3]
            const unsigned q = hw[1 + cb / 2] | (static_cast<unsigned>(hw[2 + cb / 2]) << 16);
            v = make_float4(static_cast<float>(static_cast<signed char>(q & 0xFFu)) * d,
                            static_cast<float>(static_cast<signed char>((q >> 8) & 0xFFu)) * d,
                            static_cast<float>(static_cast<signed char>((q >> 16) & 0xFFu)) * d,
                            static_cast<float>(static_cast<signed char>(q >> 24)) * d);
        } else {
            // column e < 16 is the low nibble of qs[e], e >= 16 the high nibble of qs[e - 16]
            const int b = cb & 15, shift = (cb >> 4) * 4;
            const unsigned q = hw[1 + b / 2] | (static_cast<unsigned>(hw[2 + b / 2]) << 16);
            v = make_float4(static_cast<float>(static_cast<int>((q >> shift) & 0xFu) - 8) * d,
                            static_cast<float>(static_cast<int>((q >> (8 + shift)) & 0xFu) - 8) * d,
                            static_cast<float>(static_cast<int>((q >> (16 + shift)) & 0xFu) - 8) * d,
                            static_cast<float>(static_cast<int>((q >> (24 + shift)) & 0xFu) - 8) * d);
        }
    }
    *reinterpret_cast<float4*>(out + static_cast<long long>(row) * cols + col) = v;
}

}  // namespace

hipError_t launch_dequant_rows(int type, const unsigned char* w, long long row_bytes, int rows, int cols,
                               float* out, hipStream_t s)
{
    if (rows < 1 || cols < kChunk || cols % kChunk != 0 || (type == kQ6_K && cols % 256 != 0))
        return hipErrorInvalidValue;
    const long long n = static_cast<long long>(rows) * (cols / 4);
    const dim3 grid(static_cast<unsigned>((n + kThreads - 1) / kThreads));
    switch (type) {
    case kF32: hipLaunchKernelGGL(dequant_rows_kernel<kF32>, grid, dim3(kThreads), 0, s, w, row_bytes, rows, cols, out); break;
    case kF16: hipLaunchKernelGGL(dequant_rows_kernel<kF16>, grid, dim3(kThreads), 0, s, w, row_bytes, rows, cols, out); break;
    case kQ8_0: hipLaunchKernelGGL(dequant_rows_kernel<kQ8_0>, grid, dim3(kThreads), 0, s, w, row_bytes, rows, cols, out); break;
    case kQ4_0: hipLaunchKernelGGL(dequant_rows_kernel<kQ4_0>, grid, dim3(kThreads), 0, s, w, row_bytes, rows, cols, out); break;
    case kQ6_K: hipLaunchKernelGGL(dequant_rows_kernel<kQ6_K>, grid, dim3(kThreads), 0, s, w, row_bytes, rows, cols, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

bool gemm_supported(int type) { return type == kF32 || type == kF16 || type == kQ8_0 || type == kQ4_0; }

hipError_t launch_gemm(int type, const GemmParams& p, hipStream_t s)
{
    switch (type) {
    case kF32: return launch_typed<kF32>(p, s);
    case kF16: return launch_typed<kF16>(p, s);
    case kQ8_0: return launch_typed<kQ8_0>(p, s);
    case kQ4_0: return launch_typed<kQ4_0>(p, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_rmsnorm_rows(float* out, const float* x, const float* w, int n_rows, int size, float eps,
                               hipStream_t s)
{
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(n_rows), dim3(kThreads), 0, s, out, x, w, size, eps);
    return hipGetLastError();
}

hipError_t launch_swiglu_rows(float* h, int n_rows, int n_ff, hipStream_t s)
{
    hipLaunchKernelGGL(swiglu_rows_kernel, dim3((n_ff + kThreads - 1) / kThreads, n_rows), dim3(kThreads), 0,
                       s, h, n_ff);
    return hipGetLastError();
}

}  // namespace tla
