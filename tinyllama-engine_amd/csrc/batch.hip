// Batched-prompt helpers (tla_prefill_forward, tla_matmul_batch):
//
// stream_product_kernel: the projections of a batch of up to 64 tokens with
//   the weights dequantised in registers (matmul(), src/ops.cpp:959-983,
//   block layouts src/gguf.h:56-135): the batched form of the projections
//   forward() makes per token (src/forward.cpp:180-228) when the prompt runs
//   through the model at once.  Longer batches: split_product.hip.
// rmsnorm_rows_kernel, swiglu_rows_kernel: rmsnorm and SwiGLU over every
//   token row of the batch (src/forward.cpp:180-184, 215-225).
#include "row_math.h"
#include "batch.h"

namespace tla {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float half_to_float(unsigned h)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h)));
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

// x[t] += the split product's K-range sums, then rmsnorm of the row into
// out: the product's reduce launch and the rmsnorm launch after it as one.
// Sums in the reduce launch's order (ranges in order, then added to x), the
// rmsnorm's in row_sum_squares' (16-byte pieces t, t + kThreads, ...).
__global__ __launch_bounds__(kThreads) void reduce_rmsnorm_rows_kernel(float* x, const float* part, int k_splits,
                                                                       long long plane, float* out, const float* w,
                                                                       int size, float eps)
{
    __shared__ float s_red[kThreads / 64];
    const long long row = static_cast<long long>(blockIdx.x) * size;
    float4* const xr = reinterpret_cast<float4*>(x + row);
    const float4* const pr = reinterpret_cast<const float4*>(part + row);
    const long long plane4 = plane / 4;
    float ss = 0.f;
    for (int c4 = threadIdx.x; c4 < size / 4; c4 += kThreads) {
        float4 a = pr[c4];
        for (int z = 1; z < k_splits; ++z) {
            const float4 b = pr[z * plane4 + c4];
            a = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
        }
        const float4 o = xr[c4];
        const float4 v = make_float4(o.x + a.x, o.y + a.y, o.z + a.z, o.w + a.w);
        xr[c4] = v;
        ss += sum_sq4(v);
    }
    ss = block_sum<kThreads>(ss, s_red);
    const float rms = 1.0f / sqrtf(ss / static_cast<float>(size) + eps);
    float* const o = out + row;
    const float* const xs = x + row;  // this thread's own stores, read back
    for (int c4 = threadIdx.x; c4 < size / 4; c4 += kThreads)
        for (int e = 0; e < 4; ++e) o[4 * c4 + e] = xs[4 * c4 + e] * rms * w[4 * c4 + e];
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

// ---- stream_product_kernel --------------------------------------------------
// The projections of a batch of up to 64 tokens with the weights dequantised
// in registers (no fp32 copy of the matrix): out[t][row] (+)= sum_k W[row][k]
// x[t][k] for 16 weight rows and 16 kNT tokens per workgroup (blockIdx.y
// selects the token chunk).  v_mfma_f32_16x16x4f32 with the tokens as the A
// operand and the weight rows as the B operand, so that lane l = 16 g + c
// supplies token c's and row c's value of k slot g, and holds the result of
// tokens 4 g .. 4 g + 3 for row c.  The k order inside a 32-value block is
// free as long as A and B follow it: slot g of MFMA step s (s = 0..7) takes
// value 8 g + s, except for Q4_0, where it takes (g / 2) 16 + (g % 2) 8 + s
// -- bytes (g % 2) 8 .. + 7 of the block, low nibbles for g < 2, high for
// g >= 2 -- so that every lane reads 8 contiguous weights and 8 contiguous x
// values per block.  The four waves take every fourth block of the rows,
// each keeping the loads of its next blocks in flight, and add their sums in
// LDS in wave order, so the result is the same from run to run.
constexpr int kStreamWaves = 4;

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma16(float a, float b, floatx4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// One block's operands for one lane as loaded: the weights' raw bits (F32 8
// floats, F16 8 halves, Q8_0 / Q4_0 12 bytes holding the lane's 8 bytes of
// qs, and the scale for the lanes that read from the block's start) and 8 x
// values per token tile.  Nothing is computed from them until the block's
// turn comes, so that the loads of the blocks ahead stay in flight.
template <int kType, int kNT>
struct StreamStage {
    static constexpr int kWords = kType == kF32 ? 8 : kType == kF16 ? 4 : 3;
    unsigned u[kWords];
    float4 xa[kNT], xb[kNT];
};

template <int kType, int kNT>
__device__ __forceinline__ void stream_load(StreamStage<kType, kNT>& st, const unsigned char* wrow,
                                            const float* const (&xr)[kNT], int blk, int g)
{
    if constexpr (kType == kF32) {
        const uint4* q = reinterpret_cast<const uint4*>(wrow + 4LL * (32 * blk + 8 * g));
        const uint4 a = q[0], b = q[1];
        st.u[0] = a.x; st.u[1] = a.y; st.u[2] = a.z; st.u[3] = a.w;
        st.u[4] = b.x; st.u[5] = b.y; st.u[6] = b.z; st.u[7] = b.w;
    } else if constexpr (kType == kF16) {
        const uint4 h = *reinterpret_cast<const uint4*>(wrow + 2LL * (32 * blk + 8 * g));
        st.u[0] = h.x; st.u[1] = h.y; st.u[2] = h.z; st.u[3] = h.w;
    } else {
        // One 12-byte load per lane: lanes that take qs[0..7] read bytes 0..11
        // of the block (the scale, then their 8 bytes at 2..9); the others
        // read the 12 bytes ending with their 8 (at 4..11 of the load) and
        // take the scale from their row's first lane (stream_mfma).  Blocks
        // start at even byte offsets: the loads are 2-byte aligned.
        constexpr int kBlock = kType == kQ8_0 ? 34 : 18;
        const int h = kType == kQ8_0 ? g : (g & 1);  // which 8 bytes of qs
        const unsigned char* p = wrow + static_cast<long long>(kBlock) * blk + (h ? 8 * h - 2 : 0);
        // p is only 2-byte aligned: copy the bytes (the compiler, told the
        // true alignment, still emits one dwordx3 load, since gfx950 runs
        // global memory in unaligned-access mode).
        unsigned q[3];
        __builtin_memcpy(q, p, 12);
        st.u[0] = q[0];
        st.u[1] = q[1];
        st.u[2] = q[2];
    }
#pragma unroll
    for (int ti = 0; ti < kNT; ++ti) {
        st.xa[ti] = *reinterpret_cast<const float4*>(xr[ti] + 32 * blk);
        st.xb[ti] = *reinterpret_cast<const float4*>(xr[ti] + 32 * blk + 4);
    }
}

// The block's products: each weight the reference's dequantised value (F16
// converted, Q8_0 q * d, Q4_0 (q - 8) * d), 8 MFMA steps per token tile.
template <int kType, int kNT>
__device__ __forceinline__ void stream_mfma(const StreamStage<kType, kNT>& st, int g, floatx4 (&acc)[kNT])
{
    float w[8];
    if constexpr (kType == kF32) {
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = __builtin_bit_cast(float, st.u[i]);
    } else if constexpr (kType == kF16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[2 * i] = half_to_float(st.u[i] & 0xFFFFu);
            w[2 * i + 1] = half_to_float(st.u[i] >> 16);
        }
    } else {
        // the scale from lane c (g = 0, which loaded the block's first bytes);
        // this lane's 8 bytes at bytes 2..9 of its load (h = 0) or 4..11
        const int h = kType == kQ8_0 ? g : (g & 1);
        const float d = half_to_float(__shfl(st.u[0], threadIdx.x & 15) & 0xFFFFu);
        const unsigned q[2] = {h ? st.u[1] : (st.u[0] >> 16) | (st.u[1] << 16),
                               h ? st.u[2] : (st.u[1] >> 16) | (st.u[2] << 16)};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const unsigned byte = (q[i >> 2] >> (8 * (i & 3))) & 0xFFu;
            if constexpr (kType == kQ8_0)
                w[i] = static_cast<float>(static_cast<signed char>(byte)) * d;
            else
                w[i] = static_cast<float>(static_cast<int>((byte >> ((g >> 1) * 4)) & 0xFu) - 8) * d;
        }
    }
#pragma unroll
    for (int ti = 0; ti < kNT; ++ti) {
        acc[ti] = mfma16(st.xa[ti].x, w[0], acc[ti]);
        acc[ti] = mfma16(st.xa[ti].y, w[1], acc[ti]);
        acc[ti] = mfma16(st.xa[ti].z, w[2], acc[ti]);
        acc[ti] = mfma16(st.xa[ti].w, w[3], acc[ti]);
        acc[ti] = mfma16(st.xb[ti].x, w[4], acc[ti]);
        acc[ti] = mfma16(st.xb[ti].y, w[5], acc[ti]);
        acc[ti] = mfma16(st.xb[ti].z, w[6], acc[ti]);
        acc[ti] = mfma16(st.xb[ti].w, w[7], acc[ti]);
    }
}

template <int kType, int kNT>
__global__ __launch_bounds__(kStreamWaves * 64) void stream_product_kernel(const StreamParams p)
{
    // blocks whose loads a wave has issued: 4 for one token tile, 2 for more,
    // whose larger stages (and 704-workgroup gate | up grid) gain less from
    // depth than they lose in occupancy (32-token Q4_0 prompts 2.53 ms
    // against 2.66 with 4, 2.72 with 3)
    constexpr int kDepth = kNT == 1 ? 4 : 2;
    __shared__ float s_red[kStreamWaves][kNT][4][64];
    // the wave index as a scalar, so that the block loop's branches are uniform
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int c = lane & 15, g = lane >> 4;
    const int row = blockIdx.x * 16 + c;
    // this lane's weight row (the last one for rows past the end) and its segment
    int seg = 0, r = min(row, p.total_rows - 1);
    while (seg + 1 < p.n_seg && r >= p.seg[seg].rows) r -= p.seg[seg++].rows;
    const unsigned char* const wrow = p.seg[seg].w + static_cast<long long>(r) * p.row_bytes;
    const int t0 = blockIdx.y * 16 * kNT;
    const int xoff = kType == kQ4_0 ? (g >> 1) * 16 + (g & 1) * 8 : 8 * g;
    const float* xr[kNT];
#pragma unroll
    for (int ti = 0; ti < kNT; ++ti)
        xr[ti] = p.x + static_cast<long long>(min(t0 + 16 * ti + c, p.n - 1)) * p.x_stride + xoff;
    floatx4 acc[kNT];
#pragma unroll
    for (int ti = 0; ti < kNT; ++ti) acc[ti] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    // blocks wave + kStreamWaves i for i < nb, the loads of the next kDepth - 1
    // in flight while one is multiplied (the weights come from HBM, one round
    // trip per block otherwise); loads past the wave's last block re-read its
    // first one, or the row's last block for a wave with none (never used)
    const int n_blk = p.cols >> 5;
    const int nb = wave < n_blk ? (n_blk - wave + kStreamWaves - 1) / kStreamWaves : 0;
    const auto block_of = [&](int i) { return min(wave + kStreamWaves * (i < nb ? i : 0), n_blk - 1); };
    StreamStage<kType, kNT> st[kDepth];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
        stream_load(st[d], wrow, xr, block_of(d), g);
        __builtin_amdgcn_sched_barrier(0);  // the stages' loads in issue order
    }
    for (int i0 = 0; i0 < nb; i0 += kDepth) {
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
            const int i = i0 + d;
            if (i < nb) stream_mfma(st[d], g, acc);
            __builtin_amdgcn_sched_barrier(0);
            stream_load(st[d], wrow, xr, block_of(i + kDepth), g);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int ti = 0; ti < kNT; ++ti)
#pragma unroll
        for (int v = 0; v < 4; ++v) s_red[wave][ti][v][lane] = acc[ti][v];
    __syncthreads();
    // thread (wave, lane) writes token 4 g + wave of every tile for row c
    if (row >= p.total_rows) return;
    float* const out = p.seg[seg].out + r;
    const long long stride = p.seg[seg].out_stride;
#pragma unroll
    for (int ti = 0; ti < kNT; ++ti) {
        const int t = t0 + 16 * ti + 4 * g + wave;
        if (t >= p.n) continue;
        float sum = s_red[0][ti][wave][lane];
#pragma unroll
        for (int w2 = 1; w2 < kStreamWaves; ++w2) sum += s_red[w2][ti][wave][lane];
        float* const o = out + static_cast<long long>(t) * stride;
        *o = p.add ? *o + sum : sum;
    }
}

template <int kType>
hipError_t launch_stream_typed(const StreamParams& p, hipStream_t s)
{
    const int nt = (p.n + 15) / 16;
    const dim3 grid(static_cast<unsigned>((p.total_rows + 15) / 16),
                    static_cast<unsigned>((nt + p.tiles - 1) / p.tiles));
    const dim3 block(kStreamWaves * 64);
    switch (p.tiles) {
    case 1: hipLaunchKernelGGL((stream_product_kernel<kType, 1>), grid, block, 0, s, p); break;
    case 2: hipLaunchKernelGGL((stream_product_kernel<kType, 2>), grid, block, 0, s, p); break;
    case 3: hipLaunchKernelGGL((stream_product_kernel<kType, 3>), grid, block, 0, s, p); break;
    default: hipLaunchKernelGGL((stream_product_kernel<kType, 4>), grid, block, 0, s, p); break;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t load_batch_code()
{
    hipFuncAttributes a;
    return hipFuncGetAttributes(&a, reinterpret_cast<const void*>(&swiglu_rows_kernel));
}

bool stream_supported(int type) { return type == kF32 || type == kF16 || type == kQ8_0 || type == kQ4_0; }

hipError_t launch_stream_product(int type, const StreamParams& p, hipStream_t s)
{
    if (!stream_supported(type) || p.tiles < 1 || p.tiles > kStreamMaxTiles || p.n < 1 || p.total_rows < 1 || p.cols < 32 || p.cols % 32 != 0 ||
        p.n_seg < 1 || p.n_seg > kGemvMaxSeg || p.x_stride % 4 != 0 ||
        reinterpret_cast<uintptr_t>(p.x) % 16 != 0 || p.row_bytes != weight_row_bytes(type, p.cols))
        return hipErrorInvalidValue;
    int rows = 0;
    for (int i = 0; i < p.n_seg; ++i) {
        const uintptr_t align = type == kF32 || type == kF16 ? 16 : 2;
        if (p.seg[i].rows < 1 || reinterpret_cast<uintptr_t>(p.seg[i].w) % align != 0) return hipErrorInvalidValue;
        rows += p.seg[i].rows;
    }
    if (rows != p.total_rows) return hipErrorInvalidValue;
    switch (type) {
    case kF32: return launch_stream_typed<kF32>(p, s);
    case kF16: return launch_stream_typed<kF16>(p, s);
    case kQ8_0: return launch_stream_typed<kQ8_0>(p, s);
    default: return launch_stream_typed<kQ4_0>(p, s);
    }
}

hipError_t launch_rmsnorm_rows(float* out, const float* x, const float* w, int n_rows, int size, float eps,
                               hipStream_t s)
{
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(n_rows), dim3(kThreads), 0, s, out, x, w, size, eps);
    return hipGetLastError();
}

hipError_t launch_reduce_rmsnorm_rows(float* x, const float* part, int k_splits, float* out, const float* w,
                                      int n_tok, int size, float eps, hipStream_t s)
{
    const auto a16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
    if (n_tok < 1 || size < 4 || size % 4 != 0 || k_splits < 1 || !a16(x) || !a16(part) || !a16(out))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(reduce_rmsnorm_rows_kernel, dim3(n_tok), dim3(kThreads), 0, s, x, part, k_splits,
                       static_cast<long long>(n_tok) * size, out, w, size, eps);
    return hipGetLastError();
}

hipError_t launch_swiglu_rows(float* h, int n_rows, int n_ff, hipStream_t s)
{
    hipLaunchKernelGGL(swiglu_rows_kernel, dim3((n_ff + kThreads - 1) / kThreads, n_rows), dim3(kThreads), 0,
                       s, h, n_ff);
    return hipGetLastError();
}

}  // namespace tla
