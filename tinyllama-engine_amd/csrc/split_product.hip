// split_product_kernel: the projections of a prompt of many tokens
// (tla_matmul_batch, tla_prefill_forward) as bf16 matrix-core products that
// keep fp32 accuracy: the batched form of the matmuls forward() makes per
// token (src/forward.cpp:180-228, matmul() src/ops.cpp:959-983; weight
// blocks src/gguf.h:56-135).
//
//   out[t][row] (+)= sum_k W[row][k] x[t][k]
//
// Exact splitting.  Every fp32 x is the sum of three bf16 numbers, x = x0 +
// x1 + x2 (x0 = x rounded to bf16, x1 = the remainder rounded, x2 the exact
// rest: 8 + 8 + 8 significant bits).  A quantised weight is d * q (Q4_0,
// Q8_0) or d * (sc * q) (Q6_K) with a small integer q that bf16 holds
// exactly (Q6_K's sc * q, up to 13 bits, as two bf16 pieces); an F16 weight
// is the sum of two bf16 pieces, an F32 weight of three.  Each product of
// two pieces is exact in the fp32 accumulator of v_mfma_f32_16x16x32_bf16,
// so for a block
//   sum_k q x = sum_k q x0 + sum_k q x1 + sum_k q x2
// is an fp32 sum of exact products, and the block scale d multiplies it in
// fp32, once per 32-column block.  Products of pieces below 2^-24 of the
// full product (F16 / Q6_K: w1 x2; F32: w1 x2, w2 x1, w2 x2) are left out.
// Results are fp32 sums of the reference's products in another order: the
// reference's accuracy, not its bits.  The matrix cores' bf16 rate is 16
// times their fp32 rate, so 3-6 bf16 products per fp32 multiply-add still
// leave the product well inside it.
//
// Layout.  split_rows_kernel writes x once per product as bf16 planes in
// the order the A operand reads them: for each 32-column block kb, plane p
// and 16-token subtile s, 1 KiB whose 16-byte piece 16 g + i holds plane p
// of x[16 s + i][32 kb + 8 g .. + 7] (tokens past n are zeros).  A wave's
// operand read is then 1 KiB contiguous, from global memory into LDS and
// from LDS into registers, without bank conflicts.
//
// Tiling.  A workgroup of 4 waves owns 64 kRW weight rows x 64 tokens (4
// token subtiles); wave w owns rows 16 kRW w .. + 16 kRW - 1 for all 64
// tokens, so each x plane read from LDS feeds kRW products.  The tokens are
// the A operand and the weight rows the B operand of
// v_mfma_f32_16x16x32_bf16: lane l = 16 g + j supplies token j's and row j's
// values for columns 8 g .. 8 g + 7 of the block, and holds the sums of
// tokens 4 g .. 4 g + 3 for row j -- one block scale per lane.  The x
// blocks pass through a ring of three LDS stages (12 KiB each: three planes
// of 64 tokens), staged through registers two blocks ahead; each wave loads
// its rows' weights three blocks ahead and dequantises them in registers.
// Every output is one wave's sum in a fixed order: the same bits on every
// run and for any grid.
#include "batch.h"
#include "bf16_split.h"

namespace tla {
namespace {

constexpr int kThreads = 256;  // 4 waves
constexpr int kWaves = kThreads / 64;
constexpr int kTW = 4;         // token subtiles of 16 per workgroup
constexpr int kRing = 3;       // LDS stages, x register stages and weight register stages
constexpr int kStageBytes = 3 * kTW * 1024;
constexpr int kChunksPerWave = kStageBytes / 1024 / kWaves;  // 1 KiB copies per wave and stage
static_assert(kChunksPerWave * 1024 * kWaves == kStageBytes, "a stage is whole chunks per wave");

typedef __attribute__((address_space(3))) void* lds_ptr;
typedef __attribute__((address_space(1))) void* global_ptr;

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));  // 16 raw bytes

__device__ __forceinline__ floatx4 mfma(bf16x8 a, bf16x8 b, floatx4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float half_to_float(unsigned h)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h)));
}

// Byte offset of plane p of block kb, token subtile s, in the split x.
__device__ __forceinline__ long long plane_chunk(int kb, int p, int s, int n_sub)
{
    return (static_cast<long long>(kb * 3 + p) * n_sub + s) * 1024;
}

// One thread per (block kb, token subtile s, lane slot 16 g + i): the three
// planes of x[16 s + i][32 kb + 8 g .. + 7].
__global__ __launch_bounds__(kThreads) void split_rows_kernel(const float* __restrict__ x, long long x_stride,
                                                              int n, int n_sub, int n_blk,
                                                              unsigned char* __restrict__ xs)
{
    const long long id = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (id >= static_cast<long long>(n_blk) * n_sub * 64) return;
    const int slot = static_cast<int>(id & 63), g = slot >> 4, i = slot & 15;
    const long long rest = id >> 6;
    const int s = static_cast<int>(rest % n_sub), kb = static_cast<int>(rest / n_sub);
    const int t = 16 * s + i;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (t < n) {
        const float4* src = reinterpret_cast<const float4*>(x + t * x_stride + 32 * kb + 8 * g);
        const float4 a = src[0], b = src[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
    bf16x8 p0, p1, p2;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        __bf16 a, b, c;
        split3(v[e], a, b, c);
        p0[e] = a;
        p1[e] = b;
        p2[e] = c;
    }
    *reinterpret_cast<bf16x8*>(xs + plane_chunk(kb, 0, s, n_sub) + 16 * slot) = p0;
    *reinterpret_cast<bf16x8*>(xs + plane_chunk(kb, 1, s, n_sub) + 16 * slot) = p1;
    *reinterpret_cast<bf16x8*>(xs + plane_chunk(kb, 2, s, n_sub) + 16 * slot) = p2;
}

// One lane's raw weight bits for one row and block, as loaded (decoded only
// when the block's turn comes, so that the loads ahead stay in flight).
template <int kType>
struct WRaw;
template <>
struct WRaw<kF32> {
    uint4 a, b;  // the lane's 8 floats
};
template <>
struct WRaw<kF16> {
    uint4 h;  // the lane's 8 halves
};
template <>
struct WRaw<kQ8_0> {
    unsigned u[3];  // 12 bytes holding the lane's 8 bytes of qs (and the scale for g = 0)
};
template <>
struct WRaw<kQ4_0> {
    unsigned u[3];
};
template <>
struct WRaw<kQ6_K> {
    unsigned ql[2], qh[2];  // the lane's 8 bytes of ql and of qh
    unsigned sd;            // the lane's sub-block scale (bits 0..7) and d (bits 16..31)
};

// B pieces per format, and whether a block scale multiplies each block's sum.
template <int kType>
struct Fmt {
    static constexpr int kN = kType == kF32 ? 3 : (kType == kF16 || kType == kQ6_K) ? 2 : 1;
    static constexpr bool kScaled = kType == kQ4_0 || kType == kQ8_0 || kType == kQ6_K;
};

// Loads of block kb of one weight row (wrow) for lane group g.  kRowLoads:
// the memory instructions they are at least (separate addresses the
// compiler cannot merge), which the kernel's wait for its LDS copies counts.
template <int kType>
constexpr int kRowLoads = kType == kF32 ? 2 : kType == kQ6_K ? 4 : 1;

template <int kType>
__device__ __forceinline__ void load_w(WRaw<kType>& w, const unsigned char* wrow, int kb, int g)
{
    if constexpr (kType == kF32) {
        const uint4* q = reinterpret_cast<const uint4*>(wrow + 4LL * (32 * kb + 8 * g));
        w.a = q[0];
        w.b = q[1];
    } else if constexpr (kType == kF16) {
        w.h = *reinterpret_cast<const uint4*>(wrow + 2LL * (32 * kb + 8 * g));
    } else if constexpr (kType == kQ6_K) {
        // Q6_K super-block (ql[128] qh[64] scales[16] d; 210 bytes, 256
        // values): value r = 32 (kb % 8) + 8 g + e lies in half h = (kb % 8)
        // / 4, quarter k = kb % 4, at l = 8 g + e; its 6-bit q is a nibble of
        // ql[64 h + 32 (k % 2) + l] (low for k < 2) and bits 2k of
        // qh[32 h + l]; its scale scales[8 h + 2 k + l / 16].
        const unsigned char* sb = wrow + 210LL * (kb >> 3);
        const int h = (kb & 7) >> 2, k = kb & 3;
        __builtin_memcpy(w.ql, sb + 64 * h + 32 * (k & 1) + 8 * g, 8);
        __builtin_memcpy(w.qh, sb + 128 + 32 * h + 8 * g, 8);
        const unsigned sc = sb[192 + 8 * h + 2 * k + (g >> 1)];
        unsigned short d;
        __builtin_memcpy(&d, sb + 208, 2);
        w.sd = sc | (static_cast<unsigned>(d) << 16);
    } else {
        // One 12-byte load: lanes of g = 0 (Q4_0: g = 0 and 2) read bytes
        // 0..11 of the block (the scale, then their 8 bytes at 2..9); the
        // others read the 12 bytes ending with their 8 (at 4..11) and take
        // the scale from their row's lane of g = 0.  Blocks start at even
        // byte offsets: the copy is 2-byte aligned, and gfx950 runs global
        // memory in unaligned-access mode, so it is still one dwordx3 load.
        constexpr int kBlock = kType == kQ8_0 ? 34 : 18;
        const int h = kType == kQ8_0 ? g : (g & 1);  // which 8 bytes of qs
        const unsigned char* p = wrow + static_cast<long long>(kBlock) * kb + (h ? 8 * h - 2 : 0);
        __builtin_memcpy(w.u, p, 12);
    }
}

// The lane's B pieces (their sum: the lane's 8 weights of block kb, divided
// by the block scale where there is one) and the block scale.
template <int kType>
__device__ __forceinline__ void decode_w(const WRaw<kType>& w, int kb, int g, bf16x8 (&b)[Fmt<kType>::kN],
                                         float& d)
{
    d = 1.0f;
    if constexpr (kType == kF32) {
        const unsigned u[8] = {w.a.x, w.a.y, w.a.z, w.a.w, w.b.x, w.b.y, w.b.z, w.b.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            __bf16 p0, p1, p2;
            split3(__builtin_bit_cast(float, u[e]), p0, p1, p2);
            b[0][e] = p0;
            b[1][e] = p1;
            b[2][e] = p2;
        }
    } else if constexpr (kType == kF16) {
        const unsigned u[4] = {w.h.x, w.h.y, w.h.z, w.h.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            __bf16 p0, p1;
            split2(half_to_float((u[e >> 1] >> (16 * (e & 1))) & 0xFFFFu), p0, p1);
            b[0][e] = p0;
            b[1][e] = p1;
        }
    } else if constexpr (kType == kQ6_K) {
        const int k = kb & 3;
        const int sc = static_cast<signed char>(w.sd & 0xFFu);
        d = half_to_float(w.sd >> 16);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const unsigned lo = (w.ql[e >> 2] >> (8 * (e & 3))) & 0xFFu;
            const unsigned hi = (w.qh[e >> 2] >> (8 * (e & 3))) & 0xFFu;
            const int q = static_cast<int>(((k < 2 ? lo & 0x0Fu : lo >> 4) | (((hi >> (2 * k)) & 3u) << 4))) - 32;
            __bf16 p0, p1;
            split2(static_cast<float>(sc * q), p0, p1);
            b[0][e] = p0;
            b[1][e] = p1;
        }
    } else {
        (void)kb;
        const int h = kType == kQ8_0 ? g : (g & 1);
        d = half_to_float(__shfl(w.u[0], threadIdx.x & 15) & 0xFFFFu);
        const unsigned q[2] = {h ? w.u[1] : (w.u[0] >> 16) | (w.u[1] << 16),
                               h ? w.u[2] : (w.u[1] >> 16) | (w.u[2] << 16)};
        // Each byte u (Q4_0: the nibble masked in place; Q8_0: the byte with
        // its sign bit flipped, q + 128) becomes the float 2^23 + u by one
        // byte permute into the mantissa of 2^23 (0x4B000000), and one
        // subtraction leaves u - 8 (Q4_0) or u - 128 = q (Q8_0): two
        // operations per weight.  Small integers: the bf16 packing is exact.
        constexpr float kBase = kType == kQ8_0 ? 8388736.f : 8388616.f;  // 2^23 + 128, 2^23 + 8
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const unsigned m = kType == kQ8_0 ? q[i] ^ 0x80808080u : (q[i] >> ((g >> 1) * 4)) & 0x0F0F0F0Fu;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // bytes: [m.byte e, 0, 0, 0x4B] (selector 0x0C reads zero)
                const unsigned f = __builtin_amdgcn_perm(0x4B000000u, m, 0x070C0C00u + e);
                b[0][4 * i + e] = static_cast<__bf16>(__builtin_bit_cast(float, f) - kBase);
            }
        }
    }
}

// One block's products for one (row subtile, token subtile) tile: acc (+)=
// the products of pieces (b_i, x_p) with i + p <= 2, smallest terms first,
// scaled by the block scale where there is one.
template <int kType>
__device__ __forceinline__ void tile_products(const bf16x8 (&a)[3], const bf16x8 (&b)[Fmt<kType>::kN], float d,
                                              floatx4& acc)
{
    floatx4 t = Fmt<kType>::kScaled ? floatx4{0.f, 0.f, 0.f, 0.f} : acc;
    if constexpr (Fmt<kType>::kN >= 3) t = mfma(a[0], b[2], t);
    if constexpr (Fmt<kType>::kN >= 2) {
        t = mfma(a[1], b[1], t);
        t = mfma(a[0], b[1], t);
    }
    t = mfma(a[2], b[0], t);
    t = mfma(a[1], b[0], t);
    t = mfma(a[0], b[0], t);
    if constexpr (Fmt<kType>::kScaled) {
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] = fmaf(d, t[q], acc[q]);
    } else {
        acc = t;
    }
}

// The segment holding a row: selected field by field (an index into the
// kernel-argument array would copy it to scratch memory).
struct RowSeg {
    const unsigned char* w;
    float* out;
    long long stride;
    int row;  // within the segment
};
__device__ __forceinline__ RowSeg row_seg(const SplitParams& p, int row)
{
    RowSeg r{p.seg[0].w, p.seg[0].out, p.seg[0].out_stride, row};
    int cur = 0;  // the segment r is in so far; only its successor can take the row
#pragma unroll
    for (int i = 1; i < kGemvMaxSeg; ++i) {
        const bool next = cur == i - 1 && i < p.n_seg && r.row >= p.seg[i - 1].rows;
        cur = next ? i : cur;
        r.row = next ? r.row - p.seg[i - 1].rows : r.row;
        r.w = next ? p.seg[i].w : r.w;
        r.out = next ? p.seg[i].out : r.out;
        r.stride = next ? p.seg[i].out_stride : r.stride;
    }
    return r;
}

template <int kType, int kRW>
__global__ __launch_bounds__(kThreads) void split_product_kernel(const SplitParams p)
{
    // The ring's stages as separate arrays, so that the compiler sees that a
    // stage being read is not the one a copy in flight writes.
    __shared__ __align__(16) unsigned char s_x0[kStageBytes], s_x1[kStageBytes], s_x2[kStageBytes];
    auto stage_base = [&](int u) __attribute__((always_inline)) { return u == 0 ? s_x0 : u == 1 ? s_x1 : s_x2; };
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int j = lane & 15, g = lane >> 4;
    // Tiles by linear workgroup id L, token tile fastest (y = L mod the
    // token tiles): workgroups run on XCD L mod 8, so each XCD's workgroups
    // share a few token tiles' x planes in its L2 (at 512 tokens one XCD one
    // tile, 0.8 MB) while the weights stream through.
    const unsigned L = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    const unsigned ty = L % gridDim.y, rest = L / gridDim.y;
    const unsigned tx = rest % gridDim.x, tz = rest / gridDim.x;
    const int row0 = (tx * kWaves + wave) * 16 * kRW;
    const int s0 = ty * kTW;  // first token subtile
    // K range of this workgroup: blocks [kb_lo, kb_hi) (grid z splits K)
    const int kb_lo = tz * p.blk_per_split;
    const int kb_hi = min(kb_lo + p.blk_per_split, p.cols >> 5);

    // this lane's weight row in each row subtile (the last row for rows past
    // the end: loaded, never stored)
    const unsigned char* wrow[kRW];
#pragma unroll
    for (int r = 0; r < kRW; ++r) {
        const RowSeg rs = row_seg(p, min(row0 + 16 * r + j, p.total_rows - 1));
        wrow[r] = rs.w + static_cast<long long>(rs.row) * p.row_bytes;
    }

    // x stage of block kb: 12 chunks of 1 KiB, chunk c = plane c / 4 of
    // token subtile s0 + c % 4, copied by direct global-to-LDS loads, three
    // per wave (lane l's 16 bytes land at byte 16 l of the chunk).  Past the
    // end the last block is copied again (never read), so every iteration
    // issues the same memory operations.
    auto copy_x = [&](int kb, int stage) __attribute__((always_inline)) {
        kb = min(kb, kb_hi - 1);
#pragma unroll
        for (int i = 0; i < kChunksPerWave; ++i) {
            const int c = kChunksPerWave * wave + i;
            __builtin_amdgcn_global_load_lds(
                (global_ptr)(p.xs + plane_chunk(kb, c / kTW, s0, p.n_sub) + 1024 * (c % kTW) + 16 * lane),
                (lds_ptr)(stage_base(stage) + 1024 * c), 16, 0, 0);
        }
    };
    auto load_ws = [&](WRaw<kType> (&wr)[kRW], int kb) __attribute__((always_inline)) {
        kb = min(kb, kb_hi - 1);
#pragma unroll
        for (int r = 0; r < kRW; ++r) load_w<kType>(wr[r], wrow[r], kb, g);
    };

    floatx4 acc[kRW][kTW];
#pragma unroll
    for (int r = 0; r < kRW; ++r)
#pragma unroll
        for (int s = 0; s < kTW; ++s) acc[r][s] = floatx4{0.f, 0.f, 0.f, 0.f};

    // Block b: LDS stage b % 3 (copied two iterations before it is read),
    // weights wr<b % 3> (loaded three iterations before use).  Iteration kb:
    // wait for block kb's copy, barrier (every wave's copy has landed and
    // every wave is done with block kb - 1), copy block kb + 2 into block
    // kb - 1's stage, multiply block kb, load block kb + 3's weights.  The
    // wait counts memory operations: after block kb's copy this wave issued
    // block kb + 1's and kb + 2's weights (at least kRowLoads per row each)
    // and block kb + 1's copy (kChunksPerWave), so waiting until no more than
    // that many are outstanding means the copy has landed (they complete in
    // order; a count below the true one only waits longer).  Scheduling
    // barriers keep that order.  Separate arrays per ring
    // slot, chosen at compile time, stay in registers.
    // The prologue issues its operations in the loop's order (weights of
    // block b + 3 after the copy of block b + 2), as if iterations kb_lo - 3
    // .. kb_lo - 1 had run.
    WRaw<kType> wr0[kRW], wr1[kRW], wr2[kRW];
    load_ws(wr0, kb_lo);
    __builtin_amdgcn_sched_barrier(0);
    copy_x(kb_lo, 0);
    __builtin_amdgcn_sched_barrier(0);
    load_ws(wr1, kb_lo + 1);
    __builtin_amdgcn_sched_barrier(0);
    copy_x(kb_lo + 1, 1);
    __builtin_amdgcn_sched_barrier(0);
    load_ws(wr2, kb_lo + 2);
    __builtin_amdgcn_sched_barrier(0);

    constexpr int kAfterCopy = kChunksPerWave + 2 * kRW * kRowLoads<kType>;
    static_assert(kAfterCopy < 64, "vmcnt holds 6 bits");
    constexpr int kVmcntWait = (kAfterCopy & 15) | ((kAfterCopy >> 4) << 14) | 0xF70;  // vmcnt(kAfterCopy)
    auto iteration = [&](int kb, auto& wr_this, const int u, const int u2) __attribute__((always_inline)) {
        // A bare barrier: __syncthreads' release fence would wait for every
        // outstanding load (the copies write LDS through the vector memory
        // path), weights included.  The LDS reads of block kb - 1 were used
        // before this point, so its stage is free once every wave is here.
        __builtin_amdgcn_s_waitcnt(kVmcntWait);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        copy_x(kb + 2, u2);
        __builtin_amdgcn_sched_barrier(0);
        if (kb < kb_hi) {  // uniform
            // the row subtiles' weights first, then the token subtiles one
            // at a time (their x pieces read from LDS just before use)
            bf16x8 b[kRW][Fmt<kType>::kN];
            float d[kRW];
#pragma unroll
            for (int r = 0; r < kRW; ++r) decode_w<kType>(wr_this[r], kb, g, b[r], d[r]);
#pragma unroll
            for (int s = 0; s < kTW; ++s) {
                bf16x8 a[3];
#pragma unroll
                for (int pl = 0; pl < 3; ++pl)
                    a[pl] = *reinterpret_cast<const bf16x8*>(stage_base(u) + (pl * kTW + s) * 1024 + 16 * lane);
#pragma unroll
                for (int r = 0; r < kRW; ++r) tile_products<kType>(a, b[r], d[r], acc[r][s]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        load_ws(wr_this, kb + 3);
        __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll 1
    for (int kb0 = kb_lo; kb0 < kb_hi; kb0 += kRing) {
        iteration(kb0, wr0, 0, 2);
        iteration(kb0 + 1, wr1, 1, 0);
        iteration(kb0 + 2, wr2, 2, 1);
    }
    // the copies past the end land before the workgroup's LDS is released
    __builtin_amdgcn_s_waitcnt(0);

    // lane (g, j) holds tokens 16 (s0 + s) + 4 g + q of row row0 + 16 r + j;
    // with K split, the sums go to part[z][t][row] for split_reduce_kernel
#pragma unroll
    for (int r = 0; r < kRW; ++r) {
        const int row = row0 + 16 * r + j;
        if (row >= p.total_rows) continue;
        if (p.part) {
            float* const o = p.part + static_cast<long long>(tz) * p.n * p.total_rows + row;
#pragma unroll
            for (int s = 0; s < kTW; ++s)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int t = 16 * (s0 + s) + 4 * g + q;
                    if (t < p.n) o[static_cast<long long>(t) * p.total_rows] = acc[r][s][q];
                }
            continue;
        }
        const RowSeg rs = row_seg(p, row);
        float* const out = rs.out + rs.row;
        const long long stride = rs.stride;
#pragma unroll
        for (int s = 0; s < kTW; ++s)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int t = 16 * (s0 + s) + 4 * g + q;
                if (t >= p.n) continue;
                float* const o = out + static_cast<long long>(t) * stride;
                *o = p.add ? *o + acc[r][s][q] : acc[r][s][q];
            }
    }
}

// out[t][row] (+)= sum over the K splits z, in order, of part[z][t][row]:
// one thread per (t, row).
__global__ __launch_bounds__(kThreads) void split_reduce_kernel(const SplitParams p)
{
    const long long id = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (id >= static_cast<long long>(p.n) * p.total_rows) return;
    const int t = static_cast<int>(id / p.total_rows), row = static_cast<int>(id % p.total_rows);
    const long long plane = static_cast<long long>(p.n) * p.total_rows;
    float sum = p.part[id];
    for (int z = 1; z < p.k_splits; ++z) sum += p.part[z * plane + id];
    const RowSeg rs = row_seg(p, row);
    float* const o = rs.out + rs.row + static_cast<long long>(t) * rs.stride;
    *o = p.add ? *o + sum : sum;
}

template <int kType, int kRW>
hipError_t launch_product(const SplitParams& p, hipStream_t s)
{
    const dim3 grid(static_cast<unsigned>((p.total_rows + 64 * kRW - 1) / (64 * kRW)),
                    static_cast<unsigned>(p.n_sub / kTW), static_cast<unsigned>(p.k_splits));
    hipLaunchKernelGGL((split_product_kernel<kType, kRW>), grid, dim3(kThreads), 0, s, p);
    return hipGetLastError();
}

template <int kType>
hipError_t launch_typed(const SplitParams& p, hipStream_t s)
{
    hipError_t err;
    switch (p.rows_per_wave) {
    case 1: err = launch_product<kType, 1>(p, s); break;
    case 2: err = launch_product<kType, 2>(p, s); break;
    default: err = launch_product<kType, 4>(p, s); break;
    }
    if (err != hipSuccess || !p.part || p.defer_reduce) return err;
    const long long n = static_cast<long long>(p.n) * p.total_rows;
    hipLaunchKernelGGL(split_reduce_kernel, dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, s, p);
    return hipGetLastError();
}

}  // namespace

size_t split_x_bytes(int n, int cols)
{
    return static_cast<size_t>(split_tokens(n)) * static_cast<size_t>(cols) * 6;
}

size_t split_part_bytes(int n, int total_rows, int k_splits)
{
    return static_cast<size_t>(n) * static_cast<size_t>(total_rows) * static_cast<size_t>(k_splits) * sizeof(float);
}

int split_tokens(int n)
{
    return (n + 16 * kTW - 1) / (16 * kTW) * (16 * kTW);
}

hipError_t launch_split_rows(const float* x, long long x_stride, int n, int cols, unsigned char* xs, hipStream_t s)
{
    if (n < 1 || cols < 32 || cols % 32 != 0 || x_stride % 4 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0)
        return hipErrorInvalidValue;
    const int n_sub = split_tokens(n) / 16, n_blk = cols / 32;
    const long long threads = static_cast<long long>(n_blk) * n_sub * 64;
    hipLaunchKernelGGL(split_rows_kernel, dim3(static_cast<unsigned>((threads + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, s, x, x_stride, n, n_sub, n_blk, xs);
    return hipGetLastError();
}

hipError_t launch_split_product(int type, const SplitParams& p, hipStream_t s)
{
    if (p.n < 1 || p.total_rows < 1 || p.cols < 32 || p.cols % 32 != 0 || (type == kQ6_K && p.cols % 256 != 0) ||
        p.n_sub != split_tokens(p.n) / 16 || p.n_seg < 1 || p.n_seg > kGemvMaxSeg ||
        p.row_bytes != static_cast<long long>(weight_row_bytes(type, p.cols)) ||
        (p.rows_per_wave != 1 && p.rows_per_wave != 2 && p.rows_per_wave != 4) || p.k_splits < 1 ||
        p.blk_per_split < 1 || static_cast<long long>(p.k_splits - 1) * p.blk_per_split >= p.cols / 32 ||
        static_cast<long long>(p.k_splits) * p.blk_per_split < p.cols / 32 || (p.k_splits > 1) != (p.part != nullptr))
        return hipErrorInvalidValue;
    int rows = 0;
    for (int i = 0; i < p.n_seg; ++i) {
        const uintptr_t align = type == kF32 || type == kF16 ? 16 : 2;
        if (p.seg[i].rows < 1 || reinterpret_cast<uintptr_t>(p.seg[i].w) % align != 0) return hipErrorInvalidValue;
        rows += p.seg[i].rows;
    }
    if (rows != p.total_rows) return hipErrorInvalidValue;
    switch (type) {
    case kF32: return launch_typed<kF32>(p, s);
    case kF16: return launch_typed<kF16>(p, s);
    case kQ8_0: return launch_typed<kQ8_0>(p, s);
    case kQ4_0: return launch_typed<kQ4_0>(p, s);
    case kQ6_K: return launch_typed<kQ6_K>(p, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace tla
