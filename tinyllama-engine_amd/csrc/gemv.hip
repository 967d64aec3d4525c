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
//     src/forward.cpp:210-213);
//   - SwiGLU, either in the x staging of the down projection (silu(x) * x2)
//     or, for one vector of a block format, in the epilogue of the gate/up
//     launch, whose lane groups hold gate row r and up row r together
//     (src/forward.cpp:215-228);
//   - RoPE epilogue for the q and k rows (row pairs 2i, 2i+1 of a head are
//     one wave's two lane groups), whose k and v outputs can be the cache
//     row itself: RoPE + append (src/forward.cpp:192-196).
//
// Work decomposition: the weights of a row are cut into units of 64 (two
// Q8_0/Q4_0 blocks, 128 B of F16, 256 B of F32, a quarter of a Q6_K
// super-block).  With cols a multiple of 64 every Q8_0/Q4_0 unit starts on a
// 4-byte boundary, so it is read with aligned dword loads; Q6_K super-blocks
// (210 B) are 2-byte aligned and read with 16-bit loads.  32 lanes serve a
// row when it has at most 32 units (cols <= 2048), else 64; the lanes' dot
// products meet in a DPP reduction.  x sits in LDS (padded against bank
// conflicts), read as float4.
//
// Products and sums are fp32 but grouped differently from the reference's
// sequential loops, so results match it to fp32 rounding, not bit for bit.
#include <algorithm>

#include "rope_math.h"
#include "row_math.h"
#include "tla_internal.h"

namespace tla {
namespace {

constexpr int kThreads = 256;
constexpr int kUnit = 64;  // weights per lane step

// x sits in LDS with 4 floats of padding after every 64: the lanes of a row
// read 64-float spans 256 B apart, which without padding all start in the
// same bank; with it, lane i starts 4i banks further.
__device__ __forceinline__ int xpad(int c) { return c + 4 * (c >> 6); }
__host__ __device__ constexpr int xs_floats(int cols) { return cols + cols / 16; }

__device__ __forceinline__ float half_bits_to_float(unsigned h)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h)));
}

// silu(v) = v * (1 / (1 + exp(-v))), with the reference's operation order
// (src/ops.cpp:1107-1115); expf is the device library's.
__device__ __forceinline__ float silu(float v)
{
    const float sigmoid = 1.0f / (1.0f + expf(-v));
    return v * sigmoid;
}

// kW floats of x (kW = 4, 8 or 16) from LDS starting at column c0, a multiple
// of kW, so the span does not cross a padding gap.
template <int kW>
__device__ __forceinline__ void lds_x(const float* xs, int c0, float* o)
{
    const float* base = xs + xpad(c0);
#pragma unroll
    for (int i = 0; i < kW / 4; ++i) {
        const float4 t = *reinterpret_cast<const float4*>(base + 4 * i);
        o[4 * i + 0] = t.x;
        o[4 * i + 1] = t.y;
        o[4 * i + 2] = t.z;
        o[4 * i + 3] = t.w;
    }
}

// Sum of the fused attention + W_o launch's partials at index i: the n
// (<= kAttnOutMaxParts) loads issued together (an index past n reloads
// partial 0), then added in order ((p0 + p1) + p2) + p3.
__device__ __forceinline__ float part_sum(const float* parts, int n, long long stride, long long i)
{
    float v[kAttnOutMaxParts];
#pragma unroll
    for (int g = 0; g < kAttnOutMaxParts; ++g) v[g] = parts[(g < n ? g : 0) * stride + i];
    float s = v[0];
#pragma unroll
    for (int g = 1; g < kAttnOutMaxParts; ++g)
        if (g < n) s += v[g];
    return s;
}

// F32 and F16 weights are read once per launch, each load instruction of a
// row's lanes one contiguous stretch, so those loads are non-temporal (nt
// bit): 32000 x 2048 F16 20.9 against 22.8 us, as a streaming read runs ~10 %
// faster with it.  The block formats' lanes read 16-byte pieces of 34-, 18-
// or 210-byte blocks, so consecutive load instructions share cache lines:
// with nt they ran about twice as long (Q8_0 29 against 16 us), so they keep
// the default, as x does.
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ldw_f4(const float4* p)
{
    const f32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p));
    return make_float4(t.x, t.y, t.z, t.w);
}

__device__ __forceinline__ uint4 ldw_u4(const uint4* p)
{
    const u32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}

// 16 bytes from a 4-byte aligned address: one global_load_dwordx4 (the
// hardware takes dword alignment for multi-dword loads).
typedef unsigned u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ void load16_a4(const unsigned char* p, unsigned* o)
{
    const u32x4_a4 t = *reinterpret_cast<const u32x4_a4*>(p);
    o[0] = t.x;
    o[1] = t.y;
    o[2] = t.z;
    o[3] = t.w;
}

// ---- one 64-weight unit of a row -------------------------------------------
//
// The lanes serving a row step through its units together: in a step, lanes
// l < n hold units u0 + l (n = the step's active lanes).  Each format loads
// a unit's raw bytes (load), gives the dot product of its q-th group of 16
// weights with 16 x values before any scale (part), and combines the four
// parts with the unit's scales (finish).  The x values of group q sit in
// 16 / kW runs of kW columns; run j starts at xcol(u0, n, l, q, j).  x is
// read once per group and used for every row a lane holds.  s16[g] is the
// sum of x over columns 16g .. 16g+15, for the block formats' zero offsets:
// sum (q - z) x = sum q x - z sum x.
//
// F32 and F16 spread a unit over the step's span so that each load
// instruction of the n lanes reads one contiguous stretch of HBM; the block
// formats keep a unit's bytes contiguous (a unit is whole blocks).

__device__ __forceinline__ float ub(unsigned w, int k)  // byte k as float (v_cvt_f32_ubyte*)
{
    return static_cast<float>((w >> (8 * k)) & 0xFFu);
}

template <int kType>
struct Unit;

// 16 float4 pieces; piece i at column 64 u0 + 4 (l + n i).
template <>
struct Unit<kF32> {
    static constexpr int kRows = 1, kW = 4;
    float w[64];
    __device__ static int xcol(int u0, int n, int l, int q, int j) { return 64 * u0 + 4 * (l + n * (4 * q + j)); }
    __device__ void load(const unsigned char* row, int u0, int n, int l)
    {
        const float4* p = reinterpret_cast<const float4*>(row) + 16 * u0 + l;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float4 t = ldw_f4(p + n * i);
            w[4 * i] = t.x;
            w[4 * i + 1] = t.y;
            w[4 * i + 2] = t.z;
            w[4 * i + 3] = t.w;
        }
    }
    __device__ float part(int q, const float (&x)[16]) const
    {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) s += w[16 * q + i] * x[i];
        return s;
    }
    __device__ float finish(const float (&pt)[4], const float*) const
    {
        return (pt[0] + pt[1]) + (pt[2] + pt[3]);
    }
};

// 8 pieces of 8 halves (16 B); piece i at column 64 u0 + 8 (l + n i).
template <>
struct Unit<kF16> {
    static constexpr int kRows = 1, kW = 8;
    uint4 raw[8];
    __device__ static int xcol(int u0, int n, int l, int q, int j) { return 64 * u0 + 8 * (l + n * (2 * q + j)); }
    __device__ void load(const unsigned char* row, int u0, int n, int l)
    {
        const uint4* p = reinterpret_cast<const uint4*>(row) + 8 * u0 + l;
#pragma unroll
        for (int i = 0; i < 8; ++i) raw[i] = ldw_u4(p + n * i);
    }
    __device__ float part(int q, const float (&x)[16]) const
    {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint4 r = raw[2 * q + i];
            const unsigned wd[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                s += half_bits_to_float(wd[j] & 0xFFFFu) * x[8 * i + 2 * j];
                s += half_bits_to_float(wd[j] >> 16) * x[8 * i + 2 * j + 1];
            }
        }
        return s;
    }
    __device__ float finish(const float (&pt)[4], const float*) const
    {
        return (pt[0] + pt[1]) + (pt[2] + pt[3]);
    }
};

// Two Q8_0 blocks (68 bytes, 17 dwords): d0 | qs0[32] | d1 | qs1[32].  The
// int8 weights are read as bytes with the sign bit flipped, q + 128 in
// 0..255, converted by the byte-to-float instructions; the 128 comes back
// out through the block's x sum.
template <>
struct Unit<kQ8_0> {
    static constexpr int kRows = 2, kW = 16;
    unsigned dw[17];
    int u;
    __device__ static int xcol(int u0, int, int l, int q, int) { return 64 * (u0 + l) + 16 * q; }
    __device__ void load(const unsigned char* row, int u0, int, int l)
    {
        u = u0 + l;
        const unsigned char* p = row + u * 68;
#pragma unroll
        for (int i = 0; i < 4; ++i) load16_a4(p + 16 * i, dw + 4 * i);
        dw[16] = *reinterpret_cast<const unsigned*>(p + 64);
    }
    // four bytes starting at byte b (b even), as a dword
    __device__ unsigned bytes4(int b) const
    {
        return (b & 3) == 0 ? dw[b >> 2] : __builtin_amdgcn_alignbyte(dw[(b >> 2) + 1], dw[b >> 2], 2);
    }
    __device__ float part(int q, const float (&x)[16]) const
    {
        const int base = (q < 2 ? 2 : 36) + 16 * (q & 1);  // first qs byte of the group
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const unsigned w = bytes4(base + 4 * i) ^ 0x80808080u;
#pragma unroll
            for (int k = 0; k < 4; ++k) s += ub(w, k) * x[4 * i + k];
        }
        return s;
    }
    __device__ float finish(const float (&pt)[4], const float* s16) const
    {
        const float d0 = half_bits_to_float(dw[0] & 0xFFFFu), d1 = half_bits_to_float(dw[8] >> 16);
        const float* z = s16 + 4 * u;
        return d0 * ((pt[0] - 128.f * z[0]) + (pt[1] - 128.f * z[1])) +
               d1 * ((pt[2] - 128.f * z[2]) + (pt[3] - 128.f * z[3]));
    }
};

// Two Q4_0 blocks (36 bytes, 9 dwords): d0 | qs0[16] | d1 | qs1[16]; byte j
// of qs holds element j (low nibble) and j + 16 (high nibble), value - 8.
template <>
struct Unit<kQ4_0> {
    static constexpr int kRows = 2, kW = 16;
    unsigned dw[9];
    int u;
    __device__ static int xcol(int u0, int, int l, int q, int) { return 64 * (u0 + l) + 16 * q; }
    __device__ void load(const unsigned char* row, int u0, int, int l)
    {
        u = u0 + l;
        const unsigned char* p = row + u * 36;
        load16_a4(p, dw);
        load16_a4(p + 16, dw + 4);
        dw[8] = *reinterpret_cast<const unsigned*>(p + 32);
    }
    __device__ unsigned bytes4(int b) const
    {
        return (b & 3) == 0 ? dw[b >> 2] : __builtin_amdgcn_alignbyte(dw[(b >> 2) + 1], dw[b >> 2], 2);
    }
    __device__ float part(int q, const float (&x)[16]) const
    {
        const int base = q < 2 ? 2 : 20;  // qs of block q / 2
        const int shift = 4 * (q & 1);    // low nibbles, then high
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            unsigned w = (bytes4(base + 4 * i) >> shift) & 0x0F0F0F0Fu;
            // keep the four nibbles as one masked word: left visible, the
            // compiler folds the mask into a bit-field extract per weight
            asm volatile("" : "+v"(w));
#pragma unroll
            for (int k = 0; k < 4; ++k) s += ub(w, k) * x[4 * i + k];
        }
        return s;
    }
    __device__ float finish(const float (&pt)[4], const float* s16) const
    {
        const float d0 = half_bits_to_float(dw[0] & 0xFFFFu), d1 = half_bits_to_float(dw[4] >> 16);
        const float* z = s16 + 4 * u;
        return d0 * ((pt[0] - 8.f * z[0]) + (pt[1] - 8.f * z[1])) +
               d1 * ((pt[2] - 8.f * z[2]) + (pt[3] - 8.f * z[3]));
    }
};

// A quarter of a Q6_K super-block (ql[128] qh[64] scales[16] d; 210 bytes):
// half h, l = 16m .. 16m+15 of that half, i.e. elements 128h + l + 32k for
// k = 0..3, the grouping of the reference's loops; group k has one scale.
// Super-blocks start on 2-byte boundaries: each 16-byte run is read as five
// dwords from the dword boundary below it and shifted into place.
template <>
struct Unit<kQ6_K> {
    static constexpr int kRows = 2, kW = 16;
    unsigned qla[4], qlb[4], qh[4];  // ql[64h+16m ..], ql[64h+32+16m ..], qh[32h+16m ..]
    int sc[4];
    float d;
    int u;
    __device__ static int col(int u, int q)
    {
        return 256 * (u >> 2) + 128 * ((u & 3) >> 1) + 16 * (u & 1) + 32 * q;
    }
    __device__ static int xcol(int u0, int, int l, int q, int) { return col(u0 + l, q); }
    // 16 bytes at p (2-byte aligned); reads stay inside [p - 2, p + 18)
    __device__ static void load16_a2(const unsigned char* p, unsigned* o)
    {
        const unsigned sh = static_cast<unsigned>(reinterpret_cast<uintptr_t>(p)) & 3u;
        const unsigned char* p4 = p - sh;
        unsigned t[5];
        load16_a4(p4, t);
        t[4] = *reinterpret_cast<const unsigned*>(p4 + 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = __builtin_amdgcn_alignbyte(t[i + 1], t[i], sh);
    }
    __device__ void load(const unsigned char* row, int u0, int, int l)
    {
        u = u0 + l;
        const int b = u >> 2, q = u & 3, h = q >> 1, m = q & 1;
        const unsigned char* sb = row + 210 * b;
        load16_a2(sb + 64 * h + 16 * m, qla);
        load16_a2(sb + 64 * h + 32 + 16 * m, qlb);
        load16_a2(sb + 128 + 32 * h + 16 * m, qh);
        // scales 8h .. 8h+7 (bytes 192+8h ..), then d at 208, as 16-bit loads
        // (the super-block may end at the end of the buffer, so no dword may
        // reach past byte 209)
        const unsigned short* s16 = reinterpret_cast<const unsigned short*>(sb + 192 + 8 * h);
        unsigned short sw[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) sw[k] = s16[k];
#pragma unroll
        for (int k = 0; k < 4; ++k) sc[k] = static_cast<signed char>(sw[k] >> (8 * m));
        d = half_bits_to_float(*reinterpret_cast<const unsigned short*>(sb + 208));
    }
    __device__ float part(int k, const float (&x)[16]) const
    {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const unsigned la = qla[i], lb = qlb[i], hb = qh[i];
            // 4 low bits of the four weights of dword i, then their 2 high bits
            const unsigned lo = (k == 0) ? (la & 0x0F0F0F0Fu) : (k == 1) ? (lb & 0x0F0F0F0Fu)
                              : (k == 2) ? ((la >> 4) & 0x0F0F0F0Fu) : ((lb >> 4) & 0x0F0F0F0Fu);
            const unsigned q6 = lo | (((hb >> (2 * k)) & 0x03030303u) << 4);  // 0..63 per byte
#pragma unroll
            for (int j = 0; j < 4; ++j) s += ub(q6, j) * x[4 * i + j];
        }
        return s;
    }
    __device__ float finish(const float (&pt)[4], const float* s16) const
    {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k)
            s += static_cast<float>(sc[k]) * (pt[k] - 32.f * s16[col(u, k) >> 4]);
        return d * s;
    }
};

// ---- cross-lane sums with DPP (no LDS round trips) -----------------------------

template <int kCtrl, int kRowMask>
__device__ __forceinline__ float dpp_add(float v)
{
    // the moved value, or 0 where the source lane is outside the row or the
    // row is masked off
    const int moved = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, kRowMask,
                                                  0xF, true);
    return v + __builtin_bit_cast(float, moved);
}

// Sum over each group of kLanesPerRow (32 or 64) lanes; the total lands in the
// group's last lane.  Inclusive scans inside 16-lane rows (row_shr 1, 2, 4,
// 8), then row_bcast15 into rows 1 and 3, and for 64 lanes row_bcast31 into
// rows 2 and 3.
template <int kLanesPerRow>
__device__ __forceinline__ float row_sum(float v)
{
    v = dpp_add<0x111, 0xF>(v);  // row_shr:1
    v = dpp_add<0x112, 0xF>(v);  // row_shr:2
    v = dpp_add<0x114, 0xF>(v);  // row_shr:4
    v = dpp_add<0x118, 0xF>(v);  // row_shr:8
    v = dpp_add<0x142, 0xA>(v);  // row_bcast15 -> rows 1, 3
    if constexpr (kLanesPerRow == 64) v = dpp_add<0x143, 0xC>(v);  // row_bcast31 -> rows 2, 3
    return v;
}

// ---- kernel ------------------------------------------------------------------

// The rows one lane group holds in a pass: kRows rows kRowsPerWave apart,
// located in their segments, with the unit step u0 loaded.  Every lane
// loads: rows past the end read row 0 of the first segment and lanes without
// a unit in the step read lane 0's, addresses the wave reads anyway or that
// sit in cache, so the loads need no branch (a branch around a load makes
// the compiler wait for every load in flight where the paths join).
// The segment table in scalar registers (readfirstlane pins each field
// there).  Segments 1 and 2 are kept as byte offsets from segment 0's
// pointers, so every address a lane forms derives from a kernel-argument
// pointer and stays a global-memory access.
__device__ __forceinline__ int sreg(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ long long sreg(long long v)
{
    const unsigned long long u = static_cast<unsigned long long>(v);
    const unsigned lo = static_cast<unsigned>(sreg(static_cast<int>(static_cast<unsigned>(u))));
    const unsigned hi = static_cast<unsigned>(sreg(static_cast<int>(static_cast<unsigned>(u >> 32))));
    return static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo);
}
__device__ __forceinline__ long long byte_gap(const void* a, const void* b)
{
    return sreg(static_cast<long long>(reinterpret_cast<uintptr_t>(a)) -
                static_cast<long long>(reinterpret_cast<uintptr_t>(b)));
}

struct SegRegs {
    // Each field of segments 1 and 2 is kept as a difference from the
    // previous segment's, so that locating a row adds terms selected against
    // zero: a select between fields of one struct can compile to an indexed
    // load from a private copy of the struct (scratch memory).
    long long w_d1, w_d2, out_d1, out_d2;  // byte offsets: segment 1 - 0, 2 - 1
    long long stride0, stride_d1, stride_d2;
    int rows0, rows1;
    int n_seg;
    long long row_bytes;

    __device__ explicit SegRegs(const GemvParams& p)
    {
        static_assert(kGemvMaxSeg == 3, "three segments at most");
        w_d1 = byte_gap(p.seg[1].w, p.seg[0].w);
        w_d2 = byte_gap(p.seg[2].w, p.seg[1].w);
        out_d1 = byte_gap(p.seg[1].out, p.seg[0].out);
        out_d2 = byte_gap(p.seg[2].out, p.seg[1].out);
        stride0 = sreg(p.seg[0].out_stride);
        stride_d1 = sreg(p.seg[1].out_stride - p.seg[0].out_stride);
        stride_d2 = sreg(p.seg[2].out_stride - p.seg[1].out_stride);
        rows0 = sreg(p.seg[0].rows);
        rows1 = sreg(p.seg[1].rows);
        n_seg = sreg(p.n_seg);
        row_bytes = sreg(static_cast<long long>(p.row_bytes));
    }
};

// Epilogue of a one-vector launch, a template parameter so that plain
// launches carry none of the others' code: kPlain (y (+)= W.x), kPairEpi
// (gate and up rows paired, SwiGLU written), kRopeEpi (q and k row pairs
// rotated), kPartsEpi (y += W.x with the residual partials: rparts).
constexpr int kPlain = 0, kPairEpi = 1, kRopeEpi = 2, kPartsEpi = 3, kAmaxEpi = 4;

// Argmax keys: the larger key is the larger value, or the equal value at the
// smaller index (the reference's strict '>' scan from index 0,
// src/ops.cpp:1587-1597).  Values map to unsigned integers in their order
// (sign bit set: complemented, else the sign bit added), -0 taken as +0 so
// that it ties with +0 as the comparison does; the index goes in the low
// word, complemented.  A NaN never wins, except at index 0, where the scan
// never leaves it: the largest key.  Every real key is above 0, the empty
// slot.
__device__ __forceinline__ unsigned long long amax_key(float v, int i)
{
    if (v != v) return i == 0 ? ~0ULL : 0ULL;
    const unsigned u = __builtin_bit_cast(unsigned, v + 0.0f);
    const unsigned ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<unsigned long long>(ord) << 32) | (0xFFFFFFFFu - static_cast<unsigned>(i));
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const unsigned lo = __shfl_xor(static_cast<unsigned>(v), o);
        const unsigned hi = __shfl_xor(static_cast<unsigned>(v >> 32), o);
        const unsigned long long w = (static_cast<unsigned long long>(hi) << 32) | lo;
        v = w > v ? w : v;
    }
    return v;
}

// The token the kAmaxSlots keys give (every lane of the wave): the largest
// key's index; 0 if no key was posted.
__device__ __forceinline__ int amax_token(const unsigned long long* amax)
{
    static_assert(kAmaxSlots == 64, "one slot per lane");
    const unsigned long long k = wave_max_u64(amax[threadIdx.x & 63]);
    return k ? static_cast<int>(0xFFFFFFFFu - static_cast<unsigned>(k)) : 0;
}

// kSteps: unit steps of a row held at once (a row of up to kSteps x lanes
// units is requested whole); rows with more units load the rest step by step.
template <int kType, int kRows, int kSteps, bool kParts = false>
struct RowGroup {
    Unit<kType> un[kSteps][kRows];
    const unsigned char* w[kRows];
    float* out[kRows];
    long long out_stride[kRows];
    bool valid[kRows];
    int row[kRows];  // row index in the launch (segments in order)

    // Segment lookups select among the segment fields held in scalar
    // registers (SegRegs) instead of indexing the kernel arguments with a
    // per-lane segment number, which would turn them into vector loads
    // waited for behind the weights in flight.
    __device__ void locate(const GemvParams& p, const SegRegs& sr, int r_first, int spacing)
    {
#pragma unroll
        for (int k = 0; k < kRows; ++k) {
            const int r = r_first + spacing * k;
            row[k] = r;
            valid[k] = r < p.total_rows;
            int rr = valid[k] ? r : 0;
            const bool in1 = sr.n_seg > 1 && rr >= sr.rows0;
            rr = in1 ? rr - sr.rows0 : rr;
            const bool in2 = in1 && sr.n_seg > 2 && rr >= sr.rows1;
            rr = in2 ? rr - sr.rows1 : rr;
            const long long w_off = (in1 ? sr.w_d1 : 0) + (in2 ? sr.w_d2 : 0);
            const long long out_off = (in1 ? sr.out_d1 : 0) + (in2 ? sr.out_d2 : 0);
            w[k] = p.seg[0].w + w_off + static_cast<long long>(rr) * sr.row_bytes;
            out[k] = reinterpret_cast<float*>(reinterpret_cast<char*>(p.seg[0].out) + out_off) + rr;
            out_stride[k] = sr.stride0 + (in1 ? sr.stride_d1 : 0) + (in2 ? sr.stride_d2 : 0);
        }
    }
    // Unit step `s` (units u0 .. u0+n-1) into buffer b.
    __device__ void load(int b, int u0, int n, int l)
    {
        const int lc = l < n ? l : 0;
#pragma unroll
        for (int k = 0; k < kRows; ++k) un[b][k].load(w[k], u0, n, lc);
    }
    // The first kSteps unit steps of the rows (every lane loads: a step
    // past the row's end reloads step 0).
    __device__ void load_head(int units, int lanes, int l)
    {
#pragma unroll
        for (int b = 0; b < kSteps; ++b) {
            const int u0 = b * lanes < units ? b * lanes : 0;
            load(b, u0, min(lanes, units - u0), l);
        }
    }
    // One vector: the pass's first steps, the outputs' old values (for the
    // residual add) and the rows' RoPE pair (cos, sin), requested together
    // so that all arrive before anything requested later.
    float old[kRows];
    float2 cs[kRows];
    template <int kEpi>
    __device__ void request(const GemvParams& p, const SegRegs& sr, int r_first, int spacing, int units,
                            int lanes, int l)
    {
        locate(p, sr, r_first, spacing);
        load_head(units, lanes, l);
#pragma unroll
        for (int k = 0; k < kRows; ++k) {
            old[k] = *out[k];
            if constexpr (kEpi == kRopeEpi) cs[k] = p.rope[(row[k] & 63) >> 1];
        }
        if constexpr (kParts) {
#pragma unroll
            for (int k = 0; k < kRows; ++k) {
                const float* pr = p.rparts + (out[k] - p.seg[0].out);
#pragma unroll
                for (int g = 0; g < kAttnOutMaxParts; ++g)
                    pv[k][g] = pr[static_cast<long long>(g < p.n_parts ? g : 0) * p.seg[0].rows];
            }
        }
    }
    // The residual's old value of row k: with residual partials, old + ((p0
    // + p1) + ...), summed here, where it is used, so that their loads stay
    // in flight behind the pass's weights until then.
    float pv[kParts ? kRows : 1][kParts ? kAttnOutMaxParts : 1];
    __device__ float residual(const GemvParams& p, int k) const
    {
        if constexpr (!kParts) return old[k];
        float a = pv[k][0];
#pragma unroll
        for (int g = 1; g < kAttnOutMaxParts; ++g)
            if (g < p.n_parts) a += pv[k][g];
        return old[k] + a;
    }
};

// y[v][r] (+)= W[r] . x[v].  A pass of a wave covers kRows rows per lane
// group (kRowsPerWave groups).  kMulti: any number of vectors (one row per
// group then: the dequantised weights of a row stay in registers across the
// vectors, and those of several rows would not fit); else exactly one.
//
// Pipelining: a wave requests its first pass's weights before x is staged,
// so the HBM round trip overlaps the staging, and each later pass's weights
// before it computes the current one (two register buffers, A and B).  The
// grid holds as many workgroups as fit on the GPU at once, so waves keep
// loads in flight from start to end.
template <int kType, int kLanesPerRow, int kRows, int kSteps, bool kMulti, int kEpi>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const GemvParams p)
{
    static_assert(!kMulti || kRows == 1, "several vectors take one row per lane group");
    static_assert(kEpi == kPlain || (!kMulti && (kSteps == 1 || kEpi == kPartsEpi)), "special epilogues: one vector");
    [[maybe_unused]] unsigned long long best = 0;  // kAmaxEpi: this lane's largest argmax key
    static_assert(kEpi != kPairEpi || kRows == 2, "paired rows: two per lane group");
    static_assert(kEpi != kRopeEpi || (kRows == 1 && kLanesPerRow == 32), "RoPE: pairs in one wave");
    constexpr bool kZeroOffsets = kType == kQ8_0 || kType == kQ4_0 || kType == kQ6_K;
    extern __shared__ __align__(16) float xs_all[];  // [n_vec][xs_floats(cols)] padded, then [n_vec][cols / 16] run sums
    __shared__ float s_red[kThreads / 64];

    constexpr int kRowsPerWave = 64 / kLanesPerRow;
    constexpr int kPassRows = kRowsPerWave * kRows;
    const int lane = threadIdx.x & 63;
    const int sub = lane / kLanesPerRow;  // which row of the wave's group
    const int l = lane % kLanesPerRow;
    const int wave = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int n_waves = gridDim.x * (kThreads / 64);
    const int units = p.cols / kUnit;
    const int n_vec = kMulti ? p.n_vec : 1;
    // Paired (SwiGLU) launches: a pass covers kRowsPerWave rows of the gate
    // segment, and each lane group holds row r of the gate and row r of the
    // up matrix (its kRows = 2 rows are seg[0].rows apart).
    constexpr bool pair = kEpi == kPairEpi;
    constexpr int pass_rows = pair ? kRowsPerWave : kPassRows;
    const int spacing = pair ? __builtin_amdgcn_readfirstlane(p.seg[0].rows) : kRowsPerWave;
    const int n_pass = pair ? (p.seg[0].rows + kRowsPerWave - 1) / kRowsPerWave
                            : (p.total_rows + kPassRows - 1) / kPassRows;

    // x for one vector of up to kXRegs x kThreads columns is requested
    // before the weights (loads complete in order, so anything requested
    // after the weights could only be used once they have all arrived), in
    // 16-byte pieces: thread t holds columns 4(t + i kThreads) .. +3.
    // (x for a row of kLanesPerRow x kSteps units, at most)
    constexpr int kXRegs = kLanesPerRow * kSteps * kUnit / kThreads;
    constexpr int kX4 = (kXRegs + 3) / 4;
    const float* const nw = p.norm_w ? p.norm_w : p.x2 ? p.x2 : p.x;
    // The attention + W_o partials are added here only where x is at most 2
    // float4 per thread (their loads, issued together, would otherwise take
    // the registers of the weights in flight); elsewhere the staging below
    // adds them.
    constexpr bool kPartsEarly = kX4 <= 2;
    const bool x_early = !kMulti && p.cols <= kXRegs * kThreads && !(p.norm_w && p.x2) &&
                         (kPartsEarly || !p.xparts) && aligned16(p.x) && aligned16(nw);
    const int cols4 = p.cols / 4;
    float4 xr[kX4], nr[kX4];
    if (x_early) {
#pragma unroll
        for (int i = 0; i < kX4; ++i) {
            const int c4 = threadIdx.x + i * kThreads;
            const int cc = c4 < cols4 ? 4 * c4 : 0;
            xr[i] = ldg4(p.x + cc);
            nr[i] = ldg4(nw + cc);
        }
    }
    // The fused attention + W_o launch's partials for x, requested with x;
    // added once the weights are requested too (a use here would hold the
    // weights' request back until they arrive).
    float4 pp[kPartsEarly ? kX4 : 1][kAttnOutMaxParts];
    const bool parts_early = kPartsEarly && x_early && p.xparts;
    if (parts_early) {
#pragma unroll
        for (int i = 0; i < (kPartsEarly ? kX4 : 1); ++i) {
            const int c4 = threadIdx.x + i * kThreads;
            const int cc = c4 < cols4 ? 4 * c4 : 0;
#pragma unroll
            for (int g = 0; g < kAttnOutMaxParts; ++g)
                pp[i][g] = ldg4(p.xparts + static_cast<long long>(g < p.n_parts ? g : 0) * p.cols + cc);
        }
    }

    const SegRegs sr(p);
    int ps = wave;
    constexpr bool kParts = kEpi == kPartsEpi;
    RowGroup<kType, kRows, kSteps, kParts> ga;
    [[maybe_unused]] RowGroup<kType, kRows, kSteps, kParts> gb;
    if constexpr (kMulti) {
        ga.locate(p, sr, ps * kPassRows + sub, kRowsPerWave);
        ga.load_head(units, kLanesPerRow, l);
    } else {
        ga.template request<kEpi>(p, sr, ps * pass_rows + sub, spacing, units, kLanesPerRow, l);
    }

    // Stage x in LDS (SwiGLU'd when asked), then rmsnorm's scaling in place
    // (each thread rescales the elements it wrote).
    const int xs_len = xs_floats(p.cols);
    float* const s16_all = xs_all + p.n_vec * xs_len;
    const int nb16 = p.cols / 16;
    if (x_early) {
        // One vector, from registers.  rmsnorm's sum of squares and the sums
        // of x over runs of 16 columns (block formats) come from the same
        // registers, in the orders of row_math.h (the rmsnorm kernels' and
        // the staging below's): the 4 threads of a run sit in consecutive
        // lanes.
        if (parts_early) {
            // x + ((p0 + p1) + ...)
#pragma unroll
            for (int i = 0; i < (kPartsEarly ? kX4 : 1); ++i) {
                float4 a = pp[i][0];
#pragma unroll
                for (int g = 1; g < kAttnOutMaxParts; ++g)
                    if (g < p.n_parts)
                        a = make_float4(a.x + pp[i][g].x, a.y + pp[i][g].y, a.z + pp[i][g].z, a.w + pp[i][g].w);
                xr[i] = make_float4(xr[i].x + a.x, xr[i].y + a.y, xr[i].z + a.z, xr[i].w + a.w);
            }
        }
        float4 t[kX4];
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < kX4; ++i) {
            t[i] = p.x2 ? make_float4(silu(xr[i].x) * nr[i].x, silu(xr[i].y) * nr[i].y,
                                      silu(xr[i].z) * nr[i].z, silu(xr[i].w) * nr[i].w)
                        : xr[i];
            if (threadIdx.x + i * kThreads < cols4) ss += sum_sq4(t[i]);
        }
        if (p.norm_w) {
            ss = block_sum<kThreads>(ss, s_red);
            const float rms = 1.0f / sqrtf(ss / static_cast<float>(p.cols) + p.eps);
#pragma unroll
            for (int i = 0; i < kX4; ++i)
                t[i] = make_float4(xr[i].x * rms * nr[i].x, xr[i].y * rms * nr[i].y,
                                   xr[i].z * rms * nr[i].z, xr[i].w * rms * nr[i].w);
        }
#pragma unroll
        for (int i = 0; i < kX4; ++i) {
            const int c4 = threadIdx.x + i * kThreads;
            if (c4 < cols4) *reinterpret_cast<float4*>(xs_all + xpad(4 * c4)) = t[i];
            if constexpr (kZeroOffsets) {
                // cols4 is a multiple of 16, so the 4 lanes of a run agree on c4 < cols4
                float r = sum4(t[i]);
                r += __shfl_xor(r, 1);  // (r0 + r1) + (r2 + r3) in every lane of the run
                r += __shfl_xor(r, 2);
                if (c4 < cols4 && (c4 & 3) == 0) s16_all[c4 >> 2] = r;
            }
        }
    }
    for (int v = 0; v < (x_early ? 0 : p.n_vec); ++v) {
        const float* xv = p.x + v * p.x_stride;
        float* xs = xs_all + v * xs_len;
        float ss = 0.f;
        {
            const float* x2v = p.x2 ? p.x2 + v * p.x_stride : nullptr;
            for (int c = threadIdx.x; c < p.cols; c += kThreads) {
                float t = x2v ? silu(xv[c]) * x2v[c] : xv[c];
                if (p.xparts) t = t + part_sum(p.xparts, p.n_parts, p.cols, c);  // one vector, no x2
                xs[xpad(c)] = t;
                ss += t * t;
            }
        }
        if (p.norm_w) {
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
            if (lane == 0) s_red[threadIdx.x >> 6] = ss;
            __syncthreads();
            ss = 0.f;
#pragma unroll
            for (int w = 0; w < kThreads / 64; ++w) ss += s_red[w];
            __syncthreads();  // s_red is reused by the next vector
            const float rms = 1.0f / sqrtf(ss / static_cast<float>(p.cols) + p.eps);
            for (int c = threadIdx.x; c < p.cols; c += kThreads)
                xs[xpad(c)] = xs[xpad(c)] * rms * p.norm_w[c];
        }
    }
    __syncthreads();
    if (kZeroOffsets && !x_early) {
        // sums of x over each run of 16 columns, pairwise as above (a run
        // is contiguous in LDS: 16 divides the 64-column padding period)
        for (int i = threadIdx.x; i < p.n_vec * nb16; i += kThreads) {
            const int v = i / nb16, b = i - v * nb16;
            const float4* xb = reinterpret_cast<const float4*>(xs_all + v * xs_len + xpad(16 * b));
            s16_all[i] = (sum4(xb[0]) + sum4(xb[1])) + (sum4(xb[2]) + sum4(xb[3]));
        }
        __syncthreads();
    }

    // One pass over the rows in g (its first kSteps unit steps loaded).
    auto run_pass = [&](RowGroup<kType, kRows, kSteps, kParts>& g) {
        const float* xs_base = xs_all;
        float acc[kRows][kGemvMaxVec];
#pragma unroll
        for (int k = 0; k < kRows; ++k)
#pragma unroll
            for (int v = 0; v < kGemvMaxVec; ++v) acc[k][v] = 0.f;
        // dot products of unit step (u0, n) held in buffer b
        auto step = [&](int b, int u0, int n) {
            if (l >= n) return;
#pragma unroll 1
            for (int v = 0; v < n_vec; ++v) {
                const float* xs = xs_base + v * xs_len;
                float pt[kRows][4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    constexpr int kW = Unit<kType>::kW;
                    float xv[16];
#pragma unroll
                    for (int j = 0; j < 16 / kW; ++j)
                        lds_x<kW>(xs, Unit<kType>::xcol(u0, n, l, q, j), xv + kW * j);
#pragma unroll
                    for (int k = 0; k < kRows; ++k) pt[k][q] = g.un[b][k].part(q, xv);
                }
                const float* s16 = s16_all + v * nb16;
#pragma unroll
                for (int k = 0; k < kRows; ++k) {
                    const float f = g.un[b][k].finish(pt[k], s16);
#pragma unroll
                    for (int vv = 0; vv < kGemvMaxVec; ++vv)
                        if (vv == v) acc[k][vv] += f;
                }
            }
        };
        if constexpr (kSteps == 1) {
            // steps after the first (longer rows, several-vector launches
            // only) load one after another
            for (int u0 = 0; u0 < units; u0 += kLanesPerRow) {
                const int n = min(kLanesPerRow, units - u0);
                if (u0 > 0) g.load(0, u0, n, l);
                step(0, u0, n);
            }
        } else {
#pragma unroll
            for (int b = 0; b < kSteps; ++b)
                if (b * kLanesPerRow < units) step(b, b * kLanesPerRow, min(kLanesPerRow, units - b * kLanesPerRow));
        }
        if constexpr (kEpi == kRopeEpi) {
            {
                // RoPE of the q and k projections (src/ops.cpp:1252-1262):
                // rows 2i and 2i+1 of a head are this wave's two lane groups
                // (a pass is 2 rows from an even row), so the partner's sum
                // is one lane swap away.  Rows past rope_rows (v) as computed.
                const float t = row_sum<kLanesPerRow>(acc[0][0]);
                const float u = __shfl_xor(t, 32);
                const float2 c = g.cs[0];
                float y = t;
                if (g.row[0] < p.rope_rows) y = sub == 0 ? rot_lo(t, u, c.x, c.y) : rot_hi(u, t, c.x, c.y);
                if (g.valid[0] && l == kLanesPerRow - 1) *g.out[0] = y;
                return;
            }
        }
        if constexpr (kEpi == kPairEpi) {
            {
                // silu(gate) x up with the reference's operation order
                // (src/ops.cpp:1107-1148), as the batched SwiGLU kernel
                const float tg = row_sum<kLanesPerRow>(acc[0][0]);
                const float tu = row_sum<kLanesPerRow>(acc[1][0]);
                if (g.valid[0] && l == kLanesPerRow - 1) *g.out[0] = silu(tg) * tu;
                return;
            }
        }
        // The group's last lane stores; the old values were read with the
        // pass's request (one vector) or here (several).
#pragma unroll
        for (int k = 0; k < kRows; ++k) {
#pragma unroll
            for (int v = 0; v < kGemvMaxVec; ++v) {
                if (v >= n_vec) break;
                const float t = row_sum<kLanesPerRow>(acc[k][v]);
                float* o = g.out[k] + v * g.out_stride[k];
                const float old = kMulti ? *o : g.residual(p, k);
                if (g.valid[k] && l == kLanesPerRow - 1) *o = p.add ? old + t : t;
                if constexpr (kEpi == kAmaxEpi) {
                    if (g.valid[k] && l == kLanesPerRow - 1) {
                        const unsigned long long key = amax_key(t, g.row[k]);
                        best = key > best ? key : best;
                    }
                }
            }
        }
    };

    if constexpr (kMulti) {
        // One buffer: with several vectors a pass computes long enough per
        // byte, and two buffers of weights would not fit in registers.
        while (ps < n_pass) {
            run_pass(ga);
            ps += n_waves;
            if (ps >= n_pass) break;
            ga.locate(p, sr, ps * kPassRows + sub, kRowsPerWave);
            ga.load_head(units, kLanesPerRow, l);
        }
        return;
    }
    // Passes ps, ps + n_waves, ... alternate between the buffers; the next
    // pass's request goes out before the current pass is computed.  Past the
    // last pass the request reads row 0 again (locate maps it there).
    while (ps < n_pass) {
        gb.template request<kEpi>(p, sr, (ps + n_waves) * pass_rows + sub, spacing, units, kLanesPerRow, l);
        __builtin_amdgcn_sched_barrier(0);  // the request goes out before the compute
        run_pass(ga);
        ps += n_waves;
        if (ps >= n_pass) break;
        ga.template request<kEpi>(p, sr, (ps + n_waves) * pass_rows + sub, spacing, units, kLanesPerRow, l);
        __builtin_amdgcn_sched_barrier(0);
        run_pass(gb);
        ps += n_waves;
    }
    if constexpr (kEpi == kAmaxEpi) {
        // the workgroup's largest key: over the wave, then over the waves;
        // one atomic per workgroup
        __shared__ unsigned long long s_best[kThreads / 64];
        best = wave_max_u64(best);
        if (lane == 0) s_best[threadIdx.x >> 6] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
#pragma unroll
            for (int w = 1; w < kThreads / 64; ++w) best = s_best[w] > best ? s_best[w] : best;
            if (best) atomicMax(p.amax + blockIdx.x % kAmaxSlots, best);
        }
    }
}

// ---- decode attention over a short context fused with W_o --------------------
//
// One launch in place of a decode step's attention launch and its W_o
// product (src/forward.cpp:198-213) when the context has at most
// kAttnOutMaxPos positions.  Workgroup (b, g) takes W_o rows 32b .. 32b+31
// restricted to the columns of kv head g's q heads, a row-major sub-matrix
// (the row stride of W_o, its base gqa * 64 columns in), recomputes those
// heads' attention (src/ops.cpp:1377-1511) over the cached positions, and
// writes its rows' partial products parts[g][row].  The launches after it
// add the partials to the residual (the gate/up launch's x staging, the
// W_down launch's residual base, both in the order of part_sum), so no
// workgroup waits for another: each kv head's attention is recomputed by
// the rows / 32 workgroups that need it, from cache rows that sit in L2
// after the first of them.
//
// q and the wave's first K and V tile are requested first, then the W_o
// weights of the lane (one 64-column unit of one row: 8 lanes per row, 8
// rows per wave), which are used last: loads complete in order, and the
// attention waiting behind the weights measured 532-535 against 515-516 us
// per token (Q4_0, 20 tokens after a 32-token prompt).  Wave w takes the
// 16-position tiles w, w + 4, w + 8 (each tile's successor requested before
// it is computed), with the decode kernel's MFMA layouts:
//   S^T[16 pos][16 heads] = K[16 pos][64] . Q^T[64][16 heads]   16 x v_mfma_f32_16x16x4f32
//   O^T[64 d][16 heads]  += V^T[64 d][16 pos] . P^T[16 pos][16 heads]
// (heads gqa .. 15 zero; lane 16k + i holds dims 16k .. 16k+15 of key i and
// of q head i, and the S accumulator is the P.V B operand), and a running
// maximum and sum per head.  The waves meet in LDS twice: for the heads'
// maxima, then for the sums and O scaled to them, added in wave order.  The
// output is the x of the W_o sub-matrix, staged as the GEMV stages x
// (padded, with the 16-column sums).
//
// Against the attention launch and the W_o GEMV it replaces (MI355X, Q4_0
// TinyLlama, 20 greedy tokens after prompts of 32-200 tokens): 534 against
// 580 us per token at positions 32-51, 576 against 612 at 100-119, 610
// against 632 at 140-159, 614 against 631 at 170-189 (three tiles per
// wave), 644 against 635 at 200-219 (a fourth tile): hence 192 positions.
typedef float attn_f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ attn_f4 mfma16x4(float a, float b, attn_f4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr int kAttnOutRows = 32;  // W_o rows per workgroup: 4 waves x 8 rows of 8 lanes
constexpr int kAttnOutCols = kAttnOutMaxGqa * 64;

template <int kType>
__global__ __launch_bounds__(kThreads) void attn_out_kernel(const AttnOutParams p)
{
    static_assert(kThreads == 256 && kAttnOutMaxPos % 64 == 0, "4 waves of 16-position tiles");
    __shared__ __align__(16) float xs[xs_floats(kAttnOutCols)];
    __shared__ float s16[kAttnOutCols / 16];
    __shared__ float s_max[4][16], s_sum[4][16];
    __shared__ float s_o[4][16 * 65];  // O of each wave, [head][dim], rows padded to 65

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = blockIdx.y;
    const int units = p.gqa;  // 64-column units of a row's group

    // ---- W_o: lane l of row group `sub` holds unit l of its row (loaded
    // after the attention's operands) ----
    const int sub = lane >> 3, l = lane & 7;
    const int lu = l < units ? l : 0;  // lanes past the row's units load unit 0 (not used)
    const int row = blockIdx.x * kAttnOutRows + wave * 8 + sub;
    const bool valid = row < p.rows;
    const unsigned char* wrow = p.w + static_cast<long long>(valid ? row : 0) * p.row_bytes +
                                static_cast<long long>(g) * p.group_bytes;
    Unit<kType> un;

    // ---- attention of the group's heads: wave w takes the 16-position
    // tiles w, w + 4, ... (rows past n_pos read row 0, masked; V rows there
    // are weighted by 0), with a running maximum, sum and O per head, the
    // next tile's K and V requested before the current one is computed ----
    const int i = lane & 15, k4 = lane >> 4;
    const bool head = i < p.gqa;
    const int n_tiles = (p.n_pos + 15) >> 4;
    const float* kg = p.kc + 64 * g + 16 * k4;  // this lane's K dims of position 0
    const float* vg = p.vc + 64 * g + 4 * i;    // this lane's V dims of position 0
    auto load_tile = [&](int j, float4 (&kr)[4], float4 (&vr)[4]) {
        const int pk = 16 * j + i;
        const float4* k4p = reinterpret_cast<const float4*>(kg + static_cast<long long>(pk < p.n_pos ? pk : 0) * p.kv_dim);
#pragma unroll
        for (int s = 0; s < 4; ++s) kr[s] = k4p[s];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int pv = 16 * j + 4 * k4 + s;
            vr[s] = *reinterpret_cast<const float4*>(vg + static_cast<long long>(pv < p.n_pos ? pv : 0) * p.kv_dim);
        }
    };
    float4 qr[4];
    {
        const float4* qr4 = reinterpret_cast<const float4*>(p.q + static_cast<long long>(g * p.gqa + (head ? i : 0)) * 64 +
                                                            16 * k4);
#pragma unroll
        for (int s = 0; s < 4; ++s) qr[s] = qr4[s];
    }
    float4 kb[2][4], vb[2][4];
    if (wave < n_tiles) load_tile(wave, kb[0], vb[0]);
    un.load(wrow, 0, units, lu);  // the weights after q, K and V: used last
    constexpr float kScale = 0.125f * 1.4426950408889634f;  // 1 / sqrt(64) in log2 units
    float m_run = -__builtin_huge_valf(), l_run = 0.f;
    attn_f4 o[4] = {};
#pragma unroll
    for (int it = 0; it < kAttnOutMaxPos / 64; ++it) {
        const int j = wave + 4 * it;
        if (j >= n_tiles) break;  // uniform per wave
        float4 (&kr)[4] = kb[it & 1];
        float4 (&vr)[4] = vb[it & 1];
        if (it + 1 < kAttnOutMaxPos / 64 && j + 4 < n_tiles) load_tile(j + 4, kb[(it + 1) & 1], vb[(it + 1) & 1]);
        // S^T: lane 16 k4 + i holds positions 16 j + 4 k4 + r of head i
        attn_f4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const float qv[4] = {head ? qr[s].x : 0.f, head ? qr[s].y : 0.f, head ? qr[s].z : 0.f,
                                 head ? qr[s].w : 0.f};
            const float kv[4] = {kr[s].x, kr[s].y, kr[s].z, kr[s].w};
#pragma unroll
            for (int c = 0; c < 4; ++c) sacc = mfma16x4(kv[c], qv[c], sacc);
        }
        float t[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
            t[r] = 16 * j + 4 * k4 + r < p.n_pos ? sacc[r] * kScale : -__builtin_huge_valf();
        float m = fmaxf(fmaxf(t[0], t[1]), fmaxf(t[2], t[3]));
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
        const float m_new = fmaxf(m_run, m);  // finite: position 16 j is in the context
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the wave's first tile
        float pr[4], lsum = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            pr[r] = __builtin_amdgcn_exp2f(t[r] - m_new);  // exp2(-inf) = 0 for masked positions
            lsum += pr[r];
        }
        lsum += __shfl_xor(lsum, 16);
        lsum += __shfl_xor(lsum, 32);
        l_run = l_run * alpha + lsum;
        m_run = m_new;
        // O^T block b, rows 4 k4 + r: dim 4 (4 k4 + r) + b of head i
#pragma unroll
        for (int b = 0; b < 4; ++b) o[b] *= alpha;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const float vv[4] = {vr[s].x, vr[s].y, vr[s].z, vr[s].w};
#pragma unroll
            for (int b = 0; b < 4; ++b) o[b] = mfma16x4(vv[b], pr[s], o[b]);
        }
    }
    // the waves' states scaled to the heads' common maximum (position 0 is
    // wave 0's: finite); a wave without tiles contributes 0
    if (k4 == 0) s_max[wave][i] = m_run;
    __syncthreads();
    const float mg = fmaxf(fmaxf(s_max[0][i], s_max[1][i]), fmaxf(s_max[2][i], s_max[3][i]));
    const float sw = __builtin_amdgcn_exp2f(m_run - mg);
    if (k4 == 0) s_sum[wave][i] = l_run * sw;
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) s_o[wave][65 * i + 4 * (4 * k4 + r) + b] = o[b][r] * sw;
    __syncthreads();

    // attention output of the group's heads = x of the W_o sub-matrix
    const int ncols = 64 * p.gqa;
    for (int c = threadIdx.x; c < ncols; c += kThreads) {
        const int h = c >> 6, d = c & 63;
        const float num = ((s_o[0][65 * h + d] + s_o[1][65 * h + d]) + s_o[2][65 * h + d]) + s_o[3][65 * h + d];
        const float den = ((s_sum[0][h] + s_sum[1][h]) + s_sum[2][h]) + s_sum[3][h];
        xs[xpad(c)] = num / den;
    }
    __syncthreads();
    constexpr bool kZeroOffsets = kType == kQ8_0 || kType == kQ4_0 || kType == kQ6_K;
    if constexpr (kZeroOffsets) {
        for (int b = threadIdx.x; b < ncols / 16; b += kThreads) {
            const float4* xb = reinterpret_cast<const float4*>(xs + xpad(16 * b));
            s16[b] = (sum4(xb[0]) + sum4(xb[1])) + (sum4(xb[2]) + sum4(xb[3]));
        }
        __syncthreads();
    }

    // ---- the rows' partial products ----
    float pt[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        constexpr int kW = Unit<kType>::kW;
        float xv[16];
#pragma unroll
        for (int j = 0; j < 16 / kW; ++j) lds_x<kW>(xs, Unit<kType>::xcol(0, units, lu, q, j), xv + kW * j);
        pt[q] = un.part(q, xv);
    }
    float f = l < units ? un.finish(pt, s16) : 0.f;
    f += __shfl_xor(f, 1);
    f += __shfl_xor(f, 2);
    f += __shfl_xor(f, 4);
    if (valid && l == 0) p.parts[static_cast<long long>(g) * p.rows + row] = f;
}

__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(float* out, const float* x,
                                                           const float* w, int size, float eps)
{
    __shared__ float s_red[kThreads / 64];
    const float ss = row_sum_squares<kThreads>(x, size, s_red);
    const float rms = 1.0f / sqrtf(ss / static_cast<float>(size) + eps);
    for (int c = threadIdx.x; c < size; c += kThreads) out[c] = x[c] * rms * w[c];
}

__global__ __launch_bounds__(kThreads) void vec_add_kernel(float* out, const float* x, int size)
{
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i < size) out[i] += x[i];
}

__global__ __launch_bounds__(kThreads) void silu_kernel(float* x, int size)
{
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i < size) x[i] = silu(x[i]);
}

__global__ __launch_bounds__(kThreads) void elementwise_mul_kernel(float* a, const float* b, int size)
{
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i < size) a[i] *= b[i];
}

// Element i of one table row, with embed_token()'s expressions
// (src/forward.cpp:17-134): value * scale, Q6_K d * scale * q.
__device__ float embed_elem(int type, const unsigned char* row, int i)
{
    switch (type) {
    case kF32: return reinterpret_cast<const float*>(row)[i];
    case kF16: return half_bits_to_float(reinterpret_cast<const unsigned short*>(row)[i]);
    case kQ8_0: {
        const unsigned char* blk = row + 34 * (i >> 5);
        const float scale = half_bits_to_float(blk[0] | (blk[1] << 8));
        return static_cast<float>(static_cast<signed char>(blk[2 + (i & 31)])) * scale;
    }
    case kQ4_0: {
        const unsigned char* blk = row + 18 * (i >> 5);
        const float scale = half_bits_to_float(blk[0] | (blk[1] << 8));
        const int j = i & 31;
        const int q = j < 16 ? (blk[2 + j] & 0x0F) : (blk[2 + j - 16] >> 4);
        return static_cast<float>(q - 8) * scale;
    }
    default: {  // kQ6_K
        const unsigned char* blk = row + 210 * (i >> 8);
        const int r = i & 255, h = r >> 7, k = (r & 127) >> 5, l = r & 31;
        const unsigned char* ql = blk + 64 * h;
        const unsigned char* qh = blk + 128 + 32 * h;
        const signed char* sc = reinterpret_cast<const signed char*>(blk + 192) + 8 * h;
        const float d = half_bits_to_float(blk[208] | (blk[209] << 8));
        const int lo = (k & 1) ? ql[l + 32] : ql[l];
        const int q = ((k < 2 ? (lo & 0x0F) : (lo >> 4)) | (((qh[l] >> (2 * k)) & 3) << 4)) - 32;
        return d * static_cast<float>(sc[(l >> 4) + 2 * k]) * static_cast<float>(q);
    }
    }
}

// Row blockIdx.y of out [n_tok][n] = table row tokens_dev[blockIdx.y] (or
// `token` when tokens_dev is null).
// With amax (one row): the token the argmax keys there give; token_out
// (non-null) receives it from workgroup 0.
__global__ __launch_bounds__(kThreads) void embed_kernel(int type, float* out,
                                                         const unsigned char* table, long long row_bytes,
                                                         int token, const int* tokens_dev,
                                                         const unsigned long long* amax, int* token_out, int n)
{
    const int t = amax ? amax_token(amax) : tokens_dev ? tokens_dev[blockIdx.y] : token;
    if (token_out && blockIdx.x == 0 && threadIdx.x == 0) token_out[blockIdx.y] = t;
    const unsigned char* row = table + row_bytes * t;
    float* o = out + static_cast<long long>(blockIdx.y) * n;
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < n; i += gridDim.x * kThreads)
        o[i] = embed_elem(type, row, i);
}

// (value, index) pairs: b beats a when larger, or equal at a smaller index;
// NaN values never beat anything (the reference's strict '>' scan).
__device__ __forceinline__ bool beats(float vb, int ib, float va, int ia)
{
    return vb > va || (vb == va && ib < ia);
}

__global__ __launch_bounds__(1024) void argmax_kernel(int* out, int* out2, const float* x, int n)
{
    __shared__ float s_v[16];
    __shared__ int s_i[16];
    float bv = -__builtin_huge_valf();
    int bi = 0x7fffffff;
    // x[0] (for the NaN rule below) goes out with the first batch
    const float x0 = x[0];
    // 32 independent loads in flight per thread: a 32768-entry vocabulary
    // is one round trip
    constexpr int kPer = 32;
    for (int i0 = threadIdx.x; i0 < n; i0 += kPer * 1024) {
        float v[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int i = i0 + j * 1024;
            v[j] = x[i < n ? i : i0];
        }
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int i = i0 + j * 1024;
            if (i < n && beats(v[j], i, bv, bi)) {
                bv = v[j];
                bi = i;
            }
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (beats(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        s_v[threadIdx.x >> 6] = bv;
        s_i[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; ++w)
            if (beats(s_v[w], s_i[w], bv, bi)) {
                bv = s_v[w];
                bi = s_i[w];
            }
        // nothing above -inf: index 0 (where the scan starts); a NaN at index
        // 0 is never beaten in the reference's scan, so 0 as well
        const int r = (bi == 0x7fffffff || x0 != x0) ? 0 : bi;
        *out = r;
        if (out2) *out2 = r;
    }
}

// Workgroups of one kernel that fit on the current device at once (its CU
// count x the occupancy the kernel's registers and LDS allow), cached per
// device and LDS size.
// Workgroups of one launch: as many as fit on the GPU at once, or, with
// `two_per_cu`, at most two per CU.
template <typename Kernel>
int resident_blocks(Kernel kernel, size_t lds, bool two_per_cu)
{
    struct Entry {
        int device = -1;
        size_t lds = 0;
        int blocks = 0;
        int cus = 0;
    };
    static thread_local Entry cache[4];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    for (const Entry& e : cache)
        if (e.device == dev && e.lds == lds) return two_per_cu ? std::min(e.blocks, 2 * e.cus) : e.blocks;
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, lds) != hipSuccess)
        return 256;
    cus = std::max(1, cus);
    const int blocks = cus * std::max(1, per_cu);
    static thread_local int next = 0;
    cache[next] = Entry{dev, lds, blocks, cus};
    next = (next + 1) % 4;
    return two_per_cu ? std::min(blocks, 2 * cus) : blocks;
}

template <int kType, int kLanes, int kRows, int kSteps, bool kMulti, int kEpi = kPlain>
hipError_t launch_shaped(const GemvParams& p, hipStream_t s)
{
    const size_t lds = static_cast<size_t>(p.n_vec) * (xs_floats(p.cols) + p.cols / 16) * sizeof(float);
    constexpr int kPassRowsPerBlock = (kThreads / 64) * (64 / kLanes) * kRows;
    const int needed = (p.total_rows + kPassRowsPerBlock - 1) / kPassRowsPerBlock;
    const auto kernel = gemv_kernel<kType, kLanes, kRows, kSteps, kMulti, kEpi>;
    // A launch whose x goes through a prologue (rmsnorm, SwiGLU) takes at
    // most two workgroups per CU: every workgroup stages and normalises x
    // itself, and fewer, equal shares per CU measured faster.  MI355X, greedy
    // decode at TinyLlama shapes (the rmsnorm + gate/up launch: 704 -> 512
    // workgroups; the classifier: its resident grid -> 512): Q4_0 579-588
    // against 598-601 us per token, Q8_0 645 against 656, F16 790 against
    // 806.  Launches without a prologue keep the resident grid (the 32000 x
    // 2048 GEMV alone: F16, F32, Q6_K 0.7-1.2 % slower with the cap).
    const int blocks = std::min(needed, resident_blocks(kernel, lds, p.norm_w != nullptr || p.x2 != nullptr));
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kThreads), lds, s, p);
    return hipGetLastError();
}

// Lanes per row: 32 when a row has at most 32 units (cols <= 2048), else
// 64; a row of up to 128 units (cols <= 8192) is requested whole (two unit
// steps per lane).  Rows per lane group: the format's kRows with one vector
// when the rows still give every resident wave a pass, else 1.
template <int kType>
hipError_t launch_typed(const GemvParams& p, hipStream_t s)
{
    const int units = p.cols / kUnit;
    if (p.rope_rows > 0) return launch_shaped<kType, 32, 1, 1, false, kRopeEpi>(p, s);  // gemv_can_rope
    if (p.amax) {  // one vector, one segment, rows of <= 64 units, no residual
        if (p.n_vec != 1 || p.n_seg != 1 || units > 64 || p.pair || p.add || p.rparts) return hipErrorInvalidValue;
        constexpr int kR = Unit<kType>::kRows;
        return units <= 32 ? launch_shaped<kType, 32, kR, 1, false, kAmaxEpi>(p, s)
                           : launch_shaped<kType, 64, kR, 1, false, kAmaxEpi>(p, s);
    }
    if (p.rparts) {  // gemv_can_add_parts: one vector, one segment, rows of <= 128 units
        if (p.n_vec != 1 || p.n_seg != 1 || units > 128 || p.pair) return hipErrorInvalidValue;
        return units <= 32   ? launch_shaped<kType, 32, 1, 1, false, kPartsEpi>(p, s)
               : units <= 64 ? launch_shaped<kType, 64, 1, 1, false, kPartsEpi>(p, s)
                             : launch_shaped<kType, 64, 1, 2, false, kPartsEpi>(p, s);
    }
    if (p.pair) {  // gemv_can_pair: one vector, a two-row format, rows of <= 64 units
        if constexpr (Unit<kType>::kRows == 2)
            return units <= 32 ? launch_shaped<kType, 32, 2, 1, false, kPairEpi>(p, s)
                               : launch_shaped<kType, 64, 2, 1, false, kPairEpi>(p, s);
        return hipErrorInvalidValue;
    }
    // several vectors, or rows longer than two steps of 64 lanes: one row per
    // lane group, steps beyond the first loaded one after another
    if (p.n_vec > 1 || units > 128)
        return units <= 32 ? launch_shaped<kType, 32, 1, 1, true>(p, s)
                           : launch_shaped<kType, 64, 1, 1, true>(p, s);
    if (units > 64 && units <= 128) return launch_shaped<kType, 64, 1, 2, false>(p, s);
    const bool narrow = units <= 32;
    constexpr int kR = Unit<kType>::kRows;
    if constexpr (kR > 1) {
        const int passes = (p.total_rows + kR - 1) / kR / (narrow ? 2 : 1);  // wave passes
        if (passes >= 4 * 256 * 4)
            return narrow ? launch_shaped<kType, 32, kR, 1, false>(p, s)
                          : launch_shaped<kType, 64, kR, 1, false>(p, s);
    }
    return narrow ? launch_shaped<kType, 32, 1, 1, false>(p, s) : launch_shaped<kType, 64, 1, 1, false>(p, s);
}

}  // namespace

hipError_t load_gemv_code()
{
    hipFuncAttributes a;
    return hipFuncGetAttributes(&a, reinterpret_cast<const void*>(&vec_add_kernel));
}

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

bool gemv_can_add_parts(int cols)
{
    return cols / kUnit <= 128;
}

bool gemv_can_amax(int cols)
{
    return cols / kUnit <= 64;
}

bool gemv_can_rope(int cols)
{
    return cols / kUnit <= 32;
}

bool gemv_can_pair(int type, int rows, int cols)
{
    const int units = cols / kUnit;
    const bool two_rows = type == kQ8_0 || type == kQ4_0 || type == kQ6_K;
    return two_rows && units <= 64 && rows % (units <= 32 ? 2 : 1) == 0;
}

bool attn_out_supported(int type, int gqa, int n_head_kv, int n_pos)
{
    if (gqa < 1 || gqa > kAttnOutMaxGqa || n_head_kv < 1 || n_head_kv > kAttnOutMaxParts || n_pos < 1 ||
        n_pos > kAttnOutMaxPos)
        return false;
    switch (type) {
    case kF32:
    case kF16:
    case kQ8_0:
    case kQ4_0: return true;
    case kQ6_K: return (64 * gqa) % 256 == 0;  // the group's columns are whole super-blocks
    default: return false;
    }
}

hipError_t launch_attn_out(int type, const AttnOutParams& p, hipStream_t s)
{
    if (!attn_out_supported(type, p.gqa, p.n_head_kv, p.n_pos) || p.rows < 1 || !p.q || !p.kc || !p.vc ||
        !p.w || !p.parts || p.kv_dim != 64 * p.n_head_kv)
        return hipErrorInvalidValue;
    const dim3 grid((p.rows + kAttnOutRows - 1) / kAttnOutRows, p.n_head_kv);
    switch (type) {
    case kF32: hipLaunchKernelGGL(attn_out_kernel<kF32>, grid, dim3(kThreads), 0, s, p); break;
    case kF16: hipLaunchKernelGGL(attn_out_kernel<kF16>, grid, dim3(kThreads), 0, s, p); break;
    case kQ8_0: hipLaunchKernelGGL(attn_out_kernel<kQ8_0>, grid, dim3(kThreads), 0, s, p); break;
    case kQ4_0: hipLaunchKernelGGL(attn_out_kernel<kQ4_0>, grid, dim3(kThreads), 0, s, p); break;
    case kQ6_K: hipLaunchKernelGGL(attn_out_kernel<kQ6_K>, grid, dim3(kThreads), 0, s, p); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
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

hipError_t launch_silu(float* x, int size, hipStream_t s)
{
    hipLaunchKernelGGL(silu_kernel, dim3((size + kThreads - 1) / kThreads), dim3(kThreads), 0, s, x, size);
    return hipGetLastError();
}

hipError_t launch_elementwise_mul(float* a, const float* b, int size, hipStream_t s)
{
    hipLaunchKernelGGL(elementwise_mul_kernel, dim3((size + kThreads - 1) / kThreads), dim3(kThreads), 0,
                       s, a, b, size);
    return hipGetLastError();
}

hipError_t launch_embed(int type, float* out, const unsigned char* table, int token,
                        const int* tokens_dev, int n_tok, int n, hipStream_t s,
                        const unsigned long long* amax, int* token_out)
{
    if (amax && n_tok != 1) return hipErrorInvalidValue;
    const int blocks = std::min(64, (n + kThreads - 1) / kThreads);
    hipLaunchKernelGGL(embed_kernel, dim3(blocks, n_tok), dim3(kThreads), 0, s, type, out, table,
                       weight_row_bytes(type, n), token, tokens_dev, amax, token_out, n);
    return hipGetLastError();
}

__global__ __launch_bounds__(64) void amax_token_kernel(const unsigned long long* amax, int* out)
{
    const int t = amax_token(amax);
    if (threadIdx.x == 0) *out = t;
}

hipError_t launch_amax_token(const unsigned long long* amax, int* out, hipStream_t s)
{
    hipLaunchKernelGGL(amax_token_kernel, dim3(1), dim3(64), 0, s, amax, out);
    return hipGetLastError();
}

hipError_t launch_argmax(int* out, int* out2, const float* x, int n, hipStream_t s)
{
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, out, out2, x, n);
    return hipGetLastError();
}

hipError_t launch_vec_add(float* out, const float* x, int size, hipStream_t s)
{
    hipLaunchKernelGGL(vec_add_kernel, dim3((size + kThreads - 1) / kThreads), dim3(kThreads), 0, s,
                       out, x, size);
    return hipGetLastError();
}

}  // namespace tla
