// Causal prefill attention for gfx950 (fp32 MFMA, fp32 accumulation).
//
// Reference semantics: the prompt is fed token by token (src/generate.cpp:
// 56-59); for the attention block that is, for t = 0..n_tok-1 at position
// P = pos0 + t: rope(q_t, k_t, P) (src/ops.cpp:1223-1281), append k_t,v_t at
// P (src/ops.cpp:1370-1371), then attention of q_t over cache positions
// 0..P (src/ops.cpp:1377-1511).  Because token t only ever sees keys
// 0..P, the whole prompt is one causal (lower-triangular) attention over
// the cache after all appends -- which is what these kernels compute.
//
// prefill_append_kernel: rotates every k row (when asked) and writes k and v
//   rows to the cache.  Bit-exact with the reference's append.
//
// prefill_attention_kernel: one workgroup = 4 waves = 4 q heads of one kv
//   head, over one tile of 32 query tokens.  Each wave:
//     S^T[32 keys][32 queries] = K[32][64] . Q^T[64][32]   32 x mfma_f32_32x32x2f32
//     causal mask, online softmax per query row (the running max moves
//       only when it grows by more than 2^8, so most tiles skip rescaling O)
//     O^T[64 d][32 queries]   += V^T[64][32] . P^T[32][32] 32 x mfma_f32_32x32x2f32
//   The S accumulator layout (lane l: query l%32, keys 8*(g/4)+4*(l/32)+g%4)
//   is the B operand of the P.V product as is, so P never leaves registers.
//   Q (rotated in registers with the host-built table) is loaded once.
//
// Scheduling: key/value tiles of one (layer, kv head) are read by all its
//   query tiles and q heads, so those workgroups are placed on one XCD
//   (workgroup i runs on XCD i % 8) to share that XCD's L2, and each XCD
//   starts the query tiles with the most key tiles first, across all of its
//   (layer, kv head) pairs, so the last workgroups to start are short ones.
#include "lane_math.h"
#include "rope_math.h"
#include "tla_internal.h"

namespace tla {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kQTile = 32;
constexpr int kKTile = 32;
constexpr int kWavesP = 4;
constexpr int kXcds = 8;

__device__ __forceinline__ floatx16 mfma32(float a, float b, floatx16 c)
{
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__global__ __launch_bounds__(256) void prefill_append_kernel(const PrefillParams p)
{
    const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
    const int c4 = (int)(gid & 15);  // float4 within the 64-float row
    const long long row = gid >> 4;  // (lb, t, kvh)
    const long long n_rows = (long long)p.n_lb * p.n_tok * p.n_head_kv;
    if (row >= n_rows) return;
    const int kvh = (int)(row % p.n_head_kv);
    const long long lt = row / p.n_head_kv;
    const int t = (int)(lt % p.n_tok);
    const int lb = (int)(lt / p.n_tok);
    const int pos = p.pos0 + t;
    const float* tab = reinterpret_cast<const float*>(p.rope + (long long)pos * kPairs);
    const float4 k_in = ldg4(p.k + row * kHeadDim + 4 * c4);
    const float4 cs = ldg4(tab + 4 * c4);  // loaded either way: no branch before the loads
    const float4 kx = p.rotate ? rotate4(k_in, cs) : k_in;
    const long long dst = (long long)(p.layer0 + lb) * p.layer_stride +
                          ((long long)pos * p.n_head_kv + kvh) * kHeadDim + 4 * c4;
    stg4(p.kc + dst, kx);
    stg4(p.vc + dst, ldg4(p.v + row * kHeadDim + 4 * c4));
}

struct PrefillGrid {
    int n_qt;     // query tiles
    int n_hg;     // head groups of 4 waves per kv head
    int n_pairs;  // n_lb * n_head_kv
    int per_xcd;  // workgroup slots per XCD: ceil(n_pairs / 8) * n_hg * n_qt
    // Quotients by the launch's divisors as multiply-highs: q = mulhi(n, m)
    // with m = ceil(2^32 / d), exact for n * d < 2^32 (checked at launch); a
    // divisor of 1 has m = 0 and takes q = n.  The XCDs below n_pairs % 8
    // (all when it is 0) hold ceil(n_pairs / 8) pairs, the others one fewer.
    unsigned m_rank_big, m_rank_small;  // pairs per XCD x n_hg
    unsigned m_hg;                      // n_hg
    unsigned m_kv;                      // n_head_kv
};

// The rotation of rotate4 with fused multiply-adds: 8 operations per float4
// instead of 12, each output within an ulp or so of the separately rounded
// form.  For operands that are not stored (q).
__device__ __forceinline__ float4 rotate4_fma(float4 x, float4 cs)
{
    return make_float4(__builtin_fmaf(x.x, cs.x, -(x.y * cs.y)), __builtin_fmaf(x.x, cs.y, x.y * cs.x),
                       __builtin_fmaf(x.z, cs.z, -(x.w * cs.w)), __builtin_fmaf(x.z, cs.w, x.w * cs.z));
}

__device__ __forceinline__ unsigned div_magic(unsigned n, unsigned m)
{
    return m ? __umulhi(n, m) : n;
}

constexpr float kRescaleSlack = 8.f;  // log2 units
constexpr int kRowPad = 68;  // LDS row stride (floats): 64 + 4 keeps operand reads conflict-free

__global__ __launch_bounds__(64 * kWavesP) __attribute__((amdgpu_waves_per_eu(3, 3))) void
prefill_attention_kernel(const PrefillParams p, const PrefillGrid g)
{
    // K and V tiles of 32 keys, shared by the 4 waves, double-buffered.
    __shared__ float sk[2][kKTile][kRowPad];
    __shared__ float sv[2][kKTile][kRowPad];

    // ---- XCD-aware, heavy-first mapping of workgroups to tiles ----
    // Workgroup b runs on XCD b % 8 and XCDs start their workgroups in order
    // of b / 8.  (layer, kv head) pair i belongs to XCD i % 8, so all query
    // tiles of a pair share one L2; within an XCD, query tiles are handed out
    // longest first (most key tiles) across all its pairs.
    // The quotients are multiply-highs on scalar registers: a workgroup that
    // starts beside two MFMA-bound waves gets few vector issue slots, and
    // the compiler's divisions go through the vector unit.
    const int xcd = blockIdx.x % kXcds;
    const int slot = blockIdx.x / kXcds;
    const int xcd_pairs = (g.n_pairs - xcd + kXcds - 1) / kXcds;
    const bool big = xcd_pairs * kXcds >= g.n_pairs;  // this XCD holds ceil(n_pairs / 8) pairs
    const int per_rank = xcd_pairs * g.n_hg;
    if (slot >= per_rank * g.n_qt) return;  // whole workgroup
    const int rank = (int)div_magic((unsigned)slot, big ? g.m_rank_big : g.m_rank_small);
    const int qt = g.n_qt - 1 - rank;
    const int rem = slot - rank * per_rank;
    const int pg = (int)div_magic((unsigned)rem, g.m_hg);
    const int pair = xcd + kXcds * pg;  // (lb, kvh)
    const int hg = rem - pg * g.n_hg;
    const int lb = (int)div_magic((unsigned)pair, g.m_kv);
    const int kvh = pair - lb * p.n_head_kv;

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // scalar
    const int lane = threadIdx.x & 63;
    const int hq = hg * kWavesP + wave;
    const bool computes = hq < p.gqa;  // uniform per wave; others only load tiles
    const int qh = kvh * p.gqa + (computes ? hq : 0);

    const int col = lane & 31;  // query row within the tile
    const int half = lane >> 5; // which 32 of the 64 dims (Q/K) / key sub-block
    const int i0 = qt * kQTile;
    const int trow = min(i0 + col, p.n_tok - 1);  // clamped token index
    const int qpos = p.pos0 + i0 + col;           // this row's position
    const int last_key = p.pos0 + min(i0 + kQTile - 1, p.n_tok - 1);
    const int n_kt = last_key / kKTile + 1;  // key tiles covering 0..last_key
    // Tiles below (pos0 + i0 + 1) / 32 end at or before the tile's first query
    // position: no key in them is masked for any row.
    const int n_plain = min((p.pos0 + i0 + 1) / kKTile, n_kt - 1);

    const int kv_dim = p.n_head_kv * kHeadDim;
    const long long layer_off = (long long)(p.layer0 + lb) * p.layer_stride + (long long)kvh * kHeadDim;
    const float* kc = p.kc + layer_off;
    const float* vc = p.vc + layer_off;

    // ---- cooperative tile loads: thread -> rows t/16 and t/16 + 16, float4 t%16.
    // Keys past last_key are clamped to it (masked in the scores, or never
    // used).  Byte offsets are 32-bit from a uniform base (one layer's cache
    // slice is < 4 GiB).
    const int lrow = threadIdx.x >> 4, lc4 = threadIdx.x & 15;
    auto gload = [&](const float* base, int tile, float4* dst) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const unsigned key = (unsigned)min(tile * kKTile + lrow + 16 * h, last_key);
            dst[h] = ldg4_at(base, (key * (unsigned)kv_dim + 4u * lc4) * 4u);
        }
    };
    auto lstore = [&](float (*buf)[kRowPad], const float4* src) {
#pragma unroll
        for (int h = 0; h < 2; ++h) *reinterpret_cast<float4*>(&buf[lrow + 16 * h][4 * lc4]) = src[h];
    };

    // ---- Q^T operand: lane holds q[row][32*half + s] * scale * log2(e) ----
    float4 qv[8];
    {
        const float* qrow = p.q + (((long long)lb * p.n_tok + trow) * p.n_head + qh) * kHeadDim + 32 * half;
        const float* tab = reinterpret_cast<const float*>(p.rope + (long long)(p.pos0 + trow) * kPairs);
        // All sixteen loads are issued before any is used.
        float4 cs[8];
#pragma unroll
        for (int f = 0; f < 8; ++f) {
            qv[f] = ldg4(qrow + 4 * f);
            cs[f] = ldg4(tab + 2 * (16 * half + 2 * f));
        }
        // Scaled first, then rotated with fused multiply-adds: q only enters
        // the scores, so it needs the reference's accuracy, not its bits (the
        // cache rows, which must match bit for bit, are rotated by the append
        // kernel), and the new wave does this with few vector issue slots.
#pragma unroll
        for (int f = 0; f < 8; ++f) {
            const float4 x = make_float4(qv[f].x * p.scale_log2, qv[f].y * p.scale_log2,
                                         qv[f].z * p.scale_log2, qv[f].w * p.scale_log2);
            qv[f] = p.rotate ? rotate4_fma(x, cs[f]) : x;
        }
    }

    floatx16 o0, o1;
#pragma unroll
    for (int i = 0; i < 16; ++i) { o0[i] = 0.f; o1[i] = 0.f; }
    float m_run = -INFINITY;
    float l_run = 0.f;

    // S^T = K.Q^T for the tile in K buffer b (K operand: lane holds
    // K[col][32*half + s]).  s[gi] = S[query col][key 8*(gi/4) + 4*half + gi%4].
    auto scores = [&](int b) {
        const float* krow = &sk[b][col][32 * half];
        floatx16 s;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = 0.f;
#pragma unroll
        for (int f = 0; f < 8; ++f) {
            const float4 kk = *reinterpret_cast<const float4*>(krow + 4 * f);
            s = mfma32(kk.x, qv[f].x, s);
            s = mfma32(kk.y, qv[f].y, s);
            s = mfma32(kk.z, qv[f].z, s);
            s = mfma32(kk.w, qv[f].w, s);
        }
        return s;
    };
    // Online softmax of one tile's scores (log2 units) into P, in place.
    auto softmax = [&](floatx16& s, int j0, bool masked) {
        if (masked) {
#pragma unroll
            for (int gi = 0; gi < 16; ++gi) {
                const int key = j0 + 8 * (gi >> 2) + 4 * half + (gi & 3);
                s[gi] = (key <= qpos && key <= last_key) ? s[gi] : -INFINITY;
            }
        }
        float mx = s[0];
#pragma unroll
        for (int gi = 1; gi < 16; ++gi) mx = fmaxf(mx, s[gi]);
        mx = max_xor32(mx);  // the other half of the keys
        // The running max only moves when some row's tile max exceeds it by
        // more than 2^8: probabilities then stay <= 256 and the sums in fp32
        // range, and most tiles skip the rescale of O.  The result is the
        // same softmax: O and l share whatever max they were scaled by.
        if (__any(mx > m_run + kRescaleSlack)) {
            const float m_new = fmaxf(m_run, mx);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first tile
            m_run = m_new;
            l_run *= alpha;
            o0 *= alpha;
            o1 *= alpha;
        }
        float lsum = 0.f;
#pragma unroll
        for (int gi = 0; gi < 16; ++gi) {
            s[gi] = __builtin_amdgcn_exp2f(s[gi] - m_run);
            lsum += s[gi];
        }
        l_run += lsum;
    };
    // O^T += V^T.P^T for the tile in V buffer b (V operand: lane holds
    // V[8*(gi/4) + 4*half + gi%4][2*col + dt]).  The operands come in four
    // groups of four gi, two groups in registers: the first two are read at
    // the top of the step (vread_head, before the next tile's scores and this
    // tile's softmax), each later one while the group before it is in the
    // MFMAs, so no MFMA pair waits on an LDS round trip.  The scheduling
    // barriers keep the compiler from sinking the reads to their uses.
    float2 vv[2][4];
    auto vread = [&](int b, int g, float2* dst) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            dst[i] = *reinterpret_cast<const float2*>(&sv[b][8 * g + 4 * half + i][2 * col]);
    };
    auto vread_head = [&](int b) {
        vread(b, 0, vv[0]);
        vread(b, 1, vv[1]);
        __builtin_amdgcn_sched_barrier(0);
    };
    auto accumulate = [&](const floatx16& s, int b) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                o0 = mfma32(vv[g & 1][i].x, s[4 * g + i], o0);
                o1 = mfma32(vv[g & 1][i].y, s[4 * g + i], o1);
            }
            if (g + 2 < 4) {
                vread(b, g + 2, vv[g & 1]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    // Software pipeline over key tiles j: step j computes the scores of tile
    // j+1 (MFMA) while the softmax of tile j (VALU) runs, then P.V of tile j.
    // At the start of step j the LDS holds K[j+1] and V[j]; the step stores
    // K[j+2] and V[j+1], loaded from global memory one step earlier, into the
    // buffers of K[j] and V[j-1], and issues the loads of K[j+3] and V[j+2].
    float4 ld_k[2], ld_v[2];
    gload(kc, 0, ld_k);
    gload(vc, 0, ld_v);
    lstore(sk[0], ld_k);
    lstore(sv[0], ld_v);
    gload(kc, 1, ld_k);
    gload(vc, 1, ld_v);
    lstore(sk[1], ld_k);
    gload(kc, 2, ld_k);
    __syncthreads();
    floatx16 s_cur;
    if (computes) s_cur = scores(0);
    __syncthreads();  // K[0]'s buffer is overwritten in step 0

    int j = 0;
    for (; j < n_plain; ++j) {
        if (computes) {
            vread_head(j & 1);
            const floatx16 s_next = scores((j + 1) & 1);
            softmax(s_cur, j * kKTile, false);
            accumulate(s_cur, j & 1);
            s_cur = s_next;
        }
        lstore(sk[j & 1], ld_k);
        lstore(sv[(j + 1) & 1], ld_v);
        gload(kc, j + 3, ld_k);
        gload(vc, j + 2, ld_v);
        __syncthreads();
    }
    for (; j < n_kt; ++j) {  // at most two tiles reach the diagonal
        const bool more = j + 1 < n_kt;  // uniform
        if (computes) {
            floatx16 s_next = {};  // unused after the last tile
            vread_head(j & 1);
            if (more) s_next = scores((j + 1) & 1);
            softmax(s_cur, j * kKTile, true);
            accumulate(s_cur, j & 1);
            s_cur = s_next;
        }
        if (more) {
            lstore(sk[j & 1], ld_k);
            lstore(sv[(j + 1) & 1], ld_v);
            gload(kc, j + 3, ld_k);
            gload(vc, j + 2, ld_v);
            __syncthreads();
        }
    }

    if (!computes) return;
    l_run = sum_xor32(l_run);
    if (i0 + col >= p.n_tok) return;
    const float inv = 1.0f / l_run;
    // o_dt[4a+b] = O[row][16a + 8*half + 2b + dt]
    float* orow = p.out + (((long long)lb * p.n_tok + i0 + col) * p.n_head + qh) * kHeadDim + 8 * half;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        stg4(orow + 16 * a, make_float4(o0[4 * a + 0] * inv, o1[4 * a + 0] * inv,
                                        o0[4 * a + 1] * inv, o1[4 * a + 1] * inv));
        stg4(orow + 16 * a + 4, make_float4(o0[4 * a + 2] * inv, o1[4 * a + 2] * inv,
                                            o0[4 * a + 3] * inv, o1[4 * a + 3] * inv));
    }
}

}  // namespace

hipError_t load_prefill_code()
{
    hipFuncAttributes a;
    return hipFuncGetAttributes(&a, reinterpret_cast<const void*>(&prefill_append_kernel));
}

hipError_t launch_prefill_append(const PrefillParams& p, hipStream_t s)
{
    const long long threads = (long long)p.n_lb * p.n_tok * p.n_head_kv * 16;
    const long long blocks = (threads + 255) / 256;
    hipLaunchKernelGGL(prefill_append_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_prefill_attention(const PrefillParams& p, hipStream_t s)
{
    PrefillGrid g;
    g.n_qt = (p.n_tok + kQTile - 1) / kQTile;
    g.n_hg = (p.gqa + kWavesP - 1) / kWavesP;
    g.n_pairs = p.n_lb * p.n_head_kv;
    g.per_xcd = (g.n_pairs + kXcds - 1) / kXcds * g.n_hg * g.n_qt;
    // m = ceil(2^32 / d) (0 for d <= 1); mulhi(n, m) = n / d whenever n * d < 2^32.
    auto magic = [](long long d) -> unsigned {
        return d <= 1 ? 0u : (unsigned)(((1ULL << 32) + (unsigned long long)d - 1) / (unsigned long long)d);
    };
    const long long rank_big = (long long)((g.n_pairs + kXcds - 1) / kXcds) * g.n_hg;
    const long long rank_small = (long long)(g.n_pairs / kXcds) * g.n_hg;
    if ((long long)g.per_xcd * rank_big >= (1LL << 32) || (long long)rank_big * g.n_hg >= (1LL << 32) ||
        (long long)g.n_pairs * p.n_head_kv >= (1LL << 32))
        return hipErrorInvalidValue;  // quotients by multiply-high would not be exact
    g.m_rank_big = magic(rank_big);
    g.m_rank_small = magic(rank_small);
    g.m_hg = magic(g.n_hg);
    g.m_kv = magic(p.n_head_kv);
    hipLaunchKernelGGL(prefill_attention_kernel, dim3(g.per_xcd * kXcds), dim3(64 * kWavesP), 0, s,
                       p, g);
    return hipGetLastError();
}

}  // namespace tla
