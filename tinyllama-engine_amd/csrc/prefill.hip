// Causal prefill attention for gfx950: products on the bf16 matrix cores
// with fp32 accuracy, fp32 accumulation.
//
// Reference semantics: the prompt is fed token by token (src/generate.cpp:
// 56-59); for the attention block that is, for t = 0..n_tok-1 at position
// P = pos0 + t: rope(q_t, k_t, P) (src/ops.cpp:1223-1281), append k_t,v_t at
// P (src/ops.cpp:1370-1371), then attention of q_t over cache positions
// 0..P (src/ops.cpp:1377-1511).  Because token t only ever sees keys
// 0..P, the whole prompt is one causal (lower-triangular) attention over
// the cache after all appends -- which is what these kernels compute.
//
// Exact splitting.  Every fp32 operand (q, k, v and the probabilities P) is
// the sum of three bf16 pieces, x = x0 + x1 + x2 (bf16_split.h); a product
// of two pieces is exact in fp32, so a . b is computed as the six piece
// products down to 2^-16 of a b (a0b0, a0b1, a1b0, a0b2, a1b1, a2b0) on
// v_mfma_f32_32x32x16_bf16, whose rate is 16 times that of fp32 MFMA.  The
// three left out are below 2^-24 of a b: the reference's accuracy, not its
// bits.
//
// prefill_append_kernel: one workgroup per (layer, kv head, 32-key tile):
//   rotates the prompt's k rows (when asked) and writes k and v rows to the
//   cache, bit-exact with the reference's append, and writes every key of
//   the tile (earlier ones read back from the cache) as K and V planes in
//   the layout the attention kernel's MFMA operands are read in.
//
// prefill_attention_kernel: one workgroup = 4 waves = 4 q heads of one kv
//   head, over one tile of 32 query tokens.  Each wave:
//     S^T[32 keys][32 queries] = K[32][64] . Q^T[64][32]   24 MFMAs
//     causal mask, online softmax per query row (the running max moves
//       only when it grows by more than 2^8, so most tiles skip rescaling O)
//     O^T[64 d][32 queries]   += V^T[64][32] . P^T[32][32] 24 MFMAs
//   The S accumulator layout is the B operand of the P.V product as is (K
//   rows are stored permuted, kperm), so P never leaves registers.  Q
//   (rotated in registers with the host-built table) is split once.  Tiles
//   come from the planes into LDS with direct global-to-LDS loads.
//
// Scheduling: key/value tiles of one (layer, kv head) are read by all its
//   query tiles and q heads, so those workgroups are placed on one XCD
//   (workgroup i runs on XCD i % 8) to share that XCD's L2, and each XCD
//   starts the query tiles with the most key tiles first, across all of its
//   (layer, kv head) pairs, so the last workgroups to start are short ones.
#include "bf16_split.h"
#include "lane_math.h"
#include "rope_math.h"
#include "tla_internal.h"

namespace tla {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kQTile = 32;
constexpr int kKTile = 32;
constexpr int kWavesP = 4;
constexpr int kXcds = 8;

// Planes of one 32-key tile, K then V, three bf16 planes each, each plane
// in the order the attention kernel's waves read it as an MFMA operand
// (1 KiB per read, lane l at byte 16 l):
//   K plane: byte 512 c + 16 i = dims 8c .. 8c+7 of key kperm(i);
//   V plane: byte 2048 dt + 1024 s + 512 h + 16 i = keys 16s + 8h .. +7
//            of dim 2i + dt.
constexpr int kPlane = kKTile * kHeadDim * 2;  // bytes of one bf16 plane of a tile
constexpr int kHalfTile = 3 * kPlane;          // K (or V) of a tile: 12 KiB
constexpr int kTileBytes = 2 * kHalfTile;

// Row i of a K tile holds key kperm(i) of the tile (bits 2 and 3 of the
// index swapped; its own inverse).  Score register r of lane 32 h + j then
// holds key 16 (r / 8) + 8 h + r % 8 for query j, which is what lane 32 h +
// j supplies as the B operand (P^T) of the P.V product at k step r / 8,
// element r % 8.
__device__ __forceinline__ int kperm(int i)
{
    return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1);
}

// The three planes of eight fp32 values.
__device__ __forceinline__ void split8(floatx8 v, bf16x8 (&o)[3])
{
    split3x8(v, o[0], o[1], o[2]);
}

// One workgroup per (layer, kv head, 32-key tile) of positions 0 ..
// pos0+n_tok-1, tile fastest.  Keys from pos0 on are the prompt's; earlier
// keys are read from the cache; keys past the last position are zeros.
//   K: thread t holds dims 8c .. 8c+7 of key kk (c = t / 32, kk = t % 32);
//   V: thread t holds dim d of keys 8kg .. 8kg+7 (kg = t / 64, d = 2 (t % 32)
//      + (t / 32) % 2), so each of its plane pieces is one 16-byte store and
//      each wave's cache store instruction one 256-byte key row.
__global__ __launch_bounds__(256) void prefill_append_kernel(const PrefillParams p)
{
    const int tile = (int)(blockIdx.x % (unsigned)p.n_ptiles);
    const int pair = (int)(blockIdx.x / (unsigned)p.n_ptiles);  // lb * n_head_kv + kvh
    const int kvh = pair % p.n_head_kv, lb = pair / p.n_head_kv;
    const int n_pos = p.pos0 + p.n_tok;
    const int kv_dim = p.n_head_kv * kHeadDim;
    const long long layer_off = (long long)(p.layer0 + lb) * p.layer_stride + (long long)kvh * kHeadDim;
    float* const kc = p.kc + layer_off;
    float* const vc = p.vc + layer_off;
    unsigned char* const planes = p.kvp + ((long long)pair * p.n_ptiles + tile) * kTileBytes;

    // Every load is issued before the first store (one memory round trip).
    const int kk = threadIdx.x & 31, c = threadIdx.x >> 5;
    const int kkey = tile * kKTile + kk;
    const bool k_new = kkey >= p.pos0 && kkey < n_pos;
    float* const kdst = kc + (long long)kkey * kv_dim + 8 * c;
    float4 ka = make_float4(0.f, 0.f, 0.f, 0.f), kb = ka, ca = ka, cb = ka;
    if (k_new) {
        const float* src = p.k + (((long long)lb * p.n_tok + (kkey - p.pos0)) * p.n_head_kv + kvh) * kHeadDim + 8 * c;
        const float* tab = reinterpret_cast<const float*>(p.rope + (long long)kkey * kPairs) + 8 * c;
        ka = ldg4(src);
        kb = ldg4(src + 4);
        ca = ldg4(tab);
        cb = ldg4(tab + 4);
    } else if (kkey < n_pos) {
        ka = ldg4(kdst);
        kb = ldg4(kdst + 4);
    }
    const int kg = threadIdx.x >> 6, d = 2 * (threadIdx.x & 31) + ((threadIdx.x >> 5) & 1);
    floatx8 vx;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int key = tile * kKTile + 8 * kg + e;
        float val = 0.f;
        if (key >= p.pos0 && key < n_pos)
            val = p.v[(((long long)lb * p.n_tok + (key - p.pos0)) * p.n_head_kv + kvh) * kHeadDim + d];
        else if (key < n_pos)
            val = vc[(long long)key * kv_dim + d];
        vx[e] = val;
    }

    if (k_new) {
        if (p.rotate) {
            ka = rotate4(ka, ca);
            kb = rotate4(kb, cb);
        }
        stg4(kdst, ka);
        stg4(kdst + 4, kb);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int key = tile * kKTile + 8 * kg + e;
        if (key >= p.pos0 && key < n_pos) vc[(long long)key * kv_dim + d] = vx[e];
    }
    bf16x8 pc[3];
    split8(floatx8{ka.x, ka.y, ka.z, ka.w, kb.x, kb.y, kb.z, kb.w}, pc);
#pragma unroll
    for (int q = 0; q < 3; ++q) *reinterpret_cast<bf16x8*>(planes + q * kPlane + 512 * c + 16 * kperm(kk)) = pc[q];
    split8(vx, pc);
#pragma unroll
    for (int q = 0; q < 3; ++q)
        *reinterpret_cast<bf16x8*>(planes + kHalfTile + q * kPlane + 2048 * (d & 1) + 1024 * (kg >> 1) +
                                   512 * (kg & 1) + 16 * (d >> 1)) = pc[q];
}

struct PrefillGrid {
    int n_qt;     // query tiles
    int n_hg;     // head groups of 4 waves per kv head
    int n_pairs;  // n_lb * n_head_kv
    // Pair groups: 8 (pair i on XCD i % 8) for at least 8 pairs, else 1 (all
    // query tiles over the whole GPU: one layer has 4 pairs).
    int n_grp, grp_shift;  // n_grp = 1 << grp_shift
    int per_grp;           // workgroup slots per group: ceil(n_pairs / n_grp) * n_hg * n_qt
    // Quotients by the launch's divisors as multiply-highs: q = mulhi(n, m)
    // with m = ceil(2^32 / d), exact for n * d < 2^32 (checked at launch); a
    // divisor of 1 has m = 0 and takes q = n.  The groups below
    // n_pairs % n_grp (all when it is 0) hold ceil(n_pairs / n_grp) pairs,
    // the others one fewer.
    unsigned m_rank_big, m_rank_small;  // pairs per group x n_hg
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

// Products of two split operands on v_mfma_f32_32x32x16_bf16: a . b for
// a = a0 + a1 + a2 and b = b0 + b1 + b2, the six piece products down to
// 2^-16 of a b, smallest first.
__device__ __forceinline__ floatx16 split_products(const bf16x8 (&a)[3], const bf16x8 (&b)[3], floatx16 c)
{
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], c, 0, 0, 0);
    return c;
}

typedef __attribute__((address_space(3))) void* lds_ptr;
typedef __attribute__((address_space(1))) void* global_ptr;

// Copies half a tile (12 KiB, K or V) from the planes into LDS: 12 chunks
// of 1 KiB over kWaves waves, each one direct global-to-LDS load of 16
// bytes per lane (lane l's bytes land at byte 16 l of the chunk).
template <int kWaves>
__device__ __forceinline__ void copy_half(const unsigned char* src, unsigned char* dst, int wave, int lane)
{
    constexpr int kPer = 12 / kWaves;
#pragma unroll
    for (int c = 0; c < kPer; ++c) {
        const int chunk = kPer * wave + c;
        __builtin_amdgcn_global_load_lds((global_ptr)(src + 1024 * chunk + 16 * lane), (lds_ptr)(dst + 1024 * chunk),
                                         16, 0, 0);
    }
}

// kKS key splits: the workgroup's 4 waves are 4 / kKS q heads x kKS key
// splits; split h walks key tiles h, h + kKS, ... with its own double
// buffers, and the splits' softmax states are merged in LDS at the end.
// kKS = 2 halves the longest query tile's walk for grids that do not fill
// the GPU (one layer per launch, as the batched prompt makes them).
template <int kKS>
__global__ __launch_bounds__(64 * kWavesP) __attribute__((amdgpu_waves_per_eu(3, 3))) void
prefill_attention_kernel(const PrefillParams p, const PrefillGrid g)
{
    constexpr int kHeads = kWavesP / kKS;  // q heads per workgroup
    // K and V tiles (three bf16 planes each, the planes' layout) per key
    // split, shared by its waves, double-buffered.  (Three buffers per split,
    // the copies two steps ahead, measured slower for kKS = 2: 144 KiB of
    // LDS, one workgroup per CU.)
    constexpr int kNB = 2;
    __shared__ __align__(16) unsigned char sk[kKS][kNB][kHalfTile];
    __shared__ __align__(16) unsigned char sv[kKS][kNB][kHalfTile];

    // ---- XCD-aware, heavy-first mapping of workgroups to tiles ----
    // Workgroup b runs on XCD b % 8 and XCDs start their workgroups in order
    // of b / 8.  With 8 groups, (layer, kv head) pair i belongs to XCD i % 8,
    // so all query tiles of a pair share one L2; within an XCD, query tiles
    // are handed out longest first (most key tiles) across all its pairs.
    // With one group (fewer than 8 pairs: their tiles fit every L2) the same
    // order runs over the whole GPU.
    // The quotients are multiply-highs on scalar registers: a workgroup that
    // starts beside MFMA-bound waves gets few vector issue slots, and the
    // compiler's divisions go through the vector unit.
    const int grp = blockIdx.x & (g.n_grp - 1);
    const int slot = blockIdx.x >> g.grp_shift;
    const int grp_pairs = (g.n_pairs - grp + g.n_grp - 1) >> g.grp_shift;
    const bool big = (grp_pairs << g.grp_shift) >= g.n_pairs;  // this group holds ceil(n_pairs / n_grp) pairs
    const int per_rank = grp_pairs * g.n_hg;
    if (slot >= per_rank * g.n_qt) return;  // whole workgroup
    const int rank = (int)div_magic((unsigned)slot, big ? g.m_rank_big : g.m_rank_small);
    const int qt = g.n_qt - 1 - rank;
    const int rem = slot - rank * per_rank;
    const int pg = (int)div_magic((unsigned)rem, g.m_hg);
    const int pair = grp + (pg << g.grp_shift);  // (lb, kvh)
    const int hg = rem - pg * g.n_hg;
    const int lb = (int)div_magic((unsigned)pair, g.m_kv);
    const int kvh = pair - lb * p.n_head_kv;

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // scalar
    const int lane = threadIdx.x & 63;
    const int kh = wave / kHeads, hw = wave % kHeads;  // key split, head within the workgroup
    const int hq = hg * kHeads + hw;
    const bool computes = hq < p.gqa;  // uniform per wave; others only copy tiles
    const int qh = kvh * p.gqa + (computes ? hq : 0);

    const int col = lane & 31;  // query row within the tile
    const int half = lane >> 5; // which 8 of each 16 dims (Q, K) / keys (P, V)
    const int i0 = qt * kQTile;
    const int trow = min(i0 + col, p.n_tok - 1);  // clamped token index
    const int qpos = p.pos0 + i0 + col;           // this row's position
    const int last_key = p.pos0 + min(i0 + kQTile - 1, p.n_tok - 1);
    const int n_kt = last_key / kKTile + 1;  // key tiles covering 0..last_key
    // Tiles below (pos0 + i0 + 1) / 32 end at or before the tile's first query
    // position: no key in them is masked for any row.
    const int n_plain = min((p.pos0 + i0 + 1) / kKTile, n_kt - 1);

    // The pair's tiles in the planes (tile j's K at tiles + j kTileBytes, its
    // V kHalfTile further).  Past the last tile nothing is copied.
    const unsigned char* const tiles = p.kvp + ((long long)lb * p.n_head_kv + kvh) * p.n_ptiles * kTileBytes;
    // Past the last tile the last one is copied again (never read), so that
    // every step issues the same copies and the waits can count them.
    auto copy_k = [&](int j, int b) {
        copy_half<kHeads>(tiles + (long long)min(j, n_kt - 1) * kTileBytes, sk[kh][b], hw, lane);
    };
    auto copy_v = [&](int j, int b) {
        copy_half<kHeads>(tiles + (long long)min(j, n_kt - 1) * kTileBytes + kHalfTile, sv[kh][b], hw, lane);
    };

    // ---- Q^T operand: lane 32 h + j holds, for k step s, dims 16s + 8h ..
    // +7 of query j, times scale * log2(e), as three bf16 planes ----
    bf16x8 qp[4][3];
    {
        const float* qrow = p.q + (((long long)lb * p.n_tok + trow) * p.n_head + qh) * kHeadDim + 8 * half;
        const float* tab = reinterpret_cast<const float*>(p.rope + (long long)(p.pos0 + trow) * kPairs) + 8 * half;
        // All sixteen loads are issued before any is used.
        float4 qv[8], cs[8];
#pragma unroll
        for (int f = 0; f < 8; ++f) {
            qv[f] = ldg4(qrow + 16 * (f >> 1) + 4 * (f & 1));
            cs[f] = ldg4(tab + 16 * (f >> 1) + 4 * (f & 1));  // (cos, sin) pairs of those dims
        }
        // Scaled first, then rotated with fused multiply-adds: q only enters
        // the scores, so it needs the reference's accuracy, not its bits (the
        // cache rows, which must match bit for bit, are rotated by the append
        // kernel).
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            floatx8 v;
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const float4 x0 = qv[2 * s + h2];
                const float4 x = make_float4(x0.x * p.scale_log2, x0.y * p.scale_log2, x0.z * p.scale_log2,
                                             x0.w * p.scale_log2);
                const float4 r = p.rotate ? rotate4_fma(x, cs[2 * s + h2]) : x;
                v[4 * h2 + 0] = r.x;
                v[4 * h2 + 1] = r.y;
                v[4 * h2 + 2] = r.z;
                v[4 * h2 + 3] = r.w;
            }
            split8(v, qp[s]);
        }
    }

    floatx16 o0 = {}, o1 = {};
    float m_run = -INFINITY;
    float l_run = 0.f;

    // S^T = K.Q^T for the tile in K buffer kb: s[r] = S[query col][key
    // 16 (r / 8) + 8 half + r % 8 of the tile].
    auto scores = [&](const unsigned char* kb) {
        floatx16 s = {};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            bf16x8 a[3];
#pragma unroll
            for (int q = 0; q < 3; ++q) a[q] = *reinterpret_cast<const bf16x8*>(kb + q * kPlane + 1024 * ks + 16 * lane);
            s = split_products(a, qp[ks], s);
        }
        return s;
    };
    // Online softmax of one tile's scores (log2 units) into P, in place.
    auto softmax = [&](floatx16& s, int j0, bool masked) {
        if (masked) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = j0 + 16 * (r >> 3) + 8 * half + (r & 7);
                s[r] = (key <= qpos && key <= last_key) ? s[r] : -INFINITY;
            }
        }
        float mx = s[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
        mx = max_xor32(mx);  // the other half of the keys
        // The running max only moves when some row's tile max exceeds it by
        // more than 2^8: probabilities then stay <= 256 and the sums in fp32
        // range, and most tiles skip the rescale of O.  The result is the
        // same softmax: O and l share whatever max they were scaled by.
        // A row whose keys have all been masked so far keeps m_run = -inf
        // (a key split's first tile can lie past some rows' positions): its
        // probabilities are 0, and nothing is rescaled.
        if (__any(mx > m_run + kRescaleSlack)) {
            const float m_new = fmaxf(m_run, mx);
            const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first tile
            m_run = m_new;
            l_run *= alpha;
            o0 *= alpha;
            o1 *= alpha;
        }
        const float m_use = m_run == -INFINITY ? 0.f : m_run;
        float lsum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s[r] = __builtin_amdgcn_exp2f(s[r] - m_use);
            lsum += s[r];
        }
        l_run += lsum;
    };
    // O^T += V^T.P^T for the tile in V buffer vb: o_dt[r] accumulates dim
    // 2 (8 (r / 4) + 4 half + r % 4) + dt of query col.  P^T at k step ks is
    // s[8 ks .. 8 ks + 7], split into planes just before its products.
    auto accumulate = [&](const floatx16& s, const unsigned char* vb) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            floatx8 pv;
#pragma unroll
            for (int e = 0; e < 8; ++e) pv[e] = s[8 * ks + e];
            bf16x8 pp[3];
            split8(pv, pp);
            bf16x8 a0[3], a1[3];
#pragma unroll
            for (int q = 0; q < 3; ++q) {
                a0[q] = *reinterpret_cast<const bf16x8*>(vb + q * kPlane + 1024 * ks + 16 * lane);
                a1[q] = *reinterpret_cast<const bf16x8*>(vb + q * kPlane + 2048 + 1024 * ks + 16 * lane);
            }
            o0 = split_products(a0, pp, o0);
            o1 = split_products(a1, pp, o1);
        }
    };

    // Software pipeline over this split's key tiles j_m = kh + m kKS: step m
    // computes the scores of tile j_{m+1} (MFMA) while the softmax of tile
    // j_m (VALU) runs, then P.V of tile j_m.  Tile j_m's K and V sit in
    // buffer m % kNB.  Step m copies K[j_{m+kNB}] and V[j_{m+kNB-1}] into the
    // buffers of K[j_m] and V[j_{m-1}] (both read in step m - 1), and before
    // the barrier that ends it waits for the copies step m + 1 reads, issued
    // kNB - 2 steps earlier: the copies of the last kNB - 2 steps may stay in
    // flight.  Every split runs the same number of steps (barriers); a split
    // past its last tile only copies and waits.
    constexpr int kCopies = 2 * (12 / kHeads);  // copy instructions per wave and step
    constexpr int kInFlight = (kNB - 2) * kCopies;
    static_assert(kInFlight < 64, "vmcnt holds 6 bits");
    constexpr int kWaitCopies = (kInFlight & 15) | ((kInFlight >> 4) << 14) | 0xF70;  // vmcnt(kInFlight)
    const int n_steps = (n_kt + kKS - 1) / kKS;
    auto tile_of = [&](int m) { return kh + m * kKS; };
#pragma unroll
    for (int b = 0; b < kNB; ++b) copy_k(tile_of(b), b);
#pragma unroll
    for (int b = 0; b + 1 < kNB; ++b) copy_v(tile_of(b), b);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    floatx16 s_cur = {};
    if (computes && tile_of(0) < n_kt) s_cur = scores(sk[kh][0]);
    __syncthreads();  // K[j_0]'s buffer is refilled in step 0

    // The scores of tile j_m in s_this, tile j_{m+1}'s into s_next.  Two
    // steps per loop trip, the two accumulators trading roles, so that no
    // copy of the scores is needed between steps.  Only the last one or two
    // tiles reach the diagonal (masked).
    auto step = [&](int m, floatx16& s_this, floatx16& s_next) {
        const int j = tile_of(m), jn = tile_of(m + 1);
        const bool last = m + 1 == n_steps;  // uniform
        copy_k(tile_of(m + kNB), m % kNB);
        copy_v(tile_of(m + kNB - 1), (m + kNB - 1) % kNB);
        if (computes && j < n_kt) {
            if (jn < n_kt) s_next = scores(sk[kh][(m + 1) % kNB]);
            softmax(s_this, j * kKTile, j >= n_plain);
            accumulate(s_this, sv[kh][m % kNB]);
        }
        if (!last) {
            // A bare barrier: __syncthreads' release fence would wait for
            // every copy in flight (they write LDS through the vector memory
            // path).  This step's LDS reads were used before this point.
            __builtin_amdgcn_s_waitcnt(kWaitCopies);
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        }
    };
    floatx16 s_alt = {};
    int m = 0;
    for (; m + 1 < n_steps; m += 2) {
        step(m, s_cur, s_alt);
        step(m + 1, s_alt, s_cur);
    }
    if (m < n_steps) step(m, s_cur, s_alt);
    __builtin_amdgcn_s_waitcnt(0);  // the copies past the end land before the LDS is reused or released

    if constexpr (kKS == 2) {
        // Split 1 hands its softmax state (running max, partial sum, O) to
        // split 0 through LDS (the tile buffers, free now); split 0 merges:
        // both scaled to the larger max.  Split 0 always had a tile.
        __syncthreads();
        float* const xch = reinterpret_cast<float*>(&sk[0][0][0]) + hw * 34 * 64 + lane;
        if (kh == 1 && computes) {
            xch[0] = m_run;
            xch[64] = l_run;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                xch[64 * (2 + i)] = o0[i];
                xch[64 * (18 + i)] = o1[i];
            }
        }
        __syncthreads();
        if (kh == 1) return;
        if (computes) {
            const float m_b = xch[0];
            const float m_new = fmaxf(m_run, m_b);
            const float fa = __builtin_amdgcn_exp2f(m_run - m_new), fb = __builtin_amdgcn_exp2f(m_b - m_new);
            l_run = l_run * fa + xch[64] * fb;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                o0[i] = o0[i] * fa + xch[64 * (2 + i)] * fb;
                o1[i] = o1[i] * fa + xch[64 * (18 + i)] * fb;
            }
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

size_t prefill_planes_bytes(int n_lb, int n_head_kv, int pos0, int n_tok)
{
    const long long tiles = ((long long)pos0 + n_tok + kKTile - 1) / kKTile;
    return (size_t)n_lb * n_head_kv * tiles * kTileBytes;
}

hipError_t load_prefill_code()
{
    hipFuncAttributes a;
    return hipFuncGetAttributes(&a, reinterpret_cast<const void*>(&prefill_append_kernel));
}

hipError_t launch_prefill_append(const PrefillParams& p, hipStream_t s)
{
    if (!p.kvp || p.n_ptiles != (p.pos0 + p.n_tok + kKTile - 1) / kKTile) return hipErrorInvalidValue;
    const long long blocks = (long long)p.n_lb * p.n_head_kv * p.n_ptiles;
    if (blocks >= (1LL << 31)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(prefill_append_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p);
    return hipGetLastError();
}

namespace {

// Compute units of the current device (cached per device).
int device_cus()
{
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

template <int kKS>
hipError_t launch_attention(const PrefillParams& p, hipStream_t s)
{
    constexpr int kHeads = kWavesP / kKS;
    PrefillGrid g;
    g.n_qt = (p.n_tok + kQTile - 1) / kQTile;
    g.n_hg = (p.gqa + kHeads - 1) / kHeads;
    g.n_pairs = p.n_lb * p.n_head_kv;
    g.n_grp = g.n_pairs >= kXcds ? kXcds : 1;
    g.grp_shift = g.n_grp == kXcds ? 3 : 0;
    static_assert(kXcds == 8, "grp_shift");
    g.per_grp = (g.n_pairs + g.n_grp - 1) / g.n_grp * g.n_hg * g.n_qt;
    // m = ceil(2^32 / d) (0 for d <= 1); mulhi(n, m) = n / d whenever n * d < 2^32.
    auto magic = [](long long d) -> unsigned {
        return d <= 1 ? 0u : (unsigned)(((1ULL << 32) + (unsigned long long)d - 1) / (unsigned long long)d);
    };
    const long long rank_big = (long long)((g.n_pairs + g.n_grp - 1) / g.n_grp) * g.n_hg;
    const long long rank_small = (long long)(g.n_pairs / g.n_grp) * g.n_hg;
    if ((long long)g.per_grp * rank_big >= (1LL << 32) || (long long)rank_big * g.n_hg >= (1LL << 32) ||
        (long long)g.n_pairs * p.n_head_kv >= (1LL << 32))
        return hipErrorInvalidValue;  // quotients by multiply-high would not be exact
    g.m_rank_big = magic(rank_big);
    g.m_rank_small = magic(rank_small);
    g.m_hg = magic(g.n_hg);
    g.m_kv = magic(p.n_head_kv);
    hipLaunchKernelGGL((prefill_attention_kernel<kKS>), dim3(g.per_grp * g.n_grp), dim3(64 * kWavesP), 0, s, p, g);
    return hipGetLastError();
}

}  // namespace

// Two key splits per workgroup where one split per workgroup would give at
// most one workgroup per CU (one layer per launch up to 1024 tokens: 512
// tokens 128 workgroups), else one.  (At 2048 tokens, 512 workgroups of one
// split run faster than 1024 of two.)
hipError_t launch_prefill_attention(const PrefillParams& p, hipStream_t s)
{
    if (!p.kvp || p.n_ptiles != (p.pos0 + p.n_tok + kKTile - 1) / kKTile) return hipErrorInvalidValue;
    const long long pairs = (long long)p.n_lb * p.n_head_kv;
    const long long wg1 = pairs * ((p.gqa + kWavesP - 1) / kWavesP) * ((p.n_tok + kQTile - 1) / kQTile);
    return wg1 <= device_cus() ? launch_attention<2>(p, s) : launch_attention<1>(p, s);
}

}  // namespace tla
