// Split-KV (flash-decoding) GQA decode attention for gfx950.
//
// Semantics follow attention() (src/ops.cpp:1317-1515): append the new k,v
// at `pos` (src/ops.cpp:1350-1371), then for every q head qh, with kv head
// qh / gqa (src/ops.cpp:1329, 1383): scores q.K[p] / sqrt(64) for p in 0..pos,
// softmax, and the weighted sum of V.  With `rotate`, RoPE is applied first
// to q and to the new k, as forward() does (src/forward.cpp:192-196).
//
// Work decomposition.  A "unit" is one (sequence, layer).  Its positions
// 0..pos are cut into splits of split_len positions.  One workgroup = one
// (unit, split) and holds 4 waves, one per kv head, so a workgroup streams
// whole 1 KiB position rows of K and of V.  Each wave keeps the gqa (= 8)
// q heads of its kv head in registers and walks its split in tiles of 16
// positions:
//
//   S^T[16 pos][16 heads] = K[16 pos][64] . Q^T[64][16 heads]
//                           16 x v_mfma_f32_16x16x4f32, heads 8..15 zero
//   online softmax per head (running max in log2 units, running sum)
//   O^T[64 d][16 heads]  += V^T[64 d][16 pos] . P^T[16 pos][16 heads]
//                           16 x v_mfma_f32_16x16x4f32
//
// The MFMA operand layouts are chosen so that nothing is transposed:
// the S accumulator (lane l holds S[pos = 4*(l/16)+r][head = l%16], r=0..3)
// is directly the B operand of the P.V products, and K and V are loaded
// from HBM straight into A-operand registers with 16-byte loads.  Each
// lane loads 64 B of a K row and 4 x 16 B of V rows per tile; a wave's
// loads cover 16 full 256 B head rows of K and of V.  No LDS is needed.
//
// The split that contains `pos` also appends the new token: it writes the
// (rotated) k row and the v row to the cache, and uses the same register
// values for position `pos` in its own tile, so it never reads back the
// row it has just written.
//
// With more than one split per unit, each split writes its unnormalised
// O, running max and sum to the workspace; decode_combine_kernel merges
// them with log-sum-exp weights.  A unit with one split writes `out`
// directly.
#include "rope_math.h"
#include "tla_internal.h"

namespace tla {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;  // waves per workgroup, one kv head each

__device__ __forceinline__ floatx4 mfma16(float a, float b, floatx4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__global__ __launch_bounds__(64 * kWaves) void decode_split_kernel(const DecodeParams p)
{
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int kvh = blockIdx.y * kWaves + wave;
    if (kvh >= p.n_head_kv) return;  // uniform per wave

    // blockIdx.x -> (layer step lb, sequence, split)
    const int lb = blockIdx.x / p.total_splits;
    const int rem = blockIdx.x - lb * p.total_splits;
    int lo = 0, hi = p.n_seq - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (p.split_prefix[mid] <= rem) lo = mid; else hi = mid - 1;
    }
    const int seq = lo;
    const int split = rem - p.split_prefix[seq];
    const int nsplit = p.split_prefix[seq + 1] - p.split_prefix[seq];
    const int pos = p.pos[seq];
    const int unit = seq * p.n_lb + lb;
    const int layer = p.layer0 + lb;

    const int begin = split * p.split_len;
    const int end = min(pos + 1, begin + p.split_len);  // exclusive, > begin
    const bool has_new = (pos >= begin) && (pos < end);  // this split appends

    const int kv_dim = p.n_head_kv * kHeadDim;
    const long long cache_off = (long long)seq * p.seq_stride + (long long)layer * p.layer_stride +
                                (long long)kvh * kHeadDim;
    float* kc = p.kc + cache_off;  // row r at kc + r * kv_dim
    float* vc = p.vc + cache_off;
    const float* knew = p.k + ((long long)unit * p.n_head_kv + kvh) * kHeadDim;
    const float* vnew = p.v + ((long long)unit * p.n_head_kv + kvh) * kHeadDim;

    const int hsub = lane & 15;  // q head within the group / K row within the tile
    const int grp = lane >> 4;   // 0..3

    // Dims held by this lane in the Q / K operands: d = 16*t + 4*grp + c.
    // Their rope pairs are 8*t + 2*grp + {0,1}: one float4 of the table per t.
    float4 cs_pos[4];
    if (p.rotate) {
        const float* tab = reinterpret_cast<const float*>(p.rope + (long long)pos * kPairs);
#pragma unroll
        for (int t = 0; t < 4; ++t) cs_pos[t] = ldg4(tab + 2 * (8 * t + 2 * grp));
    }

    // B operand of S^T: lane l holds q[head hsub][16t + 4grp + c].
    const bool head_ok = hsub < p.gqa;
    const int qh = kvh * p.gqa + hsub;
    float4 qv[4];
    {
        const float* qrow = p.q + ((long long)unit * p.n_head + (head_ok ? qh : 0)) * kHeadDim;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float4 x = ldg4(qrow + 16 * t + 4 * grp);
            if (p.rotate) x = rotate4(x, cs_pos[t]);
            qv[t] = head_ok ? x : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }

    // Append (attention() step 1, src/ops.cpp:1370-1371).
    if (has_new && lane < 16) {
        float4 kx = ldg4(knew + 4 * lane);
        if (p.rotate) {
            const float* tab = reinterpret_cast<const float*>(p.rope + (long long)pos * kPairs);
            kx = rotate4(kx, ldg4(tab + 4 * lane));
        }
        stg4(kc + (long long)pos * kv_dim + 4 * lane, kx);
        stg4(vc + (long long)pos * kv_dim + 4 * lane, ldg4(vnew + 4 * lane));
    }

    floatx4 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;
    float l_run = 0.f;

    for (int p0 = begin; p0 < end; p0 += kDecodeTile) {
        // ---- K tile: lane holds row p0 + hsub, dims 16t + 4grp + c ----
        float4 kv4[4];
        {
            int r = p0 + hsub;
            if (r >= end) r = begin;  // masked below; any valid row
            if (has_new && r == pos) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    float4 x = ldg4(knew + 16 * t + 4 * grp);
                    kv4[t] = p.rotate ? rotate4(x, cs_pos[t]) : x;
                }
            } else {
                const float* kr = kc + (long long)r * kv_dim + 4 * grp;
#pragma unroll
                for (int t = 0; t < 4; ++t) kv4[t] = ldg4(kr + 16 * t);
            }
        }
        // ---- V tile: register r holds row p0 + 4grp + r, dims 4hsub..+3 ----
        float4 vv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            int row = p0 + 4 * grp + r;
            if (row >= end) row = begin;
            const float* src = (has_new && row == pos) ? vnew : vc + (long long)row * kv_dim;
            vv[r] = ldg4(src + 4 * hsub);
        }

        // ---- S^T = K . Q^T ----
        floatx4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            s = mfma16(kv4[t].x, qv[t].x, s);
            s = mfma16(kv4[t].y, qv[t].y, s);
            s = mfma16(kv4[t].z, qv[t].z, s);
            s = mfma16(kv4[t].w, qv[t].w, s);
        }

        // ---- online softmax (per head = lane & 15) ----
        float sc[4];
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int kp = p0 + 4 * grp + r;
            sc[r] = (kp < end) ? s[r] * p.scale_log2 : -INFINITY;
            mx = fmaxf(mx, sc[r]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        float ps[4];
        float lsum = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            ps[r] = __builtin_amdgcn_exp2f(sc[r] - m_new);
            lsum += ps[r];
        }
        l_run = l_run * alpha + lsum;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] *= alpha;

        // ---- O^T += V^T . P^T ----
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            o[0] = mfma16(vv[r].x, ps[r], o[0]);
            o[1] = mfma16(vv[r].y, ps[r], o[1]);
            o[2] = mfma16(vv[r].z, ps[r], o[2]);
            o[3] = mfma16(vv[r].w, ps[r], o[3]);
        }
    }

    // Row sums: each lane group summed different positions of the same head.
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    if (!head_ok) return;

    // o[dt][i] = O[head hsub][d = 16*grp + 4*i + dt]
    if (nsplit == 1) {
        const float inv = 1.0f / l_run;
        float* orow = p.out + ((long long)unit * p.n_head + qh) * kHeadDim + 16 * grp;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            stg4(orow + 4 * i, make_float4(o[0][i] * inv, o[1][i] * inv, o[2][i] * inv, o[3][i] * inv));
    } else {
        const long long idx = ((long long)unit * p.n_head + qh) * p.max_splits + split;
        float* po = p.part_o + idx * kHeadDim + 16 * grp;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            stg4(po + 4 * i, make_float4(o[0][i], o[1][i], o[2][i], o[3][i]));
        if (grp == 0) p.part_ml[idx] = make_float2(m_run, l_run);
    }
}

// Merge split partials: out = sum_s O_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).
// One thread per (unit, q head, d); 4 heads per 256-thread block.
__global__ __launch_bounds__(256) void decode_combine_kernel(const DecodeParams p)
{
    const int heads_per_block = 4;
    const int hblocks = (p.n_head + heads_per_block - 1) / heads_per_block;
    const int unit = blockIdx.x / hblocks;
    const int qh = (blockIdx.x - unit * hblocks) * heads_per_block + (threadIdx.x >> 6);
    const int d = threadIdx.x & 63;
    if (qh >= p.n_head) return;
    const int seq = unit / p.n_lb;
    const int nsplit = p.split_prefix[seq + 1] - p.split_prefix[seq];
    if (nsplit <= 1) return;  // written by the split kernel
    const long long base = ((long long)unit * p.n_head + qh) * p.max_splits;
    float m = -INFINITY;
    for (int s = 0; s < nsplit; ++s) m = fmaxf(m, p.part_ml[base + s].x);
    float l = 0.f, acc = 0.f;
    for (int s = 0; s < nsplit; ++s) {
        const float2 ml = p.part_ml[base + s];
        const float w = __builtin_amdgcn_exp2f(ml.x - m);
        l += ml.y * w;
        acc += p.part_o[(base + s) * kHeadDim + d] * w;
    }
    p.out[((long long)unit * p.n_head + qh) * kHeadDim + d] = acc / l;
}

}  // namespace

hipError_t launch_decode(const DecodeParams& p, hipStream_t s)
{
    dim3 grid(p.total_splits * p.n_lb, (p.n_head_kv + kWaves - 1) / kWaves);
    hipLaunchKernelGGL(decode_split_kernel, grid, dim3(64 * kWaves), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_decode_combine(const DecodeParams& p, hipStream_t s)
{
    const int hblocks = (p.n_head + 3) / 4;
    dim3 grid(p.n_seq * p.n_lb * hblocks);
    hipLaunchKernelGGL(decode_combine_kernel, grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

}  // namespace tla
