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
// The next tile's loads are issued before the current tile is computed.
//
// The split that contains `pos` also appends the new token: it writes the
// (rotated) k row and the v row to the cache, and uses the same register
// values for position `pos` in its own tile, so it never reads back the
// row it has just written.
//
// Merge.  With one split, the wave writes `out` directly.  With several,
// each split writes its unnormalised O and (running max, sum) to the
// workspace, then bumps the unit's arrival counter; the workgroup that
// arrives last merges all splits of the unit with log-sum-exp weights and
// resets the counter to zero for the next launch.  One launch per step.
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

// Split partials cross workgroups (and XCDs, each with its own L2) inside one
// launch.  They are stored and loaded with agent-scope relaxed atomics, which
// go to the device-coherent level instead of a non-coherent L2 copy, so no
// cache-wide writeback/invalidate (what an agent-scope fence costs) is needed.
__device__ __forceinline__ void st_dev(float* p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float ld_dev(const float* p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float4 ld_dev4(const float* p)
{
    return make_float4(ld_dev(p), ld_dev(p + 1), ld_dev(p + 2), ld_dev(p + 3));
}

struct Tile {
    float4 k[4];  // K row (p0 + hsub), dims 16t + 4grp + c
    float4 v[4];  // V row (p0 + 4grp + r), dims 4hsub + c
};

// Merge the n_split partials of one unit: out = sum_s O_s w_s / sum_s l_s w_s
// with w_s = 2^(m_s - max m).  256 threads: thread -> (head, 8-float chunk).
// Splits are merged online in chunks of 8 whose loads are all issued before
// any is used, so a unit costs one memory round trip per 8 splits.
__device__ void merge_unit(const DecodeParams& p, int unit, int nsplit)
{
    constexpr int kChunk = 8;
    const int c = threadIdx.x & 7;
    for (int h = threadIdx.x >> 3; h < p.n_head; h += 32) {
        const long long base = ((long long)unit * p.n_head + h) * p.max_splits;
        float m = -INFINITY, l = 0.f;
        float4 a0 = make_float4(0.f, 0.f, 0.f, 0.f), a1 = a0;
        for (int s0 = 0; s0 < nsplit; s0 += kChunk) {
            float2 ml[kChunk];
            float4 x0[kChunk], x1[kChunk];
#pragma unroll
            for (int j = 0; j < kChunk; ++j) {
                if (s0 + j < nsplit) {
                    const float* mlp = reinterpret_cast<const float*>(p.part_ml + base + s0 + j);
                    ml[j] = make_float2(ld_dev(mlp), ld_dev(mlp + 1));
                    const float* src = p.part_o + (base + s0 + j) * kHeadDim + 8 * c;
                    x0[j] = ld_dev4(src);
                    x1[j] = ld_dev4(src + 4);
                } else {
                    ml[j] = make_float2(-INFINITY, 0.f);
                    x0[j] = x1[j] = make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
            float mc = m;
#pragma unroll
            for (int j = 0; j < kChunk; ++j) mc = fmaxf(mc, ml[j].x);
            const float r = __builtin_amdgcn_exp2f(m - mc);  // 0 on the first chunk
            m = mc;
            l *= r;
            a0.x *= r; a0.y *= r; a0.z *= r; a0.w *= r;
            a1.x *= r; a1.y *= r; a1.z *= r; a1.w *= r;
#pragma unroll
            for (int j = 0; j < kChunk; ++j) {
                const float w = __builtin_amdgcn_exp2f(ml[j].x - m);
                l += ml[j].y * w;
                a0.x += x0[j].x * w; a0.y += x0[j].y * w; a0.z += x0[j].z * w; a0.w += x0[j].w * w;
                a1.x += x1[j].x * w; a1.y += x1[j].y * w; a1.z += x1[j].z * w; a1.w += x1[j].w * w;
            }
        }
        const float inv = 1.0f / l;
        float* dst = p.out + ((long long)unit * p.n_head + h) * kHeadDim + 8 * c;
        stg4(dst, make_float4(a0.x * inv, a0.y * inv, a0.z * inv, a0.w * inv));
        stg4(dst + 4, make_float4(a1.x * inv, a1.y * inv, a1.z * inv, a1.w * inv));
    }
}

__global__ __launch_bounds__(64 * kWaves) void decode_split_kernel(const DecodeParams p)
{
    __shared__ int s_last;
    __shared__ float4 s_new[kWaves][32];  // appended k row (16 float4) | v row (16 float4)
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int kvh = blockIdx.y * kWaves + wave;
    const bool active = kvh < p.n_head_kv;  // uniform per wave

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
    const bool has_new = (pos >= begin) && (pos < end);  // this split appends; pos = end-1

    const int hsub = lane & 15;  // q head within the group / K row within the tile
    const int grp = lane >> 4;   // 0..3
    const bool head_ok = hsub < p.gqa;
    const int qh = kvh * p.gqa + hsub;
    const unsigned kv_dim = (unsigned)p.n_head_kv * kHeadDim;

    // Cache slice of this (sequence, layer, kv head): row r at base + r*kv_dim.
    const long long cache_off = (long long)seq * p.seq_stride + (long long)layer * p.layer_stride +
                                (long long)(active ? kvh : 0) * kHeadDim;
    float* const kc = p.kc + cache_off;
    float* const vc = p.vc + cache_off;
    const float* const tab = reinterpret_cast<const float*>(p.rope + (long long)pos * kPairs);

    // Append (attention() step 1, src/ops.cpp:1370-1371): 16 lanes write the
    // (rotated) k row and the v row to the cache and keep a copy in LDS for
    // this split's last tile.
    if (active && has_new && lane < 16) {
        const long long row = ((long long)unit * p.n_head_kv + kvh) * kHeadDim + 4 * lane;
        float4 kx = ldg4(p.k + row);
        if (p.rotate) kx = rotate4(kx, ldg4(tab + 4 * lane));
        const float4 vx = ldg4(p.v + row);
        stg4(kc + (long long)pos * kv_dim + 4 * lane, kx);
        stg4(vc + (long long)pos * kv_dim + 4 * lane, vx);
        s_new[wave][lane] = kx;
        s_new[wave][16 + lane] = vx;
    }
    __syncthreads();

    floatx4 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;
    float l_run = 0.f;

    if (active) {
        // B operand of S^T: lane holds q[head hsub][16t + 4grp + c], rotated
        // with the pairs 8t + 2grp + {0,1} of the table row for `pos`.
        float4 qv[4];
        {
            const float* qrow = p.q + ((long long)unit * p.n_head + (head_ok ? qh : 0)) * kHeadDim;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                float4 x = ldg4(qrow + 16 * t + 4 * grp);
                if (p.rotate) x = rotate4(x, ldg4(tab + 2 * (8 * t + 2 * grp)));
                qv[t] = head_ok ? x : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }

        // Rows past `end` are masked; they load row `begin` (always valid).
        // Offsets are 32-bit (a unit's cache slice is < 4 GiB) from a
        // wave-uniform base.
        auto load_tile = [&](int p0, Tile& tl) {
            int r = p0 + hsub;
            if (r >= end) r = begin;
            const unsigned ko = (unsigned)r * kv_dim + 4u * grp;
#pragma unroll
            for (int t = 0; t < 4; ++t) tl.k[t] = ldg4(kc + ko + 16u * t);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int row = p0 + 4 * grp + i;
                if (row >= end) row = begin;
                tl.v[i] = ldg4(vc + ((unsigned)row * kv_dim + 4u * hsub));
            }
        };

        Tile cur;
        load_tile(begin, cur);
        for (int p0 = begin; p0 < end; p0 += kDecodeTile) {
            const bool more = p0 + kDecodeTile < end;  // uniform
            Tile nxt;
            if (more) load_tile(p0 + kDecodeTile, nxt);

            if (has_new && !more) {
                // Last tile of the appending split: position `pos` comes from
                // the row kept in LDS, not from the cache row just written.
                if (min(p0 + hsub, end - 1) == pos || (p0 + hsub >= end && begin == pos)) {
#pragma unroll
                    for (int t = 0; t < 4; ++t) cur.k[t] = s_new[wave][4 * t + grp];
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = p0 + 4 * grp + i;
                    if (row == pos || (row >= end && begin == pos)) cur.v[i] = s_new[wave][16 + hsub];
                }
            }

            // ---- S^T = K . Q^T ----
            floatx4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                s = mfma16(cur.k[t].x, qv[t].x, s);
                s = mfma16(cur.k[t].y, qv[t].y, s);
                s = mfma16(cur.k[t].z, qv[t].z, s);
                s = mfma16(cur.k[t].w, qv[t].w, s);
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
                o[0] = mfma16(cur.v[r].x, ps[r], o[0]);
                o[1] = mfma16(cur.v[r].y, ps[r], o[1]);
                o[2] = mfma16(cur.v[r].z, ps[r], o[2]);
                o[3] = mfma16(cur.v[r].w, ps[r], o[3]);
            }
            if (more) cur = nxt;
        }

        // Row sums: each lane group summed different positions of the same head.
        l_run += __shfl_xor(l_run, 16);
        l_run += __shfl_xor(l_run, 32);

        // o[dt][i] = O[head hsub][d = 16*grp + 4*i + dt]
        if (head_ok) {
            if (nsplit == 1) {
                const float inv = 1.0f / l_run;
                float* orow = p.out + ((long long)unit * p.n_head + qh) * kHeadDim + 16 * grp;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    stg4(orow + 4 * i,
                         make_float4(o[0][i] * inv, o[1][i] * inv, o[2][i] * inv, o[3][i] * inv));
            } else {
                const long long idx = ((long long)unit * p.n_head + qh) * p.max_splits + split;
                float* po = p.part_o + idx * kHeadDim + 16 * grp;
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int dt = 0; dt < 4; ++dt) st_dev(po + 4 * i + dt, o[dt][i]);
                if (grp == 0) {
                    float* mlp = reinterpret_cast<float*>(p.part_ml + idx);
                    st_dev(mlp, m_run);
                    st_dev(mlp + 1, l_run);
                }
            }
        }
    }

    if (nsplit == 1) return;  // uniform per workgroup
    // Wait until this wave's partial stores are acknowledged at device scope,
    // then count the split in; the workgroup that completes the count merges.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(p.counters + unit, 1, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT) == nsplit * (int)gridDim.y - 1;
    __syncthreads();
    if (!s_last) return;
    merge_unit(p, unit, nsplit);
    if (threadIdx.x == 0)
        __hip_atomic_store(p.counters + unit, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

hipError_t launch_decode(const DecodeParams& p, hipStream_t s)
{
    dim3 grid(p.total_splits * p.n_lb, (p.n_head_kv + kWaves - 1) / kWaves);
    hipLaunchKernelGGL(decode_split_kernel, grid, dim3(64 * kWaves), 0, s, p);
    return hipGetLastError();
}

}  // namespace tla
