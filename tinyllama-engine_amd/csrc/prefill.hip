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
//     causal mask, online softmax per query row
//     O^T[64 d][32 queries]   += V^T[64][32] . P^T[32][32] 32 x mfma_f32_32x32x2f32
//   The S accumulator layout (lane l: query l%32, keys 8*(g/4)+4*(l/32)+g%4)
//   is the B operand of the P.V product as is, so P never leaves registers.
//   Q (rotated in registers with the host-built table) is loaded once.
//
// Scheduling: key/value tiles of one (layer, kv head) are read by all its
//   query tiles and q heads, so those workgroups are placed on one XCD
//   (workgroup i runs on XCD i % 8) to share that XCD's L2, and within a
//   (layer, kv head) the query tiles with the most key tiles go first.
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
    float4 kx = ldg4(p.k + row * kHeadDim + 4 * c4);
    if (p.rotate) {
        const float* tab = reinterpret_cast<const float*>(p.rope + (long long)pos * kPairs);
        kx = rotate4(kx, ldg4(tab + 4 * c4));
    }
    const long long dst = (long long)(p.layer0 + lb) * p.layer_stride +
                          ((long long)pos * p.n_head_kv + kvh) * kHeadDim + 4 * c4;
    stg4(p.kc + dst, kx);
    stg4(p.vc + dst, ldg4(p.v + row * kHeadDim + 4 * c4));
}

struct PrefillGrid {
    int n_qt;       // query tiles
    int n_hg;       // head groups of 4 waves per kv head
    int n_logical;  // n_lb * n_head_kv * n_hg * n_qt
    int per_xcd;    // ceil(n_logical / 8)
};

constexpr int kRowPad = 68;  // LDS row stride (floats): 64 + 4 keeps operand reads conflict-free

__global__ __launch_bounds__(64 * kWavesP) __attribute__((amdgpu_waves_per_eu(3, 3))) void
prefill_attention_kernel(const PrefillParams p, const PrefillGrid g)
{
    // K and V tiles of 32 keys, shared by the 4 waves, double-buffered.
    __shared__ float sk[2][kKTile][kRowPad];
    __shared__ float sv[2][kKTile][kRowPad];

    // ---- XCD-aware, heavy-first mapping of workgroups to tiles ----
    const int bid = blockIdx.x;
    const int logical = (bid % kXcds) * g.per_xcd + bid / kXcds;
    if (logical >= g.n_logical) return;  // whole workgroup
    const int per_pair = g.n_qt * g.n_hg;
    const int pair = logical / per_pair;  // (lb, kvh)
    const int r = logical - pair * per_pair;
    const int qt = g.n_qt - 1 - r / g.n_hg;
    const int hg = r % g.n_hg;
    const int lb = pair / p.n_head_kv;
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

    const int kv_dim = p.n_head_kv * kHeadDim;
    const long long layer_off = (long long)(p.layer0 + lb) * p.layer_stride + (long long)kvh * kHeadDim;
    const float* kc = p.kc + layer_off;
    const float* vc = p.vc + layer_off;

    // ---- cooperative tile load: thread -> rows (t/16, t/16 + 16), float4 t%16.
    // Keys past last_key are clamped (masked in the scores).  Byte offsets are
    // 32-bit from a uniform base (a layer's cache slice is < 4 GiB).
    const int lrow = threadIdx.x >> 4, lc4 = threadIdx.x & 15;
    float4 stage[4];  // K row lrow, K row lrow+16, V row lrow, V row lrow+16
    auto gload = [&](int j0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const unsigned key = (unsigned)min(j0 + lrow + 16 * h, last_key);
            const unsigned off = (key * (unsigned)kv_dim + 4u * lc4) * 4u;
            stage[h] = ldg4_at(kc, off);
            stage[2 + h] = ldg4_at(vc, off);
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            *reinterpret_cast<float4*>(&sk[buf][lrow + 16 * h][4 * lc4]) = stage[h];
            *reinterpret_cast<float4*>(&sv[buf][lrow + 16 * h][4 * lc4]) = stage[2 + h];
        }
    };

    // ---- Q^T operand: lane holds q[row][32*half + s], s = 0..31 ----
    float4 qv[8];
    {
        const float* qrow = p.q + (((long long)lb * p.n_tok + trow) * p.n_head + qh) * kHeadDim + 32 * half;
        const float* tab = reinterpret_cast<const float*>(p.rope + (long long)(p.pos0 + trow) * kPairs);
#pragma unroll
        for (int f = 0; f < 8; ++f) {
            float4 x = ldg4(qrow + 4 * f);
            if (p.rotate) x = rotate4(x, ldg4(tab + 2 * (16 * half + 2 * f)));
            qv[f] = x;
        }
    }

    floatx16 o0, o1;
#pragma unroll
    for (int i = 0; i < 16; ++i) { o0[i] = 0.f; o1[i] = 0.f; }
    float m_run = -INFINITY;
    float l_run = 0.f;

    // One key tile from LDS buffer `buf`: S^T = K.Q^T (K operand: lane holds
    // K[j0 + col][32*half + s]), causal mask, online softmax, O^T += V^T.P^T
    // (V operand: lane holds V[key(gi)][2*col + dt], key(gi) = 8*(gi/4) + 4*half + gi%4).
    auto step = [&](int buf, int j0) {
        const float* krow = &sk[buf][col][32 * half];
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
        // s[gi] = S[query col][key j0 + 8*(gi/4) + 4*half + gi%4]
        float mx = -INFINITY;
#pragma unroll
        for (int gi = 0; gi < 16; ++gi) {
            const int key = j0 + 8 * (gi >> 2) + 4 * half + (gi & 3);
            const float x = (key <= qpos && key <= last_key) ? s[gi] * p.scale_log2 : -INFINITY;
            s[gi] = x;
            mx = fmaxf(mx, x);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        float lsum = 0.f;
#pragma unroll
        for (int gi = 0; gi < 16; ++gi) {
            s[gi] = __builtin_amdgcn_exp2f(s[gi] - m_new);
            lsum += s[gi];
        }
        l_run = l_run * alpha + lsum;
        o0 *= alpha;
        o1 *= alpha;
#pragma unroll
        for (int gi = 0; gi < 16; ++gi) {
            const int kin = 8 * (gi >> 2) + 4 * half + (gi & 3);
            const float2 vv = *reinterpret_cast<const float2*>(&sv[buf][kin][2 * col]);
            o0 = mfma32(vv.x, s[gi], o0);
            o1 = mfma32(vv.y, s[gi], o1);
        }
    };

    // Tile j is computed from LDS while tile j+1's global loads are in flight;
    // they land in the other buffer before the barrier that ends the step.
    gload(0);
    lstore(0);
    __syncthreads();
    int buf = 0;
    for (int j0 = 0; j0 <= last_key; j0 += kKTile) {
        const bool more = j0 + kKTile <= last_key;  // uniform
        if (more) gload(j0 + kKTile);
        if (computes) step(buf, j0);
        if (more) lstore(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }

    if (!computes) return;
    l_run += __shfl_xor(l_run, 32);
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
    g.n_logical = p.n_lb * p.n_head_kv * g.n_hg * g.n_qt;
    g.per_xcd = (g.n_logical + kXcds - 1) / kXcds;
    hipLaunchKernelGGL(prefill_attention_kernel, dim3(g.per_xcd * kXcds), dim3(64 * kWavesP), 0, s,
                       p, g);
    return hipGetLastError();
}

}  // namespace tla
