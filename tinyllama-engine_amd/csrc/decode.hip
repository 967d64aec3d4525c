// Split-KV (flash-decoding) GQA decode attention for gfx950.
//
// Semantics follow attention() (src/ops.cpp:1317-1515): append the new k,v
// at `pos` (src/ops.cpp:1350-1371), then for every q head qh, with kv head
// qh / gqa (src/ops.cpp:1329, 1383): scores q.K[p] / sqrt(64) for p in 0..pos,
// softmax, and the weighted sum of V.  With `rotate`, RoPE is applied first
// to q and to the new k, as forward() does (src/forward.cpp:192-196).
//
// Work decomposition.  A "unit" is one (sequence, layer); its positions
// 0..pos form tiles of 16.  The tiles of all units of a launch, laid end to
// end, are cut into equal ranges, one per workgroup (about one per CU), so
// every workgroup streams the same number of tiles however long the units
// are.  A range holds one or more segments (the part of one unit inside
// it); the segments of a unit are its splits.  One workgroup covers a group
// of 1, 2 or 4 kv heads with two waves per kv head, which interleave a
// segment's tiles (wave `sub` takes tiles sub, sub + 2, ...): 256 B, 512 B
// or whole 1 KiB runs of each position row of K and of V.  Smaller
// workgroups measured faster where fixed costs weigh most (one layer at 128
// positions: 7.3 / 8.2 / 10.6 us with 1 / 2 / 4 kv heads per workgroup; 22
// layers at 2048 positions: 23.05 / 23.4 / 24.3 us), 2 kv heads for many
// rounds of whole sequences (600 against 626 us with 1);
// one 8-wave workgroup with 1 KiB runs faster for long ranges (one
// sequence at 16384: 133 against 138 us; 8 at 16384: 955 against 972).  Each
// wave keeps the gqa (<= 16) q heads of its kv head in registers and, per
// tile:
//
//   S^T[16 pos][16 heads] = K[16 pos][64] . Q^T[64][16 heads]
//                           16 x v_mfma_f32_16x16x4f32, heads gqa..15 zero
//   online softmax per head (running max in log2 units, running sum)
//   O^T[64 d][16 heads]  += V^T[64 d][16 pos] . P^T[16 pos][16 heads]
//                           16 x v_mfma_f32_16x16x4f32
//
// The MFMA operand layouts are chosen so that nothing is transposed:
// the S accumulator (lane l holds S[pos = 4*(l/16)+r][head = l%16], r=0..3)
// is directly the B operand of the P.V products, and K and V are loaded
// from HBM straight into A-operand registers with 16-byte loads.  Each
// lane loads 64 B of a K row and 4 x 16 B of V rows per tile; a wave's
// loads cover 16 full 256 B head rows of K and of V.  No LDS staging is
// needed.  Two tiles are in flight per wave: the next tile's loads are
// issued before the current tile is computed, and q and the first two
// tiles are requested together at the start.  Cache rows are read through
// buffer resources that end at the segment's last row, so rows past it
// read as zeros without a memory request.
//
// The split that contains `pos` also appends the new token: it writes the
// (rotated) k row and the v row to the cache and uses the same values,
// kept in LDS, for position `pos` in its own tile (the value its tile load
// got from the cache for that row, possibly older than the append, is
// discarded).  With in_cache (TLA_KV_IN_CACHE) the caller's projection has
// already written the row, and nothing is appended.
//
// Merge.  The two waves of a kv head combine in LDS.  With one split, the
// result goes to `out` directly.  With several, each split writes its
// unnormalised O and (running max, sum) to the workspace, waits for the
// stores, then bumps the arrival counter of its (unit, kv head group); the
// workgroup that arrives last merges all splits of the unit with
// log-sum-exp weights, in split order, and resets the counter to zero for
// the next launch.  The aligned plan's merger takes its own partial from
// LDS; a balanced-plan workgroup defers its arrivals to the end of its
// range and reads every partial from the workspace.  Either way the sums
// do not depend on which workgroup merges.  One launch per step.
#include "lane_math.h"
#include "rope_math.h"
#include "tla_internal.h"

namespace tla {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kSub = 2;  // position halves per kv head; waves per workgroup = kv heads * kSub
// Deferred split arrivals per workgroup: only a range's first and last
// segments can share their unit with another range (every segment between
// them is a whole unit, merged in place).
constexpr int kMaxPending = 2;

__device__ __forceinline__ floatx4 mfma16(float a, float b, floatx4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Split partials cross workgroups (and XCDs, each with its own L2) inside one
// launch.  They are written and read with device-scope (sc1) buffer accesses,
// which go to the device-coherent level instead of a non-coherent L2 copy,
// so no cache-wide writeback/invalidate (what an agent-scope fence costs) is
// needed.  16-byte accesses keep each request a whole vector.
//
// Why the hand-off is ordered (LLVM AMDGPU memory model, GFX942 code
// sequences, which gfx950 follows):
//   * a monotonic agent-scope atomic store / load is the plain instruction
//     with sc1 = 1, so every partial word and every counter access here is an
//     agent-scope atomic access at the ISA level, coherent across XCDs;
//   * a release at agent scope is "buffer_wbl2 sc1; s_waitcnt vmcnt(0)"
//     before the releasing operation, an acquire "s_waitcnt vmcnt(0);
//     buffer_inv sc1" after the acquiring one.  The waits order the memory
//     operations; the L2 writeback / invalidate exist for non-atomic data,
//     whose lines an L2 may hold non-coherently, and nothing of that kind is
//     handed over here.
// So the writer keeps the ordering half of a release (s_waitcnt vmcnt(0)
// after its sc1 stores, before the counter atomic, with a compiler barrier
// so that no store moves past the wait) and the merger issues its sc1 loads
// only after the counter atomic has returned and a barrier has passed.
// Measured on MI355X (22 layers x 2048, batch 1; 8 x 16384): the full
// release + acquire pair on the counter atomic took 61 us against 23.2 us,
// the release alone 58.5 us (an L2 writeback in each of ~1000 splits), the
// acquire alone in the merging workgroup 24.4 us (+1.1 us) and +1.1 % at
// 8 x 16384.
constexpr int kDeviceScope = 16;             // cache-policy bit SC1: device scope
constexpr int kRawBufferWord3 = 0x00020000;  // untyped 32-bit buffer (gfx9 family)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(float* base, int bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(base, 0, bytes, kRawBufferWord3);
}

// The buffer builtins move raw 32-bit words: bit-cast, never value-convert.
typedef unsigned uintx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void st_dev4(floatx4 v, __amdgpu_buffer_rsrc_t rs, int byte_off)
{
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uintx4, v), rs, byte_off, 0,
                                           kDeviceScope);
}

__device__ __forceinline__ void st_dev1(float v, __amdgpu_buffer_rsrc_t rs, int byte_off)
{
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), rs, byte_off, 0,
                                          kDeviceScope);
}

__device__ __forceinline__ floatx4 ld_dev4(__amdgpu_buffer_rsrc_t rs, int byte_off)
{
    return __builtin_bit_cast(floatx4,
                              __builtin_amdgcn_raw_buffer_load_b128(rs, byte_off, 0, kDeviceScope));
}

// Bounded cache reads: a raw buffer load whose offset is past the
// resource's byte count returns zeros without a memory request.  The cache
// rows are read once per launch, so the loads are non-temporal: a streaming
// read of the same bytes runs ~10 % faster with the nt bit than without
// (tla_read_floor, 185 MB-5.9 GB).
constexpr unsigned kOutOfRange = 0x80000000u;  // > any slice (engine: < 2^31 - 256 B)
constexpr int kNonTemporal = 2;                // cache-policy bit NT (gfx940 family)

__device__ __forceinline__ float4 ld_rows4(__amdgpu_buffer_rsrc_t rs, unsigned byte_off)
{
    return __builtin_bit_cast(float4,
                              __builtin_amdgcn_raw_buffer_load_b128(rs, byte_off, 0, kNonTemporal));
}

__device__ __forceinline__ float ld_dev1(__amdgpu_buffer_rsrc_t rs, int byte_off)
{
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_raw_buffer_load_b32(rs, byte_off, 0, kDeviceScope));
}

struct Tile {
    float4 k[4];  // K row (p0 + hsub), dims 16t + 4grp + c
    float4 v[4];  // V row (p0 + 4grp + r), dims 4hsub + c
};

// Partial layout, per (unit, split, kv head) slot, for the gqa real heads
// only (MFMA columns gqa..15 are padding): for i = 0..3, the float4
// O[head hsub][16*grp + 4*i .. +3] of lane li = grp*gqa + hsub at float
// offset (i*4*gqa + li)*4; then m[hsub] at 64*gqa and l[hsub] at 65*gqa.
// One 16-byte store (or load) instruction covers 4*gqa contiguous float4s.
__device__ __forceinline__ int part_floats(int gqa)
{
    return 66 * gqa;
}

__device__ __forceinline__ long long part_slot(const DecodeParams& p, int unit, int split, int kvh)
{
    return (((long long)unit * p.max_splits + split) * p.n_head_kv + kvh) * part_floats(p.gqa);
}

// Running state of one lane: O[head hsub][16*grp + 4*i + c] in acc[i][c],
// the head's running max (log2 units) and sum.
struct Partial {
    floatx4 acc[4];
    float m;
    float l;
};

// Combine the state of the wave one position-half above (in LDS) into this
// wave's: the two halves of a kv head meet here.  Either side may be empty
// (m = -inf, l = 0, acc = 0) but not both.
template <int kKv>  // kv heads per workgroup
struct HalfExchange {
    floatx4 acc[kKv][4][64];
    float m[kKv][16];
    float l[kKv][16];
};

// Online merge of the partials of splits [s_lo, s_hi) of one unit for one
// kv head, each lane merging the same 16 values it produces in the main
// loop: O = sum_s O_s w_s, l = sum_s l_s w_s with w_s = 2^(m_s - max m).
// Split `own` (the merging workgroup's) is read from `mine` in LDS, every
// other from the workspace, so the order of the sums does not depend on
// which workgroup merges.  Chunks of 8 splits whose loads are all issued
// before any is used.
template <int kKv>
__device__ Partial merge_range(const DecodeParams& p, int unit, int s_lo, int s_hi, int own,
                               const HalfExchange<kKv>& mine, int slot, int kvh, int lane)
{
    constexpr int kChunk = 8;
    const int hsub = lane & 15, grp = lane >> 4;
    const int li = grp * p.gqa + hsub;
    const int slot_bytes = part_floats(p.gqa) * 4;
    Partial r;
    r.m = -INFINITY;
    r.l = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) r.acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (hsub >= p.gqa) return r;  // padding columns hold no partials
    for (int s0 = s_lo; s0 < s_hi; s0 += kChunk) {
        float ms[kChunk], ls[kChunk];
        floatx4 x[kChunk][4];
        auto read = [&](int j) {
            const auto rs = part_rsrc(p.part + part_slot(p, unit, s0 + j, kvh), slot_bytes);
#pragma unroll
            for (int i = 0; i < 4; ++i) x[j][i] = ld_dev4(rs, (i * 4 * p.gqa + li) * 16);
            ms[j] = ld_dev1(rs, (64 * p.gqa + hsub) * 4);
            ls[j] = ld_dev1(rs, (65 * p.gqa + hsub) * 4);
        };
        auto use = [&](int j) { return s0 + j < s_hi && s0 + j != own; };
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            if (use(j)) {
                read(j);
            } else if (s0 + j < s_hi) {  // s0 + j == own
#pragma unroll
                for (int i = 0; i < 4; ++i) x[j][i] = mine.acc[slot][i][lane];
                ms[j] = mine.m[slot][hsub];
                ls[j] = mine.l[slot][hsub];
            } else {
                ms[j] = -INFINITY;
                ls[j] = 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i) x[j][i] = floatx4{0.f, 0.f, 0.f, 0.f};
            }
        }
        float mc = r.m;
#pragma unroll
        for (int j = 0; j < kChunk; ++j) mc = fmaxf(mc, ms[j]);
        const float sc = __builtin_amdgcn_exp2f(r.m - mc);  // 0 on the first chunk
        r.m = mc;
        r.l *= sc;
#pragma unroll
        for (int i = 0; i < 4; ++i) r.acc[i] *= sc;
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            const float w = __builtin_amdgcn_exp2f(ms[j] - r.m);
            r.l += ls[j] * w;
#pragma unroll
            for (int i = 0; i < 4; ++i) r.acc[i] += x[j][i] * w;
        }
    }
    return r;
}

template <int kKv>
__device__ __forceinline__ void put_half(HalfExchange<kKv>& x, int slot, int lane, const Partial& r)
{
#pragma unroll
    for (int i = 0; i < 4; ++i) x.acc[slot][i][lane] = r.acc[i];
    if (lane < 16) {
        x.m[slot][lane] = r.m;
        x.l[slot][lane] = r.l;
    }
}

template <int kKv>
__device__ __forceinline__ void add_half(const HalfExchange<kKv>& x, int slot, int lane, Partial& r)
{
    const float m1 = x.m[slot][lane & 15], l1 = x.l[slot][lane & 15];
    const float mm = fmaxf(r.m, m1);
    const float a0 = __builtin_amdgcn_exp2f(r.m - mm), a1 = __builtin_amdgcn_exp2f(m1 - mm);
    r.m = mm;
    r.l = r.l * a0 + l1 * a1;
#pragma unroll
    for (int i = 0; i < 4; ++i) r.acc[i] = r.acc[i] * a0 + x.acc[slot][i][lane] * a1;
}

// kSeg: balanced plan, more than one segment per workgroup possible; the
// aligned plan's instantiation runs the segment body exactly once.
// kKvWaves: kv heads per workgroup (two waves each).
template <int kMaxSeq, bool kSeg, int kKvWaves>
__global__ __launch_bounds__(64 * kSub * kKvWaves) void decode_split_kernel(
    const DecodeParams p, const DecodeSeqs<kMaxSeq> b)
{
    __shared__ int s_last;
    __shared__ float4 s_new[kKvWaves][32];  // appended k row (16 float4) | v row (16 float4)
    __shared__ HalfExchange<kKvWaves> s_half;
    __shared__ HalfExchange<kKvWaves> s_mine;  // this split's partial, for the merge (!kSeg)
    __shared__ int2 s_pend[kMaxPending];  // (unit, nsplit) of deferred arrivals (kSeg)
    __shared__ int s_pend_last[kMaxPending];
    // Every pointer argument is needed before the first memory request; the
    // empty asm takes them in scalar registers here, so their loads go out
    // with the other kernel arguments in one batch (else the compiler
    // issues them after the first batch has arrived: one more round trip).
    asm volatile("" ::"s"(p.q), "s"(p.k), "s"(p.v), "s"(p.out), "s"(p.kc), "s"(p.vc), "s"(p.rope),
                 "s"(p.part));
    // Likewise every scalar field the first loads depend on (the compiler
    // fetches the ones it needs later in a second batch, after the first has
    // arrived: one more round trip before the first tile is requested), and
    // for one sequence its position and offsets.
    asm volatile("" ::"s"(p.counters), "s"(p.seq_stride), "s"(p.layer_stride), "s"(p.wg_tiles),
                 "s"(p.total_tiles), "s"(p.aligned), "s"(p.in_cache), "s"(p.rotate), "s"(p.n_lb),
                 "s"(p.layer0));
    if constexpr (kMaxSeq == 1)
        asm volatile("" ::"s"(b.pos[0]), "s"(b.seq_id[0]), "s"(b.tile_prefix[0]));
    const int lane = threadIdx.x & 63;
    // wave index made explicitly scalar so cache bases stay in SGPRs
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slot = wave % kKvWaves;  // kv head within the workgroup
    const int sub = wave / kKvWaves;   // which half of the split's positions
    const int group = blockIdx.y;  // kv group
    const int kvh = group * kKvWaves + slot;
    const bool active = kvh < p.n_head_kv;  // uniform per wave

    // Workgroup w takes the flat tiles [w * wg_tiles, (w + 1) * wg_tiles).
    // The range falls into one or more segments, each the part of one unit
    // inside it; the segments of one unit, in workgroup order, are its
    // splits.  Balanced (aligned = 0): units end to end, every workgroup
    // streams the same number of tiles.  Aligned: each unit padded to whole
    // ranges, so a workgroup has exactly one segment (the unit's last range
    // may be short).  The loop is uniform per workgroup.
    const int f_lo = blockIdx.x * p.wg_tiles;
    const int f_hi = min(f_lo + p.wg_tiles, p.total_tiles);
    int f = f_lo;
    int n_pend = 0;  // segments whose arrival is deferred (kSeg)
    do {
        // The rank holding flat tile f: the last with tile_prefix <= f.  Up
        // to 8 sequences, an unrolled scan selecting among fields at fixed
        // offsets, so every kernel-argument load goes out in the first batch
        // (an index found by a search would cost a dependent round trip per
        // step, microseconds per launch at small contexts).
        int pos, seq, prefix;
        if constexpr (kMaxSeq <= 8) {
            pos = b.pos[0];
            seq = b.seq_id[0];
            prefix = b.tile_prefix[0];
#pragma unroll
            for (int r = 1; r < kMaxSeq; ++r) {
                const bool take = r < p.n_seq && b.tile_prefix[r] <= f;
                pos = take ? b.pos[r] : pos;
                seq = take ? b.seq_id[r] : seq;
                prefix = take ? b.tile_prefix[r] : prefix;
            }
        } else {
            int lo = 0, hi = p.n_seq - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (b.tile_prefix[mid] <= f) lo = mid; else hi = mid - 1;
            }
            pos = b.pos[lo];
            seq = b.seq_id[lo];
            prefix = b.tile_prefix[lo];
        }
        const int unit_tiles = pos / kDecodeTile + 1;
        // With `aligned`, each unit's space is padded to whole ranges.
        const int unit_span =
            p.aligned ? (unit_tiles + p.wg_tiles - 1) / p.wg_tiles * p.wg_tiles : unit_tiles;
        const int lb = (f - prefix) / unit_span;
        const int u0 = prefix + lb * unit_span;  // the unit's first flat tile
        const int u1 = u0 + unit_tiles;
        const int seg_end = min(f_hi, u1);
        const int split = blockIdx.x - u0 / p.wg_tiles;
        const int nsplit = (u1 - 1) / p.wg_tiles - u0 / p.wg_tiles + 1;
        const int unit = seq * p.n_lb + lb;
        const int layer = p.layer0 + lb;

        // The segment's positions [begin, end) are cut into tiles of 16.  The
        // two waves of a kv head interleave them, wave `sub` taking tiles sub,
        // sub + 2, sub + 4, ...: a fixed assignment, so results do not depend
        // on timing.
        const int begin = (f - u0) * kDecodeTile;
        const int end = min(pos + 1, (seg_end - u0) * kDecodeTile);  // exclusive
        const int n_tiles = seg_end - f;
        f = seg_end < u1 ? seg_end : min(f_hi, u0 + unit_span);  // past the padding
        const bool appends = !p.in_cache && pos < end;  // this split holds `pos` and appends it
        const int special = appends ? n_tiles - 1 : n_tiles;

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

        // Append (attention() step 1, src/ops.cpp:1370-1371): 16 lanes of the
        // first wave of the kv head write the (rotated) k row and the v row to
        // the cache and keep a copy in LDS for the split's last tile.
        if (active && appends && sub == 0 && lane < 16) {
            const long long row = ((long long)unit * p.n_head_kv + kvh) * kHeadDim + 4 * lane;
            const float4 k_in = ldg4(p.k + row);
            const float4 cs = ldg4(tab + 4 * lane);  // loaded either way: no branch before the loads
            const float4 vx = ldg4(p.v + row);
            const float4 kx = p.rotate ? rotate4(k_in, cs) : k_in;
            stg4(kc + (long long)pos * kv_dim + 4 * lane, kx);
            stg4(vc + (long long)pos * kv_dim + 4 * lane, vx);
            s_new[slot][lane] = kx;
            s_new[slot][16 + lane] = vx;
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
            // The q and table loads, then the first two tiles' loads, are all
            // issued before q is rotated (below).
            float4 qv[4], qcs[4];
            {
                const float* qrow = p.q + ((long long)unit * p.n_head + (head_ok ? qh : 0)) * kHeadDim;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    qv[t] = ldg4(qrow + 16 * t + 4 * grp);
                    qcs[t] = ldg4(tab + 2 * (8 * t + 2 * grp));
                }
            }

            // Rows at or past `end` are masked; their loads fall outside the
            // buffer of rows [0, end) and return zeros without a memory
            // request, so a tile past the end costs no traffic.  Byte offsets
            // are 32-bit (a slice is < 2 GiB) from a wave-uniform base.
            const unsigned slice_bytes = (unsigned)end * kv_dim * 4u;
            const auto krs = __builtin_amdgcn_make_buffer_rsrc(kc, 0, slice_bytes, kRawBufferWord3);
            const auto vrs = __builtin_amdgcn_make_buffer_rsrc(vc, 0, slice_bytes, kRawBufferWord3);
            auto load_tile = [&](int tile, Tile& tl) {
                const int p0 = begin + tile * kDecodeTile;
                const int r = p0 + hsub;
                const unsigned ko = r < end ? ((unsigned)r * kv_dim + 4u * grp) * 4u : kOutOfRange;
#pragma unroll
                for (int t = 0; t < 4; ++t) tl.k[t] = ld_rows4(krs, ko + 64u * t);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = p0 + 4 * grp + i;
                    tl.v[i] = ld_rows4(
                        vrs, row < end ? ((unsigned)row * kv_dim + 4u * hsub) * 4u : kOutOfRange);
                }
            };

            // One tile: S^T = K.Q^T, online softmax, O^T += V^T.P^T.
            auto step = [&](const Tile& tl, int tile) {
                const int p0 = begin + tile * kDecodeTile;
                floatx4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    s = mfma16(tl.k[t].x, qv[t].x, s);
                    s = mfma16(tl.k[t].y, qv[t].y, s);
                    s = mfma16(tl.k[t].z, qv[t].z, s);
                    s = mfma16(tl.k[t].w, qv[t].w, s);
                }
                // s[r] = S[position p0 + 4grp + r][head hsub]
                float sc[4];
                float mx = -INFINITY;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int kp = p0 + 4 * grp + r;
                    sc[r] = (kp < end) ? s[r] * p.scale_log2 : -INFINITY;
                    mx = fmaxf(mx, sc[r]);
                }
                mx = max_xor32(max_xor16(mx));  // the tile's 16 positions (lane groups)
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
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    o[0] = mfma16(tl.v[r].x, ps[r], o[0]);
                    o[1] = mfma16(tl.v[r].y, ps[r], o[1]);
                    o[2] = mfma16(tl.v[r].z, ps[r], o[2]);
                    o[3] = mfma16(tl.v[r].w, ps[r], o[3]);
                }
            };

            // The appending split's last tile holds `pos`; that row comes from
            // LDS (the copy kept at append), not from the cache, which the
            // append may not have reached when the tile was loaded.  (K rows
            // past `pos` take it too; they are masked.)
            auto substitute = [&](Tile& tl, int tile) {
                const int p0 = begin + tile * kDecodeTile;
                if (p0 + hsub >= pos) {
#pragma unroll
                    for (int t = 0; t < 4; ++t) tl.k[t] = s_new[slot][4 * t + grp];
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = p0 + 4 * grp + i;
                    if (row == pos) tl.v[i] = s_new[slot][16 + hsub];
                }
            };
            auto process = [&](Tile& tl, int tile) {
                if (tile == special) substitute(tl, tile);  // uniform branch
                step(tl, tile);
            };

            // Two tiles in flight: while one is computed the other is loading.
            // In the steady-state loop both next tiles exist and every load is
            // unconditional, so the count of loads in flight is the same on
            // every path and waiting for one tile never waits for the other.
            // The last round is peeled so that no load is issued for a tile
            // past the end: an unused load would still hold the wave (and the
            // split's arrival) for a round trip.  The first ta and tb may lie
            // past the end (n_tiles <= 2 + sub): their loads are out of range
            // and fetch nothing.
            constexpr int kStride = 2 * kSub;  // tiles between a wave's ta and its next ta
            int ca = sub, cb = kSub + sub;
            Tile ta, tb;
            load_tile(ca, ta);
            __builtin_amdgcn_sched_barrier(0);  // all of ta's loads before tb's
            load_tile(cb, tb);
            if (p.rotate) {
#pragma unroll
                for (int t = 0; t < 4; ++t) qv[t] = rotate4(qv[t], qcs[t]);
            }
            if (!head_ok) {
#pragma unroll
                for (int t = 0; t < 4; ++t) qv[t] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
            while (cb + kStride < n_tiles) {  // uniform; ca < cb
                process(ta, ca);
                load_tile(ca + kStride, ta);
                process(tb, cb);
                load_tile(cb + kStride, tb);
                ca += kStride;
                cb += kStride;
            }
            if (ca + kStride < n_tiles) {  // one more ta, no more tb
                process(ta, ca);
                load_tile(ca + kStride, ta);
                process(tb, cb);
                process(ta, ca + kStride);
            } else {
                if (ca < n_tiles) process(ta, ca);
                if (cb < n_tiles) process(tb, cb);
            }

            // Row sums: each lane group summed different positions of the same head.
            l_run = sum_xor32(sum_xor16(l_run));
        }

        // The two halves of each kv head meet in LDS; the first half continues.
        // o[dt][i] = O[head hsub][16*grp + 4*i + dt]  ->  r.acc[i][dt]
        Partial r;
#pragma unroll
        for (int i = 0; i < 4; ++i) r.acc[i] = floatx4{o[0][i], o[1][i], o[2][i], o[3][i]};
        r.m = m_run;
        r.l = l_run;
        if (active && sub == 1) put_half(s_half, slot, lane, r);
        __syncthreads();
        if (active && sub == 0) {
            add_half(s_half, slot, lane, r);
            // r.acc[i][c] = O[head hsub][d = 16*grp + 4*i + c]
            if (nsplit == 1) {
                if (head_ok) {
                    const float inv = 1.0f / r.l;
                    float* orow = p.out + ((long long)unit * p.n_head + qh) * kHeadDim + 16 * grp;
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        stg4(orow + 4 * i, make_float4(r.acc[i][0] * inv, r.acc[i][1] * inv,
                                                       r.acc[i][2] * inv, r.acc[i][3] * inv));
                }
            } else {
                // The partial goes to the workspace for whichever workgroup merges
                // (and, with one segment, to LDS in case it is this one).
                if constexpr (!kSeg) put_half(s_mine, slot, lane, r);
                if (head_ok) {
                    const auto rs =
                        part_rsrc(p.part + part_slot(p, unit, split, kvh), part_floats(p.gqa) * 4);
                    const int li = grp * p.gqa + hsub;
#pragma unroll
                    for (int i = 0; i < 4; ++i) st_dev4(r.acc[i], rs, (i * 4 * p.gqa + li) * 16);
                    if (grp == 0) {
                        st_dev1(r.m, rs, (64 * p.gqa + hsub) * 4);
                        st_dev1(r.l, rs, (65 * p.gqa + hsub) * 4);
                    }
                }
            }
        }

        // Merge of all mn splits of unit mu (split `own` from s_mine, -1: none):
        // both halves of each kv head merge half of the splits, then meet in LDS.
        auto merge_unit = [&](int mu, int mn, int own) {
            const int s_mid = (mn + 1) / 2;
            Partial mr;
            if (active)
                mr = merge_range(p, mu, sub == 0 ? 0 : s_mid, sub == 0 ? s_mid : mn, own, s_mine,
                                 slot, kvh, lane);
            if (active && sub == 1) put_half(s_half, slot, lane, mr);
            __syncthreads();
            if (active && sub == 0 && head_ok) {
                add_half(s_half, slot, lane, mr);
                const float inv = 1.0f / mr.l;
                float* orow = p.out + ((long long)mu * p.n_head + qh) * kHeadDim + 16 * grp;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    stg4(orow + 4 * i, make_float4(mr.acc[i][0] * inv, mr.acc[i][1] * inv,
                                                   mr.acc[i][2] * inv, mr.acc[i][3] * inv));
            }
        };

        if constexpr (kSeg) {
            // Arrivals are deferred to the end of the range: the partial
            // stores drain while the next segment streams, instead of
            // stalling the workgroup in mid-run.
            if (nsplit > 1) {
                if (threadIdx.x == 0) s_pend[n_pend] = make_int2(unit, nsplit);
                ++n_pend;  // uniform
            }
            if (n_pend < kMaxPending && f < f_hi) continue;
            if (n_pend == 0) continue;
            // The partial stores are acknowledged before the arrivals count:
            // the compiler barrier keeps them above the wait (the wait
            // intrinsic itself does not order memory operations for the
            // compiler).
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (threadIdx.x < n_pend) {
                const int2 pu = s_pend[threadIdx.x];
                int* const counter = p.counters + (long long)pu.x * p.n_groups + group;
                const bool last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT) == pu.y - 1;
                if (last)  // every split has arrived: ready for the next launch
                    __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                s_pend_last[threadIdx.x] = last;
            }
            __syncthreads();
            for (int t = 0; t < n_pend; ++t) {
                if (!s_pend_last[t]) continue;  // uniform
                const int2 pu = s_pend[t];
                merge_unit(pu.x, pu.y, -1);
                __syncthreads();  // s_half is reused by the next merge
            }
            n_pend = 0;
        } else {
            if (nsplit == 1) continue;  // uniform per workgroup
            // Wait until this wave's partial stores are acknowledged at device
            // scope (compiler barrier first, as above), then count the split in;
            // the workgroup that completes the count of its (unit, kv head
            // group) merges.
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            int* const counter = p.counters + (long long)unit * p.n_groups + group;
            if (threadIdx.x == 0)
                s_last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT) == nsplit - 1;
            __syncthreads();
            if (!s_last) continue;
            if (threadIdx.x == 0)  // every split has arrived: ready for the next launch
                __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            merge_unit(unit, nsplit, split);
        }
    } while (kSeg && f < f_hi);  // segments
}

// Balanced ranges always use the large group (one 8-wave workgroup).
template <int kMaxSeq>
void launch_shape(const DecodeParams& p, const DecodeSeqs<kMaxSeq>& b, dim3 grid, dim3 block,
                  hipStream_t s)
{
    if (!p.aligned)
        hipLaunchKernelGGL((decode_split_kernel<kMaxSeq, true, kDecodeKvGroupLarge>), grid, block,
                           0, s, p, b);
    else if (p.kv_group == kDecodeKvGroupSmall)
        hipLaunchKernelGGL((decode_split_kernel<kMaxSeq, false, kDecodeKvGroupSmall>), grid, block,
                           0, s, p, b);
    else if (p.kv_group == kDecodeKvGroupMid)
        hipLaunchKernelGGL((decode_split_kernel<kMaxSeq, false, kDecodeKvGroupMid>), grid, block,
                           0, s, p, b);
    else
        hipLaunchKernelGGL((decode_split_kernel<kMaxSeq, false, kDecodeKvGroupLarge>), grid, block,
                           0, s, p, b);
}

}  // namespace

hipError_t load_decode_code()
{
    hipFuncAttributes a;
    return hipFuncGetAttributes(&a, reinterpret_cast<const void*>(&decode_split_kernel<1, false, kDecodeKvGroupSmall>));
}

size_t decode_part_bytes(long long units, int max_splits, int n_head_kv, int gqa)
{
    return static_cast<size_t>(units) * max_splits * n_head_kv * 66 * gqa * sizeof(float);
}

hipError_t launch_decode(const DecodeParams& p, const DecodeSeqs<kMaxSeqPerLaunch>& seqs,
                         hipStream_t s)
{
    if ((p.kv_group != kDecodeKvGroupSmall && p.kv_group != kDecodeKvGroupMid &&
         p.kv_group != kDecodeKvGroupLarge) ||
        (!p.aligned && p.kv_group != kDecodeKvGroupLarge))
        return hipErrorInvalidValue;
    const dim3 grid((p.total_tiles + p.wg_tiles - 1) / p.wg_tiles, p.n_groups);
    const dim3 block(64 * kSub * p.kv_group);
    if (p.n_seq == 1) {
        DecodeSeqs<1> one{};
        one.pos[0] = seqs.pos[0];
        one.seq_id[0] = seqs.seq_id[0];
        one.tile_prefix[0] = seqs.tile_prefix[0];
        one.tile_prefix[1] = seqs.tile_prefix[1];
        launch_shape(p, one, grid, block, s);
    } else if (p.n_seq <= 8) {
        DecodeSeqs<8> small{};
        for (int i = 0; i < p.n_seq; ++i) {
            small.pos[i] = seqs.pos[i];
            small.seq_id[i] = seqs.seq_id[i];
        }
        for (int i = 0; i <= p.n_seq; ++i) small.tile_prefix[i] = seqs.tile_prefix[i];
        launch_shape(p, small, grid, block, s);
    } else {
        launch_shape(p, seqs, grid, block, s);
    }
    return hipGetLastError();
}

}  // namespace tla
