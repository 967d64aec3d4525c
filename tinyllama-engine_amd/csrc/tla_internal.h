// Internal declarations shared by the HIP sources of libtla.so.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "tla_attention.h"

namespace tla {

constexpr int kHeadDim = 64;        // head_dim the kernels implement
constexpr int kPairs = kHeadDim / 2;
constexpr int kMaxGqa = 16;         // q heads per kv head (MFMA N = 16)
constexpr int kMaxSeqPerLaunch = 256;
constexpr int kDecodeTile = 16;     // positions per decode MFMA tile
// kv heads per decode workgroup (grid y = groups), two waves each, chosen
// per launch: 1 (2-wave workgroups, four per CU), 2 (two 4-wave workgroups
// per CU) or 4 (one 8-wave workgroup).
constexpr int kDecodeKvGroupSmall = 1;
constexpr int kDecodeKvGroupMid = 2;
constexpr int kDecodeKvGroupLarge = 4;
constexpr int kMaxRopePairs = 128;  // tla_rope: head_dim <= 256

// ---- decode ------------------------------------------------------------
// Split partials of one decode launch: per (unit, split, kv head), 66 floats
// per q head of the kv head (64 output floats, running max and sum).
size_t decode_part_bytes(long long units, int max_splits, int n_head_kv, int gqa);

// One "unit" = one (sequence, layer) decode problem.  unit = seq * n_lb + lb.
struct DecodeParams {
    const float* q;      // [n_seq][n_lb][n_head][64]
    const float* k;      // [n_seq][n_lb][n_head_kv][64] new keys
    const float* v;      // [n_seq][n_lb][n_head_kv][64] new values
    float* out;          // [n_seq][n_lb][n_head][64]
    float* kc;           // cache base (seq 0, layer 0)
    float* vc;
    const float2* rope;  // [n_ctx][32] (cos, sin)
    float* part;         // split partials, [unit][max_splits][n_head_kv][66 * gqa]
    int* counters;       // [unit][kv head group] split arrivals; zero between launches
    long long seq_stride;    // floats
    long long layer_stride;  // floats = n_ctx * kv_dim
    int n_seq;
    int n_lb;
    int layer0;
    int n_head;
    int n_head_kv;
    int gqa;
    int wg_tiles;      // tiles of kDecodeTile positions per workgroup
    int max_splits;    // split stride in `part`: most workgroups sharing one unit
    int total_tiles;   // tile_prefix[n_seq]
    int aligned;       // units padded to a multiple of wg_tiles in the flat space
    int in_cache;      // k, v rows at pos already in the cache: no append
    int kv_group;      // kv heads per workgroup: kDecodeKvGroupSmall / Large
    int rotate;
    float scale_log2;  // log2(e) / sqrt(head_dim)
    int n_groups;      // kv groups = ceil(n_head_kv / kv_group) (grid y)
};

// Per-sequence positions and tile offsets of one launch, passed by value in
// the kernel arguments.  Sequences appear by rank, longest first; seq_id maps
// a rank to the caller's sequence index.  The units of rank r are its n_lb
// layers, each of pos[r] / kDecodeTile + 1 tiles (padded to a multiple of
// wg_tiles when aligned), laid end to end from tile_prefix[r] in one flat
// tile space that the workgroups cut into equal ranges.  The kernel is instantiated for up to 8 and up to 256 sequences
// so small batches do not pay for a 3 KiB argument block (about 1 us per
// launch).
template <int kMaxSeq>
struct DecodeSeqs {
    int pos[kMaxSeq];              // by rank
    int seq_id[kMaxSeq];           // rank -> sequence index
    int tile_prefix[kMaxSeq + 1];  // first flat tile of each rank's units
};

hipError_t launch_decode(const DecodeParams& p, const DecodeSeqs<kMaxSeqPerLaunch>& seqs,
                         hipStream_t s);

// ---- prefill -------------------------------------------------------------
struct PrefillParams {
    const float* q;   // [n_lb][n_tok][n_head][64]
    const float* k;   // [n_lb][n_tok][n_head_kv][64]
    const float* v;
    float* out;       // [n_lb][n_tok][n_head][64]
    float* kc;        // cache base of the sequence (layer 0)
    float* vc;
    const float2* rope;
    long long layer_stride;  // floats
    int n_lb;
    int layer0;
    int pos0;
    int n_tok;
    int n_head;
    int n_head_kv;
    int gqa;
    int rotate;
    float scale_log2;
    // K and V of every 32-key tile of positions 0 .. pos0+n_tok-1 as bf16
    // planes, written by the append and read by the attention kernel:
    // [n_lb][n_head_kv][n_ptiles] tiles of prefill_tile_bytes()
    unsigned char* kvp;
    int n_ptiles;
};

size_t prefill_planes_bytes(int n_lb, int n_head_kv, int pos0, int n_tok);
hipError_t launch_prefill_append(const PrefillParams& p, hipStream_t s);
hipError_t launch_prefill_attention(const PrefillParams& p, hipStream_t s);

// ---- projections (matrix-vector products) ---------------------------------
// Weight type ids: the reference's ggml_type values (src/gguf.h:23-32).
enum WeightType { kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ8_0 = 8, kQ6_K = 14 };
constexpr int kGemvMaxVec = 8;    // vectors per launch (x staged in LDS)
constexpr int kGemvMaxSeg = 3;    // matrices per launch (Wq, Wk, Wv)
constexpr int kAttnOutMaxParts = 4;   // kv heads of a fused attention + W_o launch
constexpr int kAttnOutMaxGqa = 8;     // q heads per kv head there
constexpr int kAttnOutMaxPos = 192;   // context positions there (3 tiles of 16 per wave)
constexpr int kAmaxSlots = 64;        // argmax key slots of a GEMV launch (GemvParams::amax)

struct GemvSegment {
    const unsigned char* w;  // [rows][row_bytes]
    float* out;              // out[v * out_stride + row]
    int rows;
    long long out_stride;
};

struct GemvParams {
    GemvSegment seg[kGemvMaxSeg];
    int n_seg;
    int total_rows;          // sum of seg[].rows
    int cols;                // multiple of 64 (of 256 for Q6_K)
    int row_bytes;
    int n_vec;               // 1..kGemvMaxVec
    const float* x;          // x[v * x_stride + col]
    long long x_stride;
    const float* x2;         // non-null: x is replaced by silu(x) * x2 (SwiGLU), same stride
    const float* norm_w;     // non-null: x is (then) replaced by rmsnorm(x, norm_w, eps)
    float eps;
    int add;                 // 1: out += W.x (residual), 0: out = W.x
    int pair;                // 1: segments 0 and 1 are the gate and up matrices (equal rows,
                             // one vector); seg[0].out[r] = silu(gate_r . x) * (up_r . x),
                             // the reference's SwiGLU; seg[1].out is read, not written
    const float2* rope;      // (cos, sin) of the token's position, head_dim / 2 = 32 pairs;
                             // non-null in every launch (read whether or not used)
    int rope_rows;           // rows [0, rope_rows) are rotated in pairs (2i, 2i+1) of each
                             // 64-row head (RoPE of the q and k projections); 0: none
    // Partial sums of the fused attention + W_o launch (launch_attn_out),
    // n_parts vectors of cols (xparts) or rows (rparts) floats each, added
    // to x in the order ((x + (p0 + p1 + ...)), partials summed first, in
    // order):
    const float* xparts;     // non-null: x is replaced by that sum before anything else (no x2)
    const float* rparts;     // non-null (one segment, add = 1): the residual's old out[r] is
    int n_parts;             // replaced by that sum; 1..kAttnOutMaxParts
    // Non-null (one vector, one segment, add = 0, rows of <= 64 units): each
    // workgroup also posts the largest (value, first index) of its outputs,
    // as an argmax key, with an atomic max into amax[blockIdx % kAmaxSlots]
    // (which start at zero).  The largest key of the slots is the argmax of
    // all outputs, by the rule of launch_argmax.
    unsigned long long* amax;
};

// Decode attention of one token over a short context fused with the W_o
// product (launch_attn_out): parts[g][r] = W_o[r][cols of kv head g's q
// heads] . attention output of those heads, for g < n_head_kv.
struct AttnOutParams {
    const float* q;          // [n_head][64], rotated
    const float* kc;         // the layer's key cache [n_ctx][kv_dim] (position n_pos - 1 appended)
    const float* vc;         // the layer's value cache
    int n_pos;               // positions 0 .. n_pos - 1, 1..kAttnOutMaxPos
    int kv_dim;              // n_head_kv * 64
    int gqa;                 // q heads per kv head, 1..kAttnOutMaxGqa
    int n_head_kv;           // 1..kAttnOutMaxParts
    const unsigned char* w;  // W_o [rows][row_bytes], rows x (n_head_kv * gqa * 64)
    long long row_bytes;
    long long group_bytes;   // bytes of gqa * 64 columns of a row
    int rows;
    float* parts;            // [n_head_kv][rows]
};
// Whether launch_attn_out takes this shape.
bool attn_out_supported(int type, int gqa, int n_head_kv, int n_pos);
hipError_t launch_attn_out(int type, const AttnOutParams& p, hipStream_t s);

// Whether launch_gemv can pair gate and up rows (pair = 1) for this shape.
bool gemv_can_pair(int type, int rows, int cols);
// Whether a one-vector launch_gemv over rows of `cols` columns takes
// residual partials (rparts): rows of at most 128 units (cols <= 8192).
bool gemv_can_add_parts(int cols);
// Whether a one-vector launch_gemv over rows of `cols` columns posts argmax
// keys (amax): rows of at most 64 units (cols <= 4096).
bool gemv_can_amax(int cols);
// Whether launch_gemv can rotate row pairs in its epilogue (rope_rows > 0):
// one vector, rows of at most 32 units (cols <= 2048).
bool gemv_can_rope(int cols);

long long weight_row_bytes(int type, int cols);  // 0 if the type is unknown
hipError_t launch_gemv(int type, const GemvParams& p, hipStream_t s);
hipError_t launch_rmsnorm(float* out, const float* x, const float* w, int size, float eps,
                          hipStream_t s);
hipError_t launch_vec_add(float* out, const float* x, int size, hipStream_t s);
hipError_t launch_silu(float* x, int size, hipStream_t s);
hipError_t launch_elementwise_mul(float* a, const float* b, int size, hipStream_t s);
// out[t][n] = table row tokens_dev[t] for t < n_tok (tokens_dev null: one
// row, `token`).
// With amax non-null (one row): the token is the argmax the kAmaxSlots keys
// there give, also stored at token_out when that is non-null.
hipError_t launch_embed(int type, float* out, const unsigned char* table, int token,
                        const int* tokens_dev, int n_tok, int n, hipStream_t s,
                        const unsigned long long* amax = nullptr, int* token_out = nullptr);
// *out = the argmax the kAmaxSlots keys at amax give.
hipError_t launch_amax_token(const unsigned long long* amax, int* out, hipStream_t s);
// *out = first index of the largest value (NaN never wins; a NaN at 0 gives 0),
// also stored at out2 when non-null.
hipError_t launch_argmax(int* out, int* out2, const float* x, int n, hipStream_t s);

// ---- token batches (batch.hip) -------------------------------------------
hipError_t launch_rmsnorm_rows(float* out, const float* x, const float* w, int n_rows, int size, float eps,
                               hipStream_t s);
// h rows of [gate | up] (2 n_ff floats): gate = silu(gate) * up in place.
hipError_t launch_swiglu_rows(float* h, int n_rows, int n_ff, hipStream_t s);

// ---- small ops -------------------------------------------------------------
struct RopeParams {
    float* q;
    float* k;
    int n_head;
    int n_head_kv;
    int head_dim;
    float2 cs[kMaxRopePairs];
};
hipError_t launch_rope(const RopeParams& p, hipStream_t s);
hipError_t launch_softmax(float* x, int size, hipStream_t s);
hipError_t launch_copy(void* dst, const void* src, size_t bytes, hipStream_t s);
// Streaming read of `bytes` (16-byte aligned, whole 16-byte words) by n_wg
// workgroups, each a contiguous chunk, with load form `kind` (0 global, 1
// global nt, 2 buffer, 3 buffer nt) and `depth` (8, 16 or 32) loads in flight
// per thread; sink [n_wg] is never written in practice.
hipError_t launch_read_floor(const void* src, size_t bytes, int n_wg, int kind, int depth, float* sink,
                             hipStream_t s);
// bf16 MFMA floor: n_wg workgroups of 4 waves, each wave iters x 16
// v_mfma_f32_32x32x16_bf16; sink [n_wg] is never written in practice.
hipError_t launch_mfma_floor(int n_wg, int iters, float* sink, hipStream_t s);
// Zero fill by a kernel (no memset node: safe under stream capture).
hipError_t launch_zero(void* dst, size_t bytes, hipStream_t s);

// Each source file's kernels are one code object, which the runtime loads
// (allocating device memory) on first use unless something asks for it
// earlier; the engine asks for all of them when it is created, so that no
// later call allocates for it.
hipError_t load_decode_code();
hipError_t load_prefill_code();
hipError_t load_gemv_code();
hipError_t load_batch_code();
hipError_t load_small_ops_code();

}  // namespace tla
