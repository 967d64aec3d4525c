// Streamed batched products (batch.hip): the projections of a batch of a few
// tokens with the weights dequantised in registers.
#ifndef TLA_BATCH_H
#define TLA_BATCH_H

#include "tla_internal.h"

namespace tla {

// out[t][row] (+)= W[row] . x[t] for t < n, 16 rows x 16 `tiles` tokens per
// workgroup; more tokens take further token chunks, each reading the weights
// again.  F32 / F16 / Q8_0 / Q4_0 rows of cols % 32 == 0 columns; x rows
// 16-byte aligned (x_stride % 4 == 0), F32 / F16 weights 16-byte aligned.
constexpr int kStreamMaxTiles = 4;
struct StreamParams {
    GemvSegment seg[kGemvMaxSeg];
    int n_seg;
    int total_rows;          // sum of seg[].rows
    int cols;
    long long row_bytes;
    const float* x;          // x[t * x_stride + col]
    long long x_stride;
    int n;                   // token vectors
    int add;                 // 1: out += W.x, 0: out = W.x
    int tiles;               // token tiles of 16 per workgroup, 1..kStreamMaxTiles
};
bool stream_supported(int type);
hipError_t launch_stream_product(int type, const StreamParams& p, hipStream_t s);

// Products of many tokens on the bf16 matrix cores with fp32 accuracy
// (split_product.hip): x is first split into three bf16 planes
// (launch_split_rows, split_x_bytes(n, cols) bytes at xs), then
// out[t][row] (+)= W[row] . x[t] for every format of the reference
// (F32 / F16 16-byte aligned, Q8_0 / Q4_0 / Q6_K 2-byte aligned), 64 x
// rows_per_wave rows x 64 tokens per workgroup, K in k_splits ranges.
struct SplitParams {
    GemvSegment seg[kGemvMaxSeg];
    int n_seg;
    int total_rows;            // sum of seg[].rows
    int cols;                  // multiple of 32 (of 256 for Q6_K)
    long long row_bytes;
    const unsigned char* xs;   // the planes of launch_split_rows
    int n;                     // tokens
    int n_sub;                 // split_tokens(n) / 16
    int add;                   // 1: out += W.x, 0: out = W.x
    int rows_per_wave;         // 16-row subtiles per wave: 1, 2 or 4
    int k_splits;              // K cut into this many ranges of blk_per_split 32-column
    int blk_per_split;         // blocks (grid z); each split's sums go to part, and a
    float* part;               // second launch adds them in split order: [k_splits][n][total_rows]
    int defer_reduce;          // 1: that launch is left to the caller (launch_reduce_rmsnorm_rows)
};
// x[t][c] += the K ranges' sums part[z][t][c] (z in order, as the split
// product's own second launch adds them), then out[t] = rmsnorm(x[t]) * w
// (the rmsnorm rows' arithmetic): n_tok rows of size floats, one workgroup
// per row.  x, part, out 16-byte aligned, size a multiple of 4.
hipError_t launch_reduce_rmsnorm_rows(float* x, const float* part, int k_splits, float* out, const float* w,
                                      int n_tok, int size, float eps, hipStream_t s);
size_t split_part_bytes(int n, int total_rows, int k_splits);
int split_tokens(int n);                  // tokens padded to the 64-token tile
size_t split_x_bytes(int n, int cols);    // bytes of the planes
hipError_t launch_split_rows(const float* x, long long x_stride, int n, int cols, unsigned char* xs,
                             hipStream_t s);
hipError_t launch_split_product(int type, const SplitParams& p, hipStream_t s);

}  // namespace tla

#endif  // TLA_BATCH_H
