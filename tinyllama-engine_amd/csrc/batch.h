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

}  // namespace tla

#endif  // TLA_BATCH_H
