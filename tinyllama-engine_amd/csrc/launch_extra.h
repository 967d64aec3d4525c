// Launchers that only the C ABI (engine.hip) calls and that no decode,
// prefill or GEMV kernel depends on, kept apart from tla_internal.h (which
// those kernels' source digests cover).
#pragma once

#include <hip/hip_runtime.h>

namespace tla {

// fp32 MFMA floor (small_ops.hip): n_wg workgroups of 4 waves, each wave
// iters x 16 v_mfma_f32_32x32x2f32; sink [n_wg] is never written in practice.
hipError_t launch_mfma_floor(int n_wg, int iters, float* sink, hipStream_t s);

// Weights of `rows` rows of `cols` columns in format `type` (row_bytes per
// row) expanded to fp32 [rows][cols] at out (gemm.hip), with the values the
// batched product multiplies: F32 as is, F16 converted, Q8_0 q * d, Q4_0
// (q - 8) * d, Q6_K d * scale * q.  cols a multiple of 32 (256 for Q6_K).
hipError_t launch_dequant_rows(int type, const unsigned char* w, long long row_bytes, int rows, int cols,
                               float* out, hipStream_t s);

}  // namespace tla
