// Projections on either side of the attention path: burn's nn::Linear as MultiHeadAttention
// applies it (crates/sketchpad-core/src/transformer.rs:196-208, :249-253), as hand-written MFMA
// GEMMs (linear.hip).
#pragma once

#include "sp_common.hpp"

namespace sp {

// Rows of x one call takes: the row tiles (64 rows each at most) index the grid's y dimension.
constexpr int64_t kLinearMaxRows = 65535LL * 64;

struct LinearPlan {
  bool big;        // 256 x 256 tiles (M >= 512, K % 64 == 0)
  int tile_m;      // 256, 128 or 64 (M <= 64)
  int splits;      // split-K factor (1: no partials)
  int64_t k_per_split;
  size_t ws_bytes; // fp32 partials [splits][M][N] when splits > 1
};

// The tiling and split-K factor for y[M, N] = x[M, K] . w^T; max_ws bounds the partials.
LinearPlan plan_linear(int64_t M, int64_t K, int64_t N, size_t max_ws);

// y[M, N] = x[M, K] . w[N, K]^T (+ bias[N]); the bias is added to the product already rounded to
// the element type, then rounded again (the reference's matmul and + bias as two ops).
int launch_linear(void* y, const void* x, const void* w_nk, const void* bias, int64_t M,
                  int64_t K, int64_t N, sp_dtype dtype, void* workspace, size_t workspace_bytes,
                  hipStream_t stream);

// dst[N, K] = src[K, N]^T (the reference's [in, out] weight into the kernels' [out, in]).
int launch_weight_transpose(void* dst, const void* src, int64_t K, int64_t N, sp_dtype dtype,
                            hipStream_t stream);

}  // namespace sp
