// gemm.hpp — the F32 MFMA matrix product of the prefill projections
// (gemm.hip), called by ikv_mul_mat_f32 for more than one token.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ikv {

// Whether gemm_nt_f32 takes the shape: n_out % 64 == 0, k % 64 == 0.
bool gemm_nt_supported(int64_t n_out, int64_t k, int64_t m);

// Tile shape (a gemm_nt_tile code) and number of K splits for a product.
struct GemmPlan {
  int tile;
  int split;
};
GemmPlan gemm_plan(int64_t n_out, int64_t k, int64_t m, bool may_split);

// One launch on tile shape `tile` (tokens x outputs: 0 128 x 128 (n_out %
// 128 == 0), 1 64 x 64, 2 64 x 32, 3 32 x 64, 4 32 x 32) with K cut into
// n_split ranges (1 <= n_split <= k / 64); for n_split > 1, counters (one
// per tile, all 0; 0 again after the launch) and part (n_split partial
// tiles per tile).
int gemm_nt_tile(int tile, int n_split, const float *w, const float *x, float *out,
                 const float *residual, int n_out, int k, int m, float *part, int *counters,
                 hipStream_t s);

// out[m][n_out] = x[m][k] w[n_out][k]^T (+ residual[m][n_out], which may be
// out itself); w and x 16-byte aligned. With may_split, a product whose tiles
// do not fill the CUs splits K, on a workspace of the stream (allocated on
// the first such call for the device and stream, 8 MiB, kept until exit).
// 0, or -ENOTSUP / -EINVAL / -EOVERFLOW / -ENOMEM before any launch, or the
// hipError_t of the allocation or launch.
int gemm_nt_f32(const float *w, const float *x, float *out, const float *residual, int64_t n_out,
                int64_t k, int64_t m, bool may_split, hipStream_t s);

}  // namespace ikv
