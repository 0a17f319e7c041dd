// gemm.hpp — the F32 MFMA matrix product of the prefill projections
// (gemm.hip), called by ikv_mul_mat_f32 for more than 64 tokens.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ikv {

// ikv_mul_mat_f32 takes gemm_nt_f32 from this many tokens on and rocBLAS
// below: with fewer tokens the tiles leave CUs idle for the whole K loop
// (no split of K here), measured 1.1-2.3x the rocBLAS time at 200-1024
// tokens, against 1.02-1.10x at 2048 and 4096.
constexpr int64_t kGemmMinTokens = 2048;

// Whether gemm_nt_f32 takes the shape: n_out % 64 == 0, k % 64 == 0.
bool gemm_nt_supported(int64_t n_out, int64_t k, int64_t m);

// out[m][n_out] = x[m][k] w[n_out][k]^T (+ residual[m][n_out], which may be
// out itself); w and x 16-byte aligned. 0, or -ENOTSUP / -EINVAL / -EOVERFLOW
// before any launch, or the launch's hipError_t.
int gemm_nt_f32(const float *w, const float *x, float *out, const float *residual, int64_t n_out,
                int64_t k, int64_t m, hipStream_t s);

}  // namespace ikv
