// rope_norm.hip — RMSNorm, NeoX RoPE and the fused qk-RMSNorm + RoPE that
// feed the KV append.
//
// Both ops are bit-identical to the reference CPU backend:
//   RMSNorm  (reference src/backends/cpu_backend.cpp:335-382): float squares
//            accumulated in double in index order, scale =
//            float(1.0 / sqrt(sum/dim + eps)) in double, out = (x*scale)*w.
//   RoPE     (src/backends/cpu_backend.cpp:443-523): o_j = x0*c - x1*s,
//            o_{j+h} = x0*s + x1*c with c, s the glibc cosf/sinf of the angle
//            table entry; here they come from sin/cos tables built once on the
//            host (ikv_rope_sincos_table_f32) and kept resident in HBM.
// Contraction into FMA is disabled in this file so every product and sum
// rounds exactly as the reference's separate float operations do.
//
// Layout: each workgroup is one wavefront owning up to 64 rows. Rows are
// loaded with coalesced accesses into LDS (row stride dim+1 floats, so the
// per-lane row walks below are bank-conflict free), each lane then runs the
// ordered double-precision sum of its own row, normalises and rotates it in
// LDS, and the block is stored back coalesced. Rows are independent, so
// x == out (in place) is safe.
#pragma clang fp contract(off)

#include "ikv_common.hpp"
#include "../../include/ikv.h"

#include <climits>

namespace {

constexpr int kLdsFloats = 64 * 129;  // 33 KB: 64 rows of 128, or fewer longer rows

int rows_per_block(int dim) {
  int r = kLdsFloats / (dim + 1);
  if (r > 64) r = 64;
  if (r < 1) r = 1;
  return r;
}

template <bool NORM, bool ROPE>
__global__ __launch_bounds__(64) void row_kernel(const float *__restrict__ x,
                                                 const float *__restrict__ w, float *out,
                                                 const int32_t *__restrict__ pos, int64_t rows,
                                                 int dim, int rpb, float eps, int n_heads,
                                                 const float *__restrict__ sin_tab,
                                                 const float *__restrict__ cos_tab, int64_t n_ctx,
                                                 int *status) {
  extern __shared__ float lds[];
  const int lane = threadIdx.x;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * rpb;
  const int64_t left = rows - row0;
  const int nr = static_cast<int>(left < rpb ? left : rpb);
  const int stride = dim + 1;
  const int total = nr * dim;

  const float *xb = x + row0 * dim;
  for (int i = lane; i < total; i += 64) {
    const int r = i / dim;
    const int c = i - r * dim;
    lds[r * stride + c] = xb[i];
  }
  __syncthreads();

  if (lane < nr) {
    float *rp = &lds[lane * stride];
    if (NORM) {
      double sum = 0.0;
      for (int c = 0; c < dim; ++c) {
        const float xv = rp[c];
        const float sq = xv * xv;
        sum += static_cast<double>(sq);
      }
      const float scale =
          static_cast<float>(1.0 / sqrt(sum / static_cast<double>(dim) + static_cast<double>(eps)));
      for (int c = 0; c < dim; ++c) {
        const float t = rp[c] * scale;
        rp[c] = t * w[c];
      }
    }
    if (ROPE) {
      const int64_t token = (row0 + lane) / n_heads;
      const int32_t p = pos[token];
      const int hd = dim / 2;
      if (p < 0 || p >= n_ctx) {
        for (int c = 0; c < dim; ++c) rp[c] = 0.0f;
        if (status) *status = 1;
      } else {
        const float *sn = sin_tab + static_cast<int64_t>(p) * hd;
        const float *cs = cos_tab + static_cast<int64_t>(p) * hd;
        for (int jj = 0; jj < hd; ++jj) {
          const float x0 = rp[jj];
          const float x1 = rp[jj + hd];
          const float c = cs[jj];
          const float s = sn[jj];
          const float a = x0 * c;
          const float b = x1 * s;
          const float e = x0 * s;
          const float f = x1 * c;
          rp[jj] = a - b;
          rp[jj + hd] = e + f;
        }
      }
    }
  }
  __syncthreads();

  float *ob = out + row0 * dim;
  for (int i = lane; i < total; i += 64) {
    const int r = i / dim;
    const int c = i - r * dim;
    ob[i] = lds[r * stride + c];
  }
}

template <bool NORM, bool ROPE>
int launch_rows(const float *x, const float *w, float *out, const int32_t *pos, int64_t rows,
                int dim, float eps, int n_heads, const float *sin_tab, const float *cos_tab,
                int64_t n_ctx, int *status, void *stream) {
  const int rpb = rows_per_block(dim);
  const int64_t blocks = (rows + rpb - 1) / rpb;
  if (blocks > INT_MAX) return -EOVERFLOW;
  const size_t shmem = sizeof(float) * static_cast<size_t>(rpb) * (dim + 1);
  row_kernel<NORM, ROPE><<<static_cast<unsigned>(blocks), 64, shmem, static_cast<hipStream_t>(stream)>>>(
      x, w, out, pos, rows, dim, rpb, eps, n_heads, sin_tab, cos_tab, n_ctx, status);
  return ikv::launch_status();
}

}  // namespace

extern "C" int ikv_rms_norm_f32(const float *x, const float *w, float *out, int64_t rows,
                                int64_t dim, float eps, void *stream) {
  if (rows == 0) return 0;
  if (!x || !w || !out || rows < 0 || dim <= 0) return -EINVAL;
  if (dim > kLdsFloats - 1) return -ENOTSUP;
  if (rows > INT64_MAX / dim) return -EOVERFLOW;
  return launch_rows<true, false>(x, w, out, nullptr, rows, static_cast<int>(dim), eps, 1, nullptr,
                                  nullptr, 0, nullptr, stream);
}

extern "C" int ikv_rope_sincos_table_f32(const float *theta_host, size_t count, float *sin_host,
                                         float *cos_host) {
  if (count == 0) return 0;
  if (!theta_host || !sin_host || !cos_host) return -EINVAL;
  for (size_t i = 0; i < count; ++i) {
    sin_host[i] = sinf(theta_host[i]);
    cos_host[i] = cosf(theta_host[i]);
  }
  return 0;
}

static int check_rope_args(const float *x, float *out, const int32_t *pos, int64_t n_tokens,
                           int n_heads, int head_dim, const float *sin_tab, const float *cos_tab,
                           int64_t n_ctx) {
  if (!x || !out || !pos || !sin_tab || !cos_tab) return -EINVAL;
  if (n_tokens < 0 || n_heads <= 0 || head_dim <= 0 || (head_dim & 1) || n_ctx <= 0) return -EINVAL;
  if (head_dim > kLdsFloats - 1) return -ENOTSUP;
  if (n_tokens > INT64_MAX / n_heads / head_dim) return -EOVERFLOW;
  return 0;
}

extern "C" int ikv_rope_neox_f32(const float *x, float *out, const int32_t *pos, int64_t n_tokens,
                                 int n_heads, int head_dim, const float *sin_tab,
                                 const float *cos_tab, int64_t n_ctx, int *status, void *stream) {
  if (n_tokens == 0) return 0;
  const int rc = check_rope_args(x, out, pos, n_tokens, n_heads, head_dim, sin_tab, cos_tab, n_ctx);
  if (rc) return rc;
  return launch_rows<false, true>(x, nullptr, out, pos, n_tokens * n_heads, head_dim, 0.0f,
                                  n_heads, sin_tab, cos_tab, n_ctx, status, stream);
}

extern "C" int ikv_qk_norm_rope_f32(const float *x, const float *w, float *out, const int32_t *pos,
                                    int64_t n_tokens, int n_heads, int head_dim, float eps,
                                    const float *sin_tab, const float *cos_tab, int64_t n_ctx,
                                    int *status, void *stream) {
  if (n_tokens == 0) return 0;
  if (!w) return -EINVAL;
  const int rc = check_rope_args(x, out, pos, n_tokens, n_heads, head_dim, sin_tab, cos_tab, n_ctx);
  if (rc) return rc;
  return launch_rows<true, true>(x, w, out, pos, n_tokens * n_heads, head_dim, eps, n_heads,
                                 sin_tab, cos_tab, n_ctx, status, stream);
}
