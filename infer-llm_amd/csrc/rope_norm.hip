// rope_norm.hip — RMSNorm, NeoX RoPE and the fused qk-RMSNorm + RoPE that
// feed the KV append.
//
// Arithmetic of the reference CPU backend:
//   RMSNorm  (reference src/backends/cpu_backend.cpp:335-382): float squares
//            accumulated in double, scale = float(1.0 / sqrt(sum/dim + eps))
//            in double, out = (x*scale)*w; the order of the double sum is
//            below.
//   RoPE     (src/backends/cpu_backend.cpp:443-523): o_j = x0*c - x1*s,
//            o_{j+h} = x0*s + x1*c with c, s the glibc cosf/sinf of the angle
//            table entry; here they come from sin/cos tables built once on the
//            host (ikv_rope_sincos_table_f32) and kept resident in HBM.
// Contraction into FMA is disabled in this file so every product and sum
// rounds exactly as the reference's separate float operations do.
//
// Two sums of squares:
//  * rows shorter than kLongRow (the head_dim rows of qk-norm): one lane per
//    row adds the float squares in index order in double — exactly the
//    reference's loop, so outputs are bit-identical to it;
//  * rows of kLongRow or more floats, a multiple of 256 (the model-width
//    rows of attn_norm / ffn_norm / output_norm): one wavefront per row; lane
//    l adds, in double and in this order, the squares of elements
//    256*j + 4*l + c (j ascending, c = 0..3), then the 64 lane sums combine
//    in a fixed xor butterfly (32, 16, ..., 1). The double sum differs from
//    the sequential one only in its last bits, and the float scale derived
//    from it is the same unless the two straddle a float rounding boundary
//    (about 2^-27 of rows). The GEMV kernels that fold this norm into their
//    input (ikv_model.h) use the same order, so fused and unfused paths agree
//    bit for bit.
//
// Short rows: each workgroup is one wavefront owning up to 64 rows, loaded
// with coalesced accesses into LDS (row stride dim+1 floats, so the per-lane
// row walks are bank-conflict free); lane r sums row r; then every lane
// takes elements (or RoPE pairs) of the block in turn, so weights, sin/cos
// and outputs move coalesced. Rows are independent and each output element is
// written by the lane that read its inputs, so x == out (in place) is safe.
#pragma clang fp contract(off)

#include "ikv_common.hpp"
#include "../../include/ikv.h"

#include <climits>

namespace {

constexpr int kLdsFloats = 64 * 129;  // 33 KB: 64 rows of 128, or fewer longer rows
constexpr int kLongRow = 512;

int rows_per_block(int dim) {
  int r = kLdsFloats / (dim + 1);
  if (r > 64) r = 64;
  if (r < 1) r = 1;
  return r;
}

bool long_row(int64_t dim) { return dim >= kLongRow && dim % 256 == 0; }

template <bool NORM, bool ROPE>
__global__ __launch_bounds__(64) void row_kernel(const float *__restrict__ x,
                                                 const float *__restrict__ w, float *out,
                                                 const int32_t *__restrict__ pos, int64_t rows,
                                                 int dim, int rpb, float eps, int n_heads,
                                                 const float *__restrict__ sin_tab,
                                                 const float *__restrict__ cos_tab, int64_t n_ctx,
                                                 int *status) {
  extern __shared__ float lds[];
  __shared__ float s_scale[64];
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

  if (NORM && lane < nr) {
    const float *rp = &lds[lane * stride];
    double sum = 0.0;
#pragma unroll 8
    for (int c = 0; c < dim; ++c) {
      const float xv = rp[c];
      const float sq = xv * xv;
      sum += static_cast<double>(sq);
    }
    s_scale[lane] =
        static_cast<float>(1.0 / sqrt(sum / static_cast<double>(dim) + static_cast<double>(eps)));
  }
  __syncthreads();

  float *ob = out + row0 * dim;
  if (!ROPE) {
    for (int i = lane; i < total; i += 64) {
      const int r = i / dim;
      const int c = i - r * dim;
      const float t = lds[r * stride + c] * s_scale[r];
      ob[i] = t * w[c];
    }
    return;
  }
  const int hd = dim / 2;
  for (int i = lane; i < nr * hd; i += 64) {
    const int r = i / hd;
    const int j = i - r * hd;
    float x0 = lds[r * stride + j];
    float x1 = lds[r * stride + j + hd];
    if (NORM) {
      const float sc = s_scale[r];
      const float t0 = x0 * sc;
      const float t1 = x1 * sc;
      x0 = t0 * w[j];
      x1 = t1 * w[j + hd];
    }
    const int32_t p = pos[(row0 + r) / n_heads];
    float o0 = 0.0f, o1 = 0.0f;
    if (p < 0 || p >= n_ctx) {
      if (status) *status = 1;
    } else {
      const float c = cos_tab[static_cast<int64_t>(p) * hd + j];
      const float s = sin_tab[static_cast<int64_t>(p) * hd + j];
      const float a = x0 * c;
      const float b = x1 * s;
      const float e = x0 * s;
      const float f = x1 * c;
      o0 = a - b;
      o1 = e + f;
    }
    ob[static_cast<int64_t>(r) * dim + j] = o0;
    ob[static_cast<int64_t>(r) * dim + j + hd] = o1;
  }
}

// Model-width rows: one wavefront per row, lane-strided double sum (the
// order described above), float4 loads and stores.
__global__ __launch_bounds__(256) void long_row_norm_kernel(const float *__restrict__ x,
                                                            const float *__restrict__ w, float *out,
                                                            int64_t rows, int dim, float eps) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const float4 *xr = reinterpret_cast<const float4 *>(x + row * dim);
  const float scale = ikv::rms_scale_strided(xr, dim, eps, lane);
  const float4 *w4 = reinterpret_cast<const float4 *>(w);
  float4 *o4 = reinterpret_cast<float4 *>(out + row * dim);
  for (int j = lane; j < dim / 4; j += 64) {
    const float4 v = xr[j];
    const float4 g = w4[j];
    const float a = v.x * scale, b = v.y * scale, c = v.z * scale, d = v.w * scale;
    o4[j] = make_float4(a * g.x, b * g.y, c * g.z, d * g.w);
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
  if (rows > INT64_MAX / dim) return -EOVERFLOW;
  if (long_row(dim) && dim <= INT_MAX && ikv::aligned16(x) && ikv::aligned16(w) &&
      ikv::aligned16(out)) {
    const int64_t blocks = (rows + 3) / 4;
    if (blocks > INT_MAX) return -EOVERFLOW;
    long_row_norm_kernel<<<static_cast<unsigned>(blocks), 256, 0, static_cast<hipStream_t>(stream)>>>(
        x, w, out, rows, static_cast<int>(dim), eps);
    return ikv::launch_status();
  }
  if (dim > kLdsFloats - 1) return -ENOTSUP;
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
