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
// Sums of squares: the reference adds a row's float squares in index order in
// double, a chain of dim dependent double adds (about 1.1 us for 128 on
// MI355X). The kernels add them in parallel instead and certify the float
// scale against the index-order sum (ikv::certified_rms_scale): the two sums
// differ by a bounded amount, and when the double scale is farther than that
// from a float rounding midpoint, both round to the same float. When it is
// not (about 2^-16 of rows), one lane redoes the sum in index order. Every
// scale is therefore the reference's bit for bit.
//  * rows shorter than kLongRow (the head_dim rows of qk-norm): half-wave per
//    row, lane c adds elements c, c + 32, ..., then a xor butterfly;
//  * rows of kLongRow or more floats, a multiple of 256 (the model-width
//    rows of attn_norm / ffn_norm / output_norm): one wavefront per row; lane
//    l adds the squares of elements 256*j + 4*l + c (j ascending,
//    c = 0..3), then the 64 lane sums combine in a xor butterfly
//    (ikv::rms_scale_strided). The GEMV kernels that fold this norm into
//    their input (ikv_model.h) use the same scale.
//
// Short rows: each workgroup is 4 wavefronts owning up to 16 rows. It issues
// all of its row loads at once (coalesced, float4 when aligned) together with
// the positions, norm weights and sin/cos rows of its first RoPE pairs, then
// stages the rows in LDS (row stride dim+1 floats, so the per-lane row walks
// are bank-conflict free); half-wave r sums row r while the RoPE inputs land; then
// every thread takes elements (or RoPE pairs) of the block in turn, so
// weights, sin/cos and outputs move coalesced. A block stages all its rows
// before writing any output, so x == out (in place) is safe.
#pragma clang fp contract(off)

#include "ikv_common.hpp"
#include "../../include/ikv.h"

#include <climits>
#include <vector>

namespace {

constexpr int kLdsFloats = 64 * 129;  // 33 KB: the largest short-row block staged in LDS
constexpr int kLongRow = 512;
constexpr int kRowThreads = 256;     // 4 wavefronts per short-row block
constexpr int kMaxRows = 16;         // rows per short-row block
// Staging registers per thread: every float (or float4) of the largest block.
constexpr int kStage = (kLdsFloats + kRowThreads - 1) / kRowThreads;
constexpr int kStage4 = (kLdsFloats / 4 + kRowThreads - 1) / kRowThreads;
// RoPE pairs per thread whose position, sin/cos and weights are loaded before
// the sums (all of them for head_dim 128); further pairs load afterwards.
constexpr int kPairPF = 4;

int rows_per_block(int dim) {
  int r = kLdsFloats / (dim + 1);
  if (r > kMaxRows) r = kMaxRows;
  if (r < 1) r = 1;
  return r;
}

bool long_row(int64_t dim) { return dim >= kLongRow && dim % 256 == 0; }

// Short rows (head_dim rows of qk-norm and RoPE, rows shorter than kLongRow).
// A block of 4 wavefronts owns up to kMaxRows rows. Every load the block needs
// before its sums is issued at once: the rows (float4 when `vec`), and for
// this thread's first kPairPF RoPE pairs the position, the norm weights and,
// once the position is back, the sin/cos row; those land while lanes
// 0..rows-1 of wavefront 0 run the ordered double sums. All of a block's rows
// are staged in LDS before any output is written, so x == out is safe.
template <bool NORM, bool ROPE>
__global__ __launch_bounds__(kRowThreads) void row_kernel(const float *__restrict__ x,
                                                          const float *__restrict__ w, float *out,
                                                          const int32_t *__restrict__ pos, int64_t rows,
                                                          int dim, int rpb, float eps, int n_heads,
                                                          const float *__restrict__ sin_tab,
                                                          const float *__restrict__ cos_tab,
                                                          int64_t n_ctx, int *status, int vec) {
  extern __shared__ float lds[];
  __shared__ float s_scale[kMaxRows];
  const int tid = threadIdx.x;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * rpb;
  const int64_t left = rows - row0;
  const int nr = static_cast<int>(left < rpb ? left : rpb);
  const int stride = dim + 1;
  const int total = nr * dim;
  const int hd = dim / 2;
  const int n_pairs = ROPE ? nr * hd : 0;
  const float *xb = x + row0 * dim;

  // Stage the rows: all loads first, then the LDS stores.
  if (vec) {
    const float4 *xb4 = reinterpret_cast<const float4 *>(xb);
    const int total4 = total >> 2;
    float4 v[kStage4];
#pragma unroll
    for (int k = 0; k < kStage4; ++k) {
      const int i = tid + k * kRowThreads;
      if (i < total4) v[k] = xb4[i];
    }
#pragma unroll
    for (int k = 0; k < kStage4; ++k) {
      const int i = tid + k * kRowThreads;
      if (i < total4) {
        const int e = 4 * i;  // dim % 4 == 0: the four floats share a row
        const int r = e / dim;
        float *d = &lds[r * stride + (e - r * dim)];
        d[0] = v[k].x;
        d[1] = v[k].y;
        d[2] = v[k].z;
        d[3] = v[k].w;
      }
    }
  } else {
    float v[kStage];
#pragma unroll
    for (int k = 0; k < kStage; ++k) {
      const int i = tid + k * kRowThreads;
      if (i < total) v[k] = xb[i];
    }
#pragma unroll
    for (int k = 0; k < kStage; ++k) {
      const int i = tid + k * kRowThreads;
      if (i < total) {
        const int r = i / dim;
        lds[r * stride + (i - r * dim)] = v[k];
      }
    }
  }

  // RoPE inputs of this thread's first pairs, in flight during the sums.
  int32_t pp[kPairPF];
  float w0[kPairPF], w1[kPairPF], cs[kPairPF], sn[kPairPF];
  if constexpr (ROPE) {
#pragma unroll
    for (int k = 0; k < kPairPF; ++k) {
      const int i = tid + k * kRowThreads;
      pp[k] = -1;
      if (i < n_pairs) {
        const int r = i / hd;
        const int j = i - r * hd;
        pp[k] = pos[(row0 + r) / n_heads];
        if (NORM) {
          w0[k] = w[j];
          w1[k] = w[j + hd];
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kPairPF; ++k) {
      const int i = tid + k * kRowThreads;
      cs[k] = 0.0f;
      sn[k] = 0.0f;
      if (i < n_pairs && pp[k] >= 0 && pp[k] < n_ctx) {
        const int j = i - (i / hd) * hd;
        cs[k] = cos_tab[static_cast<int64_t>(pp[k]) * hd + j];
        sn[k] = sin_tab[static_cast<int64_t>(pp[k]) * hd + j];
      }
    }
  }
  __syncthreads();

  if (NORM) {
    // Row r's sum by half-wave r % 8 (rows r and r + 8 for 16 rows): lane c
    // adds the squares of elements c, c + 32, ... in double, a xor butterfly
    // adds the lanes, and the scale is certified against the reference's
    // index-order sum; lane 0 sums in index order when it is not certain.
    // The index-order sum alone is a chain of dim dependent double adds
    // (about 1.1 us for 128).
    const int hw = tid >> 5;
    const int c = tid & 31;
    for (int r = hw; r < nr; r += kRowThreads / 32) {
      const float *rp = &lds[r * stride];
      double part = 0.0;
      for (int i = c; i < dim; i += 32) {
        const float xv = rp[i];
        const float sq = xv * xv;
        part += static_cast<double>(sq);
      }
      part = ikv::half_wave_sum_f64(part);
      float sc = 0.f;
      const bool certain =
          ikv::certified_rms_scale(part, dim, eps, (dim - 1) + (dim + 31) / 32 + 4, sc);
      if (c == 0) s_scale[r] = certain ? sc : ikv::ordered_rms_scale(rp, dim, eps);
    }
  }
  __syncthreads();

  float *ob = out + row0 * dim;
  if (!ROPE) {
    for (int i = tid; i < total; i += kRowThreads) {
      const int r = i / dim;
      const int c = i - r * dim;
      const float t = lds[r * stride + c] * s_scale[r];
      ob[i] = t * w[c];
    }
    return;
  }
  // One pair: x0 = x[j], x1 = x[j + hd] (normed first when NORM), rotated by
  // the angle of its token's position; a position outside the table gives a
  // zero pair and raises *status.
  auto rotate = [&](int i, int32_t p, float wa, float wb, float c, float s) {
    const int r = i / hd;
    const int j = i - r * hd;
    float x0 = lds[r * stride + j];
    float x1 = lds[r * stride + j + hd];
    if (NORM) {
      const float sc = s_scale[r];
      const float t0 = x0 * sc;
      const float t1 = x1 * sc;
      x0 = t0 * wa;
      x1 = t1 * wb;
    }
    float o0 = 0.0f, o1 = 0.0f;
    if (p < 0 || p >= n_ctx) {
      ikv::raise_status(status, IKV_STATUS_POSITION);
    } else {
      const float a = x0 * c;
      const float b = x1 * s;
      const float e = x0 * s;
      const float f = x1 * c;
      o0 = a - b;
      o1 = e + f;
    }
    ob[static_cast<int64_t>(r) * dim + j] = o0;
    ob[static_cast<int64_t>(r) * dim + j + hd] = o1;
  };
#pragma unroll
  for (int k = 0; k < kPairPF; ++k) {
    const int i = tid + k * kRowThreads;
    if (i < n_pairs) rotate(i, pp[k], NORM ? w0[k] : 0.0f, NORM ? w1[k] : 0.0f, cs[k], sn[k]);
  }
  for (int i = tid + kPairPF * kRowThreads; i < n_pairs; i += kRowThreads) {
    const int r = i / hd;
    const int j = i - r * hd;
    const int32_t p = pos[(row0 + r) / n_heads];
    const bool ok = p >= 0 && p < n_ctx;
    const float c = ok ? cos_tab[static_cast<int64_t>(p) * hd + j] : 0.0f;
    const float s = ok ? sin_tab[static_cast<int64_t>(p) * hd + j] : 0.0f;
    rotate(i, p, NORM ? w[j] : 0.0f, NORM ? w[j + hd] : 0.0f, c, s);
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
  // float4 staging needs 16-byte rows: dim % 4 == 0 and x 16-byte aligned.
  const int vec = (dim % 4 == 0 && ikv::aligned16(x)) ? 1 : 0;
  row_kernel<NORM, ROPE><<<static_cast<unsigned>(blocks), kRowThreads, shmem,
                           static_cast<hipStream_t>(stream)>>>(
      x, w, out, pos, rows, dim, rpb, eps, n_heads, sin_tab, cos_tab, n_ctx, status, vec);
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

extern "C" int ikv_rope_theta_table_f32(float theta_base, int head_dim, int64_t n_ctx,
                                        float *theta_host) {
  if (head_dim <= 0 || (head_dim & 1) || n_ctx < 0) return -EINVAL;
  if (n_ctx == 0) return 0;
  if (!theta_host) return -EINVAL;
  const int half = head_dim / 2;
  // the exponent 2i/d and the reciprocal power are float operations (the
  // reference's float arguments to std::pow select powf); the angle is the
  // position times the widened frequency, rounded once to float
  std::vector<double> freq(static_cast<size_t>(half));
  for (int i = 0; i < half; ++i) {
    const float e = (2.0f * static_cast<float>(i)) / static_cast<float>(head_dim);
    freq[static_cast<size_t>(i)] = static_cast<double>(1.0f / powf(theta_base, e));
  }
  for (int64_t pos = 0; pos < n_ctx; ++pos) {
    float *row = theta_host + pos * half;
    for (int i = 0; i < half; ++i)
      row[i] = static_cast<float>(static_cast<double>(pos) * freq[static_cast<size_t>(i)]);
  }
  return 0;
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
