// gemv_dev.hpp — device code of the weight-streaming matrix-vector products
// (gemv.hip), shared with the kernels that fold a projection into a larger
// launch (attn_decode.hip). See gemv.hip for the design.
#pragma once

#include "ikv_common.hpp"

namespace ikv {
namespace gemv {

constexpr int kBatch = 4;                // float4 loads per lane per row per batch
constexpr int kBatchCols = kBatch * 256; // 1024 columns

typedef float f4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 nt_load4(const float *p) {
  const f4v v = __builtin_nontemporal_load(reinterpret_cast<const f4v *>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}

// Sum over the 64 lanes, every lane getting it: the half-wave sums end on
// v_permlane16_swap and the halves meet on v_permlane32_swap, all on the
// VALU (an LDS-pipe swizzle and bpermute had two round trips of latency at
// the end of every row); the same adds of the same values as the index-
// order tree, so the same bits.
__device__ __forceinline__ float wave_sum64(float v) {
  v = ikv::half_wave_sum_valu(v);
  const auto a =
      __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}

// x[k] * scale * nw[k] for a float4 of x: the standalone RMSNorm's
// (x * scale) * w, two roundings.
__device__ __forceinline__ float4 normed(float4 v, float scale, float4 g) {
  const float a = v.x * scale, b = v.y * scale, c = v.z * scale, d = v.w * scale;
  return make_float4(a * g.x, b * g.y, c * g.z, d * g.w);
}

// ikv::rms_scale_strided(row, dim, eps, lane) with the lane's first kBatch
// float4 reads (row[64 j + lane], j < kBatch) already in first: the same adds
// in the same order, so the same scale bit for bit.
__device__ __forceinline__ float rms_scale_from_first(const float4 (&first)[kBatch], const float4 *row,
                                                      int dim, float eps, int lane) {
  double s = 0.0;
#pragma unroll
  for (int j = 0; j < kBatch; ++j) {
    const float4 v = first[j];
    const float a = v.x * v.x, b = v.y * v.y, c = v.z * v.z, d = v.w * v.w;
    s += static_cast<double>(a);
    s += static_cast<double>(b);
    s += static_cast<double>(c);
    s += static_cast<double>(d);
  }
#pragma unroll 4
  for (int j = kBatch; j < dim / 256; ++j) {
    const float4 v = row[64 * j + lane];
    const float a = v.x * v.x, b = v.y * v.y, c = v.z * v.z, d = v.w * v.w;
    s += static_cast<double>(a);
    s += static_cast<double>(b);
    s += static_cast<double>(c);
    s += static_cast<double>(d);
  }
  s = ikv::wave_sum_f64(s);
  return ikv::certified_or_ordered_scale(s, reinterpret_cast<const float *>(row), dim, eps,
                                         (dim - 1) + dim / 64 + 5, lane);
}

// Sums of NR rows (row r at rows[r], K columns, K % 1024 == 0) dotted with
// x (RMS-normalised with weight nw when nw is not null); every lane gets the
// sums.
template <int NR>
__device__ __forceinline__ void wave_dots(const float *const (&rows)[NR], const float *x, int K,
                                          float (&out)[NR], const float *nw = nullptr,
                                          float eps = 0.f) {
  const int lane = threadIdx.x & 63;
  float4 cur[NR][kBatch], nxt[NR][kBatch];
  float4 acc[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    acc[r] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < kBatch; ++j) cur[r][j] = nt_load4(rows[r] + 4 * lane + 256 * j);
  }
  // The first batch of x (and of the norm weights) is loaded once, with the
  // weights: the scale's sum starts from it (lane-strided, these are its
  // first kBatch reads) and the first batch's products use it, so no second
  // L2 round trip follows the scale.
  float4 x0[kBatch], g0[kBatch];
#pragma unroll
  for (int j = 0; j < kBatch; ++j) {
    x0[j] = *reinterpret_cast<const float4 *>(x + 4 * lane + 256 * j);
    if (nw) g0[j] = *reinterpret_cast<const float4 *>(nw + 4 * lane + 256 * j);
  }
  const float scale = nw ? rms_scale_from_first(x0, reinterpret_cast<const float4 *>(x), K, eps, lane)
                         : 1.f;
  for (int k0 = 0; k0 < K; k0 += kBatchCols) {
    const bool more = k0 + kBatchCols < K;
    if (more) {
#pragma unroll
      for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int j = 0; j < kBatch; ++j)
          nxt[r][j] = nt_load4(rows[r] + k0 + kBatchCols + 4 * lane + 256 * j);
    }
    float4 xv[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      xv[j] = k0 == 0 ? x0[j] : *reinterpret_cast<const float4 *>(x + k0 + 4 * lane + 256 * j);
    if (nw) {
#pragma unroll
      for (int j = 0; j < kBatch; ++j)
        xv[j] = normed(xv[j], scale,
                       k0 == 0 ? g0[j] : *reinterpret_cast<const float4 *>(nw + k0 + 4 * lane + 256 * j));
    }
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        acc[r].x = fmaf(cur[r][j].x, xv[j].x, acc[r].x);
        acc[r].y = fmaf(cur[r][j].y, xv[j].y, acc[r].y);
        acc[r].z = fmaf(cur[r][j].z, xv[j].z, acc[r].z);
        acc[r].w = fmaf(cur[r][j].w, xv[j].w, acc[r].w);
      }
    if (more) {
#pragma unroll
      for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int j = 0; j < kBatch; ++j) cur[r][j] = nxt[r][j];
    }
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) out[r] = wave_sum64((acc[r].x + acc[r].y) + (acc[r].z + acc[r].w));
}

}  // namespace gemv
}  // namespace ikv
