// ikv_common.hpp — helpers shared by the gfx950 kernels and their C-ABI
// wrappers. Written for CDNA4 only: 64-lane wavefronts, 32-lane half-wave
// reductions, float4 (16-byte) global accesses.
#pragma once

#include <hip/hip_runtime.h>

#include <cerrno>
#include <cmath>
#include <cstddef>
#include <climits>
#include <cstdint>

#include "../../include/ikv.h"

namespace ikv {

constexpr int kWave = 64;

// Return code of an entry point after its launches: 0, or the hipError_t of
// the failed launch (positive, as documented in ikv.h).
inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : static_cast<int>(e);
}

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Cross-lane moves on the DPP network (no LDS round trip).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i within 8 lanes
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i within 16 lanes

// Sum over the 32 lanes of a half-wave; every lane of the half gets the sum.
// Four DPP steps build sums over 4, 8 and 16 lanes; one ds_swizzle (xor 16
// inside each 32-lane group, bitmask mode) finishes.
__device__ __forceinline__ float half_wave_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppMirror>(v);
  v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
  return v;
}
// The same sum (the same bits: the last step adds the same two values)
// with the last step on the VALU (v_permlane16_swap) instead of the LDS
// pipe: shorter latency, one more VALU op. Faster in the decode with 2 query
// heads per KV head (ctx 1024 6.76 -> 6.66 us), slower with 4 (ctx 4096
// 11.37 -> 11.46 us), whose scores already keep the VALU busy.
__device__ __forceinline__ float half_wave_sum_valu(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppMirror>(v);
  const auto b =
      __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// The values of x in lanes i % 32 (.x) and 32 + i % 32 (.y), in every lane i:
// one v_permlane32_swap (lanes 32..63 of a copy trade places with lanes
// 0..31 of another), no LDS.
__device__ __forceinline__ float2 halves(float x) {
  const auto a =
      __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return make_float2(__uint_as_float(a[0]), __uint_as_float(a[1]));
}

// Double sums over the lanes of a half-wave / wave on the DPP network and
// the VALU lane swaps (no LDS round trip): the same tree as half_wave_sum
// (pairs, quads, 8, 16, 32 and, for the wave, 64 lanes), each step adding
// the same two values in both partner lanes, so every lane gets the same
// bits.
template <int CTRL>
__device__ __forceinline__ double dpp64(double v) {
  const int2 u = __builtin_bit_cast(int2, v);
  const int lo = __builtin_amdgcn_mov_dpp(u.x, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_mov_dpp(u.y, CTRL, 0xF, 0xF, false);
  return __builtin_bit_cast(double, make_int2(lo, hi));
}
__device__ __forceinline__ double half_wave_sum_f64(double v) {
  v += dpp64<kDppXor1>(v);
  v += dpp64<kDppXor2>(v);
  v += dpp64<kDppHalfMirror>(v);
  v += dpp64<kDppMirror>(v);
  const uint2 u = __builtin_bit_cast(uint2, v);
  const auto lo = __builtin_amdgcn_permlane16_swap(u.x, u.x, false, false);
  const auto hi = __builtin_amdgcn_permlane16_swap(u.y, u.y, false, false);
  return __builtin_bit_cast(double, make_uint2(lo[0], hi[0])) +
         __builtin_bit_cast(double, make_uint2(lo[1], hi[1]));
}
__device__ __forceinline__ double wave_sum_f64(double v) {
  v = half_wave_sum_f64(v);
  const uint2 u = __builtin_bit_cast(uint2, v);
  const auto lo = __builtin_amdgcn_permlane32_swap(u.x, u.x, false, false);
  const auto hi = __builtin_amdgcn_permlane32_swap(u.y, u.y, false, false);
  return __builtin_bit_cast(double, make_uint2(lo[0], hi[0])) +
         __builtin_bit_cast(double, make_uint2(lo[1], hi[1]));
}

// Max / sum over the 64 lanes, every lane getting the result: DPP steps
// over 2, 4, 8 and 16 lanes, then v_permlane16_swap and v_permlane32_swap,
// all on the VALU (an xor butterfly of LDS bpermutes was six round trips).
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppMirror>(v));
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float wave_sum(float v) {
  v = half_wave_sum_valu(v);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// 2^x on the hardware exp unit. Inputs below the float range give +0, and
// -inf gives 0, which is what masked softmax terms need.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// A 4-term dot product as one explicit fma chain: the same rounding in every
// kernel that uses it, whatever the compiler would contract.
__device__ __forceinline__ float dot4(const float4 a, const float4 b) {
  return fmaf(a.w, b.w, fmaf(a.z, b.z, fmaf(a.y, b.y, a.x * b.x)));
}

__device__ __forceinline__ float4 fma4(float s, const float4 v, const float4 acc) {
  return make_float4(fmaf(s, v.x, acc.x), fmaf(s, v.y, acc.y), fmaf(s, v.z, acc.z),
                     fmaf(s, v.w, acc.w));
}

__device__ __forceinline__ float4 scale4(float s, const float4 v) {
  return make_float4(s * v.x, s * v.y, s * v.z, s * v.w);
}

constexpr float kLog2e = 1.4426950408889634f;

// The reference's RMSNorm scale is float(1 / sqrt(S / dim + eps)), S the
// row's float squares summed in double in index order
// (src/backends/cpu_backend.cpp:335-382): a chain of dim dependent double
// adds. A kernel that sums the same squares in another order (in parallel)
// gets S' with |S' - S| <= n_err * 2^-53 * S', n_err the longest chain of
// roundings of the two orders together (dim - 1 for the index order plus the
// other order's). The doubles computed from S and S' by the same four
// correctly rounded operations then differ by at most
// (n_err / 2 + 8) * 2^-53 relative. This returns the float scale from S'
// when every double within 64 times that of its value rounds to the same
// float, which makes it the reference's float bit for bit; it returns false
// (about 2^-16 of rows; also for zero, infinite and NaN values) when the
// caller must sum in index order instead.
__device__ __forceinline__ bool certified_rms_scale(double s_any, int dim, float eps, int n_err,
                                                    float &scale) {
  const double t = 1.0 / sqrt(s_any / static_cast<double>(dim) + static_cast<double>(eps));
  if (!(t > 1e-30) || !(t < 1e30)) return false;
  const float f = static_cast<float>(t);
  const double fd = static_cast<double>(f);
  const unsigned bits = __float_as_uint(f);
  // the float next to f on t's side, and the rounding midpoint between them
  // (exact in double: two adjacent floats)
  const double nb = static_cast<double>(__uint_as_float(t >= fd ? bits + 1u : bits - 1u));
  const double mid = 0.5 * (fd + nb);
  const double rel = (0.5 * n_err + 8.0) * 0x1p-53;
  if (fabs(mid - t) <= 64.0 * rel * t) return false;
  scale = f;
  return true;
}

// The reference's scale from its index-order sum of the row's float squares.
__device__ __forceinline__ float ordered_rms_scale(const float *row, int dim, float eps) {
  double sum = 0.0;
  for (int i = 0; i < dim; ++i) {
    const float x = row[i];
    const float sq = x * x;
    sum += static_cast<double>(sq);
  }
  return static_cast<float>(1.0 / sqrt(sum / static_cast<double>(dim) + static_cast<double>(eps)));
}

// certified_rms_scale for a sum that every lane of the wave holds, else the
// index-order sum by lane 0, broadcast (wave-uniform control flow).
__device__ __forceinline__ float certified_or_ordered_scale(double s_any, const float *row,
                                                            int dim, float eps, int n_err,
                                                            int lane) {
  float scale = 0.f;
  if (certified_rms_scale(s_any, dim, eps, n_err, scale)) return scale;
  float seq = 0.f;
  if (lane == 0) seq = ordered_rms_scale(row, dim, eps);
  return __shfl(seq, 0, 64);
}

// RMSNorm scale float(1 / sqrt(sum/dim + eps)) of a row of dim floats
// (dim % 256 == 0, row 16-byte aligned) for one wavefront, equal to the
// reference's bit for bit: lane l adds in double the float squares of
// elements 256*j + 4*l + c (j ascending, c = 0..3), the 64 lane sums combine
// in wave_sum_f64's tree (every lane gets the same bits), and the
// scale is certified against the index-order sum (certified_rms_scale); when
// it is not certain, lane 0 sums the row in index order (about 9 us for 1024
// floats; rare) and every lane takes that.
__device__ __forceinline__ float rms_scale_strided(const float4 *row, int dim, float eps, int lane) {
  double s = 0.0;
#pragma unroll 4
  for (int j = 0; j < dim / 256; ++j) {
    const float4 v = row[64 * j + lane];
    const float a = v.x * v.x, b = v.y * v.y, c = v.z * v.z, d = v.w * v.w;
    s += static_cast<double>(a);
    s += static_cast<double>(b);
    s += static_cast<double>(c);
    s += static_cast<double>(d);
  }
  s = wave_sum_f64(s);
  return certified_or_ordered_scale(s, reinterpret_cast<const float *>(row), dim, eps,
                                    (dim - 1) + dim / 64 + 5, lane);
}

// ORs an IKV_STATUS_* bit into a caller's device status word (a vector
// atomic; several kernels and error kinds may share one word).
__device__ __forceinline__ void raise_status(int *status, int bit) {
  if (status) atomicOr(status, bit);
}

// A paged KV cache as the kernels see it: logical token t lives in pool row
// table[t / bt] * bt + t % bt (bt a multiple of 64).
struct Pages {
  const int32_t *table = nullptr;
  int bt = 0;
  int n_blocks = 0;
  int *status = nullptr;
};

// Offset that takes logical token t to its pool row (t + shift), shared by
// every token of t's block. A table entry outside [0, n_blocks) maps to block
// 0 (in bounds, for reads) and raises IKV_STATUS_BLOCK. t is uniform across
// the wave, so the entry is one scalar load.
__device__ __forceinline__ int64_t page_shift(const Pages &pg, int t) {
  const int b = t / pg.bt;
  int blk = pg.table[b];
  if (static_cast<unsigned>(blk) >= static_cast<unsigned>(pg.n_blocks)) {
    raise_status(pg.status, IKV_STATUS_BLOCK);
    blk = 0;
  }
  return static_cast<int64_t>(blk - b) * pg.bt;
}

// Whether logical token t's table entry names a pool block: writes to a
// token whose entry does not are dropped.
__device__ __forceinline__ bool page_ok(const Pages &pg, int64_t t) {
  return static_cast<unsigned>(pg.table[t / pg.bt]) < static_cast<unsigned>(pg.n_blocks);
}

// Host check of a paged-cache descriptor: a table, blocks of a positive
// multiple of 64 tokens, pool rows that index in int.
inline int pages_arg(const ikv_kv_pages *p, Pages &out) {
  if (!p || !p->block_table || p->block_tokens <= 0 || p->block_tokens % 64 != 0 ||
      p->n_pool_blocks <= 0)
    return -EINVAL;
  if (p->block_tokens > INT_MAX / p->n_pool_blocks) return -EOVERFLOW;
  out.table = p->block_table;
  out.bt = static_cast<int>(p->block_tokens);
  out.n_blocks = static_cast<int>(p->n_pool_blocks);
  out.status = p->status;
  return 0;
}

}  // namespace ikv
