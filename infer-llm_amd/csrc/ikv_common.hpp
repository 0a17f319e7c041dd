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

__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
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

// RMSNorm scale float(1 / sqrt(sum/dim + eps)) of a row of dim floats
// (dim % 256 == 0, row 16-byte aligned) for one wavefront: lane l adds in
// double, in this order, the float squares of elements 256*j + 4*l + c
// (j ascending, c = 0..3); the 64 lane sums combine in a fixed xor butterfly
// (32, 16, ..., 1), so every lane of every wave gets the same bits.
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
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  return static_cast<float>(1.0 / sqrt(s / static_cast<double>(dim) + static_cast<double>(eps)));
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
