// coherent.hpp — stores and loads that pass data between the workgroups of
// one launch on gfx950, coherent across the XCDs of the device (agent
// scope): the stores are performed at the device's coherence point and the
// loads (sc1) read from it, so no L2 writeback or invalidate is needed on
// either side. A writer waits for its stores (s_waitcnt) before it counts
// itself on an agent-scope atomic; the workgroup that sees the last count
// then loads what the others stored.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

namespace ikv {

constexpr int kBufWord3 = 0x00020000;  // raw dword buffer, gfx9 family
constexpr int kCpolSc1 = 16;           // cache policy: agent scope
typedef float f2v __attribute__((ext_vector_type(2)));
typedef float f4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void store_agent(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A pair of floats as one 8-byte store.
__device__ __forceinline__ void store2_agent(float *p, float a, float b) {
  const unsigned long long u = static_cast<unsigned long long>(__float_as_uint(a)) |
                               (static_cast<unsigned long long>(__float_as_uint(b)) << 32);
  __hip_atomic_store(reinterpret_cast<unsigned long long *>(p), u, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// 8- and 16-byte loads and 16-byte stores through a buffer resource over a
// workspace (raw buffer: loads past num_records return zeros).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t partial_rsrc(const float *base, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), 0,
                                           static_cast<int>(bytes), kBufWord3);
}
__device__ __forceinline__ float2 load2_agent(__amdgpu_buffer_rsrc_t r, unsigned byte_off) {
  const f2v v = __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, kCpolSc1);
  return make_float2(v.x, v.y);
}
__device__ __forceinline__ float4 load4_agent(__amdgpu_buffer_rsrc_t r, unsigned byte_off) {
  const f4v v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCpolSc1);
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store4_agent(__amdgpu_buffer_rsrc_t r, unsigned byte_off,
                                             float4 v) {
  const f4v x = {v.x, v.y, v.z, v.w};
  __builtin_amdgcn_raw_buffer_store_b128(x, r, byte_off, 0, kCpolSc1);
}
// One float stored by another workgroup of this launch (on any XCD) before
// it was counted.
__device__ __forceinline__ float load_agent(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace ikv
