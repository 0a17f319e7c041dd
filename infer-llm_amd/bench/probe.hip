// probe.hip — bandwidth and launch-cost probes for the benchmark (see
// ikv_bench.h). Not on the KV-cache path: built into libikv_bench.so only.
//
// The streaming-read probe is shaped like the decode kernel so that its time
// is a floor for one launch that reads the same bytes: workgroups of 512
// threads, each owning one contiguous slice of the buffer (as a decode split
// owns a token range), and every lane issuing U independent 16-byte
// non-temporal loads before it uses any, so a workgroup's whole slice is in
// flight at once when it fits U loads per lane.
#include "../csrc/ikv_common.hpp"
#include "ikv_bench.h"

#include <climits>

namespace {

constexpr int kProbeWG = 512;
typedef float f4v __attribute__((ext_vector_type(4)));

template <int U>
__global__ __launch_bounds__(kProbeWG) void read_kernel(const f4v *__restrict__ p, size_t n,
                                                        float *__restrict__ sink) {
  __shared__ float s[kProbeWG / 64];
  const size_t per = (n + gridDim.x - 1) / gridDim.x;
  const size_t lo = static_cast<size_t>(blockIdx.x) * per;
  const size_t hi = lo + per < n ? lo + per : n;
  float acc = 0.f;
  for (size_t i = lo + threadIdx.x; i < hi; i += static_cast<size_t>(kProbeWG) * U) {
    f4v v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t j = i + static_cast<size_t>(u) * kProbeWG;
      v[u] = j < hi ? __builtin_nontemporal_load(p + j) : f4v{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc += (v[u].x + v[u].y) + (v[u].z + v[u].w);
  }
  acc = ikv::wave_sum(acc);
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int k = 0; k < kProbeWG / 64; ++k) t += s[k];
    sink[blockIdx.x] = t;
  }
}

__global__ void empty_kernel() {}

}  // namespace

extern "C" int ikv_probe_read(const void *src, size_t bytes, float *sink, int grid,
                              int loads_per_lane, void *stream) {
  if (!src || !sink || grid <= 0 || (bytes & 15u) || !ikv::aligned16(src)) return -EINVAL;
  const f4v *p = static_cast<const f4v *>(src);
  const size_t n = bytes / 16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (loads_per_lane) {
    case 1: read_kernel<1><<<grid, kProbeWG, 0, s>>>(p, n, sink); break;
    case 4: read_kernel<4><<<grid, kProbeWG, 0, s>>>(p, n, sink); break;
    case 8: read_kernel<8><<<grid, kProbeWG, 0, s>>>(p, n, sink); break;
    case 16: read_kernel<16><<<grid, kProbeWG, 0, s>>>(p, n, sink); break;
    default: return -EINVAL;
  }
  return ikv::launch_status();
}

extern "C" int ikv_probe_empty(int grid, void *stream) {
  if (grid <= 0) return -EINVAL;
  empty_kernel<<<grid, 64, 0, static_cast<hipStream_t>(stream)>>>();
  return ikv::launch_status();
}
