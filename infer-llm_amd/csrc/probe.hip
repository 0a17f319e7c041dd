// probe.hip — bandwidth and launch-cost probes for the benchmark (see
// include/ikv_probe.h). Not on the KV-cache path.
#include "ikv_common.hpp"
#include "../../include/ikv_probe.h"

#include <climits>

namespace {

__global__ __launch_bounds__(256) void read_kernel(const float4 *__restrict__ p, size_t n,
                                                   float *__restrict__ sink) {
  __shared__ float s[256];
  float acc = 0.f;
  const size_t stride = static_cast<size_t>(gridDim.x) * 256;
  for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) {
    const float4 v = p[i];
    acc += (v.x + v.y) + (v.z + v.w);
  }
  s[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int k = 0; k < 256; ++k) t += s[k];
    sink[blockIdx.x] = t;
  }
}

__global__ void empty_kernel() {}

}  // namespace

extern "C" int ikv_probe_read(const void *src, size_t bytes, float *sink, int grid, void *stream) {
  if (!src || !sink || grid <= 0 || (bytes & 15u) || !ikv::aligned16(src)) return -EINVAL;
  read_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(static_cast<const float4 *>(src),
                                                                  bytes / 16, sink);
  return ikv::launch_status();
}

extern "C" int ikv_probe_empty(int grid, void *stream) {
  if (grid <= 0) return -EINVAL;
  empty_kernel<<<grid, 64, 0, static_cast<hipStream_t>(stream)>>>();
  return ikv::launch_status();
}
