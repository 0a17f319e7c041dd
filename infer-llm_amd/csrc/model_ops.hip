// model_ops.hip — the small ops of a Qwen3 step around the KV-cache path:
// token-embedding gather, elementwise add / mul / silu, and greedy sampling
// on the device.
//
//   get_rows  CPUBackend::compute_get_rows (src/backends/cpu_backend.cpp:
//             259-332): one workgroup per index copies a table row with
//             16-byte accesses; an out-of-range id writes zeros and raises a
//             status flag instead of reading outside the table.
//   add/mul/silu  src/backends/cpu_backend.cpp:636-703: grid-stride float4;
//             silu_mul = up * silu(gate), the SILU then MUL pair in one pass.
//   argmax    sample_greedy (src/sampler.cpp:42-65): one workgroup of 1024
//             threads scans the logits (16-byte loads, 8 in flight per
//             lane), keeps (max, lowest index) per lane, and reduces through
//             shuffles and LDS; NaN or +inf anywhere, or no finite maximum,
//             gives -1. The workspace form splits the scan over up to 64
//             workgroups and merges their pairs in the last one to arrive.
#include <climits>

#include "ikv_common.hpp"
#include "../../include/ikv_model.h"

namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void get_rows_kernel(const float *__restrict__ table,
                                                            const int32_t *__restrict__ ids,
                                                            float *__restrict__ out, int64_t row_len,
                                                            int64_t n_rows, int *status, int vec) {
  const int64_t i = blockIdx.x;
  const int32_t id = ids[i];
  float *dst = out + i * row_len;
  const bool ok = id >= 0 && id < n_rows;
  if (!ok && threadIdx.x == 0) ikv::raise_status(status, IKV_STATUS_TOKEN);
  const float *src = table + static_cast<int64_t>(ok ? id : 0) * row_len;
  if (vec) {
    for (int64_t c = threadIdx.x; c < row_len / 4; c += kThreads) {
      const float4 v = ok ? reinterpret_cast<const float4 *>(src)[c] : make_float4(0.f, 0.f, 0.f, 0.f);
      reinterpret_cast<float4 *>(dst)[c] = v;
    }
  } else {
    for (int64_t c = threadIdx.x; c < row_len; c += kThreads) dst[c] = ok ? src[c] : 0.f;
  }
}

enum class Ew { kAdd, kMul, kSilu, kSiluMul };

template <Ew OP>
__device__ __forceinline__ float ew(float a, float b) {
  if constexpr (OP == Ew::kAdd) return a + b;
  else if constexpr (OP == Ew::kMul) return a * b;
  else if constexpr (OP == Ew::kSilu) return a / (1.0f + expf(-a));
  else {  // b * silu(a): the silu value is rounded to float, then multiplied
    const float g = a / (1.0f + expf(-a));
    return b * g;
  }
}

template <Ew OP>
__global__ __launch_bounds__(kThreads) void elementwise_kernel(const float *a, const float *b,
                                                               float *out, int64_t n, int vec) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (vec) {
    const int64_t n4 = n / 4;
    for (int64_t j = i; j < n4; j += stride) {
      const float4 x = reinterpret_cast<const float4 *>(a)[j];
      const float4 y = b ? reinterpret_cast<const float4 *>(b)[j] : make_float4(0.f, 0.f, 0.f, 0.f);
      reinterpret_cast<float4 *>(out)[j] =
          make_float4(ew<OP>(x.x, y.x), ew<OP>(x.y, y.y), ew<OP>(x.z, y.z), ew<OP>(x.w, y.w));
    }
    for (int64_t j = 4 * n4 + i; j < n; j += stride) out[j] = ew<OP>(a[j], b ? b[j] : 0.f);
  } else {
    for (int64_t j = i; j < n; j += stride) out[j] = ew<OP>(a[j], b ? b[j] : 0.f);
  }
}

template <Ew OP>
int launch_ew(const float *a, const float *b, float *out, int64_t n, void *stream) {
  if (!a || !out || (OP != Ew::kSilu && !b)) return -EINVAL;
  if (n < 0) return -EINVAL;
  if (n == 0) return 0;
  const bool vec = ikv::aligned16(a) && ikv::aligned16(out) && (!b || ikv::aligned16(b));
  const int64_t work = vec ? (n + 3) / 4 : n;
  int64_t blocks = (work + kThreads - 1) / kThreads;
  if (blocks > 4096) blocks = 4096;
  elementwise_kernel<OP><<<static_cast<int>(blocks), kThreads, 0, static_cast<hipStream_t>(stream)>>>(
      a, b, out, n, vec ? 1 : 0);
  return ikv::launch_status();
}

constexpr int kArgThreads = 1024;
constexpr int kArgBatch = 8;  // float4 loads in flight per lane

// (value, index) pair order of the greedy sampler: larger value wins, equal
// values go to the lower index.
__device__ __forceinline__ void better(float &v, int &i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

__device__ __forceinline__ void visit(float x, int idx, float &best, int &bi, int &bad) {
  if (x != x || x == INFINITY) bad = 1;
  if (x > best) {  // strictly greater: the first (lowest) index of a tie stays
    best = x;
    bi = idx;
  }
}

__global__ __launch_bounds__(kArgThreads) void argmax_kernel(const float *__restrict__ logits,
                                                             int n, int32_t *token,
                                                             int32_t *mirror, int vec) {
  __shared__ float s_v[kArgThreads / 64];
  __shared__ int s_i[kArgThreads / 64];
  __shared__ int s_bad;
  const int tid = threadIdx.x;
  if (tid == 0) s_bad = 0;
  float best = -INFINITY;
  int bi = INT_MAX;
  int bad = 0;
  if (vec) {
    // Lane t reads float4 t, t + 1024, ...: its indices increase. Batches of
    // kArgBatch loads are issued together, then visited in index order.
    const int n4 = n / 4;
    for (int j0 = tid; j0 < n4; j0 += kArgBatch * kArgThreads) {
      float4 v[kArgBatch];
#pragma unroll
      for (int u = 0; u < kArgBatch; ++u) {
        const int j = j0 + u * kArgThreads;
        v[u] = j < n4 ? reinterpret_cast<const float4 *>(logits)[j]
                      : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      }
#pragma unroll
      for (int u = 0; u < kArgBatch; ++u) {
        const int j = j0 + u * kArgThreads;
        visit(v[u].x, 4 * j, best, bi, bad);
        visit(v[u].y, 4 * j + 1, best, bi, bad);
        visit(v[u].z, 4 * j + 2, best, bi, bad);
        visit(v[u].w, 4 * j + 3, best, bi, bad);
      }
    }
    for (int j = 4 * n4 + tid; j < n; j += kArgThreads) visit(logits[j], j, best, bi, bad);
  } else {
    for (int j = tid; j < n; j += kArgThreads) visit(logits[j], j, best, bi, bad);
  }
  __syncthreads();
  if (bad) s_bad = 1;  // benign race: every writer stores 1
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    better(best, bi, ov, oi);
  }
  if ((tid & 63) == 0) {
    s_v[tid >> 6] = best;
    s_i[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    float v = s_v[0];
    int i = s_i[0];
    for (int w = 1; w < kArgThreads / 64; ++w) better(v, i, s_v[w], s_i[w]);
    const int32_t t = (s_bad || v == -INFINITY || i == INT_MAX) ? -1 : i;
    *token = t;
    if (mirror) *mirror = t;
  }
}

// The workspace form: up to kArgWgs workgroups each reduce a contiguous,
// index-ordered slice of the logits to (max, lowest index), publish it with
// an agent-coherent 8-byte store (a NaN value marks a slice that held a NaN
// or +inf) and count themselves in the workspace's arrival counter; the
// workgroup that arrives last reduces the published pairs in slice order,
// writes the token and resets the counter. The pair order is the sampler's
// (larger value, then lower index), so the result is the single-workgroup
// scan's bit for bit; a single workgroup streams only ~50 GB/s, which made
// that scan 14 us for 151936 logits.
constexpr int kArgWgs = 64;
constexpr int kArgWgThreads = 256;
constexpr int kArgWgBatch = 4;       // float4 loads in flight per lane
constexpr size_t kArgWsCounter = 256;  // counter, then kArgWgs 8-byte pairs

__global__ __launch_bounds__(kArgWgThreads) void argmax_ws_kernel(const float *__restrict__ logits,
                                                                  int n, int32_t *token,
                                                                  int32_t *mirror, int vec,
                                                                  int *counter,
                                                                  unsigned long long *pairs) {
  __shared__ float s_v[kArgWgThreads / 64];
  __shared__ int s_i[kArgWgThreads / 64];
  __shared__ int s_bad;
  __shared__ int s_last;
  const int tid = threadIdx.x;
  const int wg = blockIdx.x;
  const int wgs = gridDim.x;
  if (tid == 0) s_bad = 0;
  float best = -INFINITY;
  int bi = INT_MAX;
  int bad = 0;
  const int units = vec ? n / 4 : n;  // float4s (vec) or floats
  const int per = (units + wgs - 1) / wgs;
  const int lo = min(units, wg * per);
  const int hi = min(units, lo + per);
  if (vec) {
    for (int j0 = lo + tid; j0 < hi; j0 += kArgWgBatch * kArgWgThreads) {
      float4 v[kArgWgBatch];
#pragma unroll
      for (int u = 0; u < kArgWgBatch; ++u) {
        const int j = j0 + u * kArgWgThreads;
        v[u] = j < hi ? reinterpret_cast<const float4 *>(logits)[j]
                      : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      }
#pragma unroll
      for (int u = 0; u < kArgWgBatch; ++u) {
        const int j = j0 + u * kArgWgThreads;
        visit(v[u].x, 4 * j, best, bi, bad);
        visit(v[u].y, 4 * j + 1, best, bi, bad);
        visit(v[u].z, 4 * j + 2, best, bi, bad);
        visit(v[u].w, 4 * j + 3, best, bi, bad);
      }
    }
    if (wg == wgs - 1)  // the n % 4 floats after the last float4
      for (int j = 4 * units + tid; j < n; j += kArgWgThreads) visit(logits[j], j, best, bi, bad);
  } else {
    for (int j = lo + tid; j < hi; j += kArgWgThreads) visit(logits[j], j, best, bi, bad);
  }
  __syncthreads();
  if (bad) s_bad = 1;  // benign race: every writer stores 1
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    better(best, bi, ov, oi);
  }
  if ((tid & 63) == 0) {
    s_v[tid >> 6] = best;
    s_i[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    float v = s_v[0];
    int i = s_i[0];
    for (int w = 1; w < kArgWgThreads / 64; ++w) better(v, i, s_v[w], s_i[w]);
    if (s_bad) v = __int_as_float(0x7fc00000);  // NaN: this slice held a NaN or +inf
    const unsigned long long pair = static_cast<unsigned long long>(__float_as_uint(v)) |
                                    (static_cast<unsigned long long>(static_cast<unsigned>(i)) << 32);
    __hip_atomic_store(pairs + wg, pair, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // the pair's store has completed (vmcnt counts stores) before the arrival
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const int before = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = before == wgs - 1;
    if (s_last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last || tid >= 64) return;
  float v = -INFINITY;
  int i = INT_MAX;
  int nan = 0;
  if (tid < wgs) {
    const unsigned long long pair =
        __hip_atomic_load(pairs + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    v = __uint_as_float(static_cast<unsigned>(pair));
    i = static_cast<int>(static_cast<unsigned>(pair >> 32));
    nan = v != v;
    if (nan) v = -INFINITY;
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o, 64);
    const int oi = __shfl_xor(i, o, 64);
    better(v, i, ov, oi);
  }
  const bool any_nan = __builtin_amdgcn_ballot_w64(nan != 0) != 0;
  if (tid == 0) {
    const int32_t t = (any_nan || v == -INFINITY || i == INT_MAX) ? -1 : i;
    *token = t;
    if (mirror) *mirror = t;
  }
}

}  // namespace

extern "C" int ikv_get_rows_f32(const float *table, const int32_t *ids, float *out, int64_t n_ids,
                                int64_t row_len, int64_t n_rows, int *status, void *stream) {
  if (!table || !ids || !out) return -EINVAL;
  if (n_ids < 0 || row_len < 0 || n_rows < 0) return -EINVAL;
  if (n_ids == 0 || row_len == 0) return 0;
  if (n_ids > INT_MAX) return -EOVERFLOW;
  const bool vec = row_len % 4 == 0 && ikv::aligned16(table) && ikv::aligned16(out);
  get_rows_kernel<<<static_cast<int>(n_ids), kThreads, 0, static_cast<hipStream_t>(stream)>>>(
      table, ids, out, row_len, n_rows, status, vec ? 1 : 0);
  return ikv::launch_status();
}

extern "C" int ikv_add_f32(const float *a, const float *b, float *out, int64_t n, void *stream) {
  return launch_ew<Ew::kAdd>(a, b, out, n, stream);
}

extern "C" int ikv_mul_f32(const float *a, const float *b, float *out, int64_t n, void *stream) {
  return launch_ew<Ew::kMul>(a, b, out, n, stream);
}

extern "C" int ikv_silu_f32(const float *x, float *out, int64_t n, void *stream) {
  return launch_ew<Ew::kSilu>(x, nullptr, out, n, stream);
}

extern "C" int ikv_silu_mul_f32(const float *gate, const float *up, float *out, int64_t n,
                                void *stream) {
  return launch_ew<Ew::kSiluMul>(gate, up, out, n, stream);
}

extern "C" int ikv_argmax_f32(const float *logits, int64_t n, int32_t *token,
                              int32_t *token_mirror, void *stream) {
  if (!logits || !token) return -EINVAL;
  if (n < 1) return -EINVAL;
  if (n > INT_MAX - kArgBatch * kArgThreads * 4) return -EOVERFLOW;
  argmax_kernel<<<1, kArgThreads, 0, static_cast<hipStream_t>(stream)>>>(
      logits, static_cast<int>(n), token, token_mirror, ikv::aligned16(logits) ? 1 : 0);
  return ikv::launch_status();
}

extern "C" size_t ikv_argmax_workspace_bytes(void) { return kArgWsCounter + sizeof(unsigned long long) * kArgWgs; }

extern "C" int ikv_argmax_ws_f32(const float *logits, int64_t n, int32_t *token, int32_t *token_mirror,
                                 void *workspace, size_t workspace_bytes, void *stream) {
  if (!logits || !token || !workspace) return -EINVAL;
  if (n < 1) return -EINVAL;
  if (n > INT_MAX - kArgWgBatch * kArgWgThreads * 4) return -EOVERFLOW;
  if (workspace_bytes < ikv_argmax_workspace_bytes() || reinterpret_cast<uintptr_t>(workspace) % 256)
    return -EINVAL;
  const int vec = ikv::aligned16(logits) ? 1 : 0;
  const int64_t units = vec ? n / 4 : n;
  int wgs = static_cast<int>((units + kArgWgThreads - 1) / kArgWgThreads);
  if (wgs < 1) wgs = 1;
  if (wgs > kArgWgs) wgs = kArgWgs;
  auto *ws = static_cast<char *>(workspace);
  argmax_ws_kernel<<<wgs, kArgWgThreads, 0, static_cast<hipStream_t>(stream)>>>(
      logits, static_cast<int>(n), token, token_mirror, vec, reinterpret_cast<int *>(ws),
      reinterpret_cast<unsigned long long *>(ws + kArgWsCounter));
  return ikv::launch_status();
}
