// attn_generic.hip — causal GQA attention for the shapes the tuned kernels
// (attn_decode.hip, attn_prefill.hip: head_dim 128, query groups of 1, 2, 4
// or 8) do not take: any head_dim up to kGenericMaxDim and any ratio of query
// to KV heads, contiguous or paged caches. The semantics are
// CPUBackend::compute_flash_attn's (src/backends/cpu_backend.cpp:525-634):
// key j is visible to query t iff j <= n_past + t and j < n_kv; q head h
// reads KV head h / (n_head / n_head_kv).
//
// One 64-lane workgroup per (query token, query head): the query row is
// staged in LDS; keys go 64 at a time, one per lane, each lane forming its
// key's score in a sequential loop over the row; the wave's online softmax
// (running max and sum, natural exp) rescales the output, whose dims lane,
// lane + 64, ... each lane owns, and every key's weight then multiplies its V
// row. It is simple rather than fast: a correct path for models whose heads
// the MFMA kernels were not built for.
#include "attn_generic.hpp"
#include "ikv_common.hpp"

#include <climits>

namespace {

constexpr int kMaxDim = ikv::kGenericMaxDim;
constexpr int kOut = kMaxDim / 64;  // output dims per lane

// Pool row of logical key j (per lane): table[j / bt] * bt + j % bt; an entry
// outside the pool reads block 0 and raises IKV_STATUS_BLOCK.
__device__ __forceinline__ int64_t key_row(const ikv::Pages &pg, bool paged, int j) {
  if (!paged) return j;
  const int b = j / pg.bt;
  int blk = pg.table[b];
  if (static_cast<unsigned>(blk) >= static_cast<unsigned>(pg.n_blocks)) {
    ikv::raise_status(pg.status, IKV_STATUS_BLOCK);
    blk = 0;
  }
  return static_cast<int64_t>(blk) * pg.bt + (j - b * pg.bt);
}

__global__ __launch_bounds__(64) void attn_generic_kernel(const float *__restrict__ q,
                                                          const float *__restrict__ k,
                                                          const float *__restrict__ v,
                                                          float *__restrict__ out, int n_head,
                                                          int n_head_kv, int dim, int n_kv,
                                                          int n_past, float scale, bool paged,
                                                          ikv::Pages pg) {
  __shared__ float s_q[kMaxDim];
  __shared__ float s_p[64];
  __shared__ int64_t s_row[64];
  const int t = static_cast<int>(blockIdx.x) / n_head;
  const int h = static_cast<int>(blockIdx.x) - t * n_head;
  const int g = h / (n_head / n_head_kv);
  const int lane = threadIdx.x;
  const float *qr = q + (static_cast<size_t>(t) * n_head + h) * dim;
  for (int d = lane; d < dim; d += 64) s_q[d] = qr[d];
  __syncthreads();

  const size_t tok_stride = static_cast<size_t>(n_head_kv) * dim;
  const size_t head_off = static_cast<size_t>(g) * dim;
  const int kv_end = min(n_kv, n_past + t + 1);
  float o[kOut];
#pragma unroll
  for (int i = 0; i < kOut; ++i) o[i] = 0.f;
  float m = -INFINITY, l = 0.f;
  for (int base = 0; base < kv_end; base += 64) {
    const int j = base + lane;
    const bool valid = j < kv_end;
    const int64_t row = key_row(pg, paged, valid ? j : base);
    float sc = -INFINITY;
    if (valid) {
      const float *kr = k + row * tok_stride + head_off;
      float acc = 0.f;
      for (int d = 0; d < dim; ++d) acc = fmaf(s_q[d], kr[d], acc);
      sc = acc * scale;
    }
    const float m_new = fmaxf(m, ikv::wave_max(sc));  // finite: lane 0's key is valid
    const float alpha = expf(m - m_new);              // 0 on the first chunk (m = -inf)
    const float p = valid ? expf(sc - m_new) : 0.f;
    l = l * alpha + ikv::wave_sum(p);
#pragma unroll
    for (int i = 0; i < kOut; ++i) o[i] *= alpha;
    s_p[lane] = p;
    s_row[lane] = row;
    __syncthreads();
    const int n = min(64, kv_end - base);
    for (int jj = 0; jj < n; ++jj) {
      const float pj = s_p[jj];
      const float *vr = v + s_row[jj] * tok_stride + head_off;
#pragma unroll
      for (int i = 0; i < kOut; ++i) {
        const int d = lane + 64 * i;
        if (d < dim) o[i] = fmaf(pj, vr[d], o[i]);
      }
    }
    __syncthreads();
    m = m_new;
  }
  float *orow = out + (static_cast<size_t>(t) * n_head + h) * dim;
#pragma unroll
  for (int i = 0; i < kOut; ++i) {
    const int d = lane + 64 * i;
    if (d < dim) orow[d] = o[i] / l;
  }
}

}  // namespace

namespace ikv {

bool generic_attn_shape(int n_head, int n_head_kv, int head_dim) {
  return n_head > 0 && n_head_kv > 0 && n_head % n_head_kv == 0 && head_dim >= 1 &&
         head_dim <= kGenericMaxDim;
}

int attn_generic(const float *q, const float *k, const float *v, const Pages *pages, float *out,
                 int n_head, int n_head_kv, int head_dim, int64_t n_q, int64_t n_kv,
                 int64_t n_past, float scale, hipStream_t s) {
  if (n_q == 0) return 0;
  if (!generic_attn_shape(n_head, n_head_kv, head_dim)) return -ENOTSUP;
  if (n_q < 0 || n_kv <= 0 || n_past < 0) return -EINVAL;
  if (n_q > INT_MAX / n_head || n_kv > INT_MAX / 2 || n_past > INT_MAX / 2) return -EOVERFLOW;
  if (!(scale > 0.0f)) scale = 1.0f / sqrtf(static_cast<float>(head_dim));
  attn_generic_kernel<<<static_cast<unsigned>(n_q * n_head), 64, 0, s>>>(
      q, k, v, out, n_head, n_head_kv, head_dim, static_cast<int>(n_kv),
      static_cast<int>(n_past), scale, pages != nullptr, pages ? *pages : Pages{});
  return launch_status();
}

}  // namespace ikv
