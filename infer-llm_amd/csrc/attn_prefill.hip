// attn_prefill.hip — causal GQA flash attention for n_q >= 1 query tokens on
// F32 MFMA (v_mfma_f32_32x32x2_f32), never materialising the score matrix.
//
// Replaces CUDA_F32::compute_flash_attn for prefill (reference
// src/kernels/cuda/kernel_f32.cu:452-511), which allocated Hq*n_q*n_kv floats
// of scores per call. Semantics: CPUBackend::compute_flash_attn
// (src/backends/cpu_backend.cpp:525-634): key j is visible to query t iff
// j <= n_past + t; q head h reads KV head h / G, G = n_head / n_head_kv.
//
// Decomposition:
//   * A workgroup (4 wavefronts) owns one KV head g and 128 query rows, a row
//     being a (token, q head) pair of that group: 128/G tokens x G heads. The
//     K/V tiles of head g (32 keys x 128 dims each) are staged once in LDS and
//     shared by all G query heads, so K/V are read from HBM once per
//     workgroup, not once per query head.
//   * Each wavefront owns 32 rows and computes in the transposed form
//       S^T = K Q^T   (32 keys x 32 rows, contraction over 128 dims)
//       O^T += V^T P^T (128 dims x 32 rows, contraction over 32 keys)
//     so that every lane holds one query row (lane % 32) in both products:
//     row max / row sum of the online softmax are in-lane plus one exchange
//     between the two half-waves, and the rescale of O^T needs no shuffles.
//   * The contraction order is chosen so operands come straight from
//     registers or 16-byte LDS reads: Q is held in registers (64 floats per
//     lane); each ds_read_b128 of K feeds 4 MFMAs; each ds_read_b128 of V
//     feeds the 4 output tiles, whose rows are the dims 4i+dt.
//   * The next K/V tile is prefetched into registers while the current one is
//     consumed from LDS. Workgroups are issued heaviest query block first.
#include "ikv_common.hpp"
#include "../../include/ikv.h"

#include <climits>

namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int D = 128;
constexpr int NWAVE = 4;
constexpr int WG = NWAVE * 64;
constexpr int ROWS = NWAVE * 32;  // query rows per workgroup
constexpr int BN = 32;            // keys per tile
constexpr int KS = D + 4;         // LDS row stride of K (floats): conflict-free 16-byte reads
constexpr int VS = D;             // LDS row stride of V: each half-wave reads one whole row

__device__ __forceinline__ floatx16 mfma32(float a, float b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <int G>
__global__ __launch_bounds__(WG) void prefill_kernel(const float *__restrict__ q,
                                                     const float *__restrict__ k,
                                                     const float *__restrict__ v,
                                                     float *__restrict__ out, int n_head_kv,
                                                     int n_q, int n_kv, int n_past, int n_qblocks,
                                                     float scale_log2) {
  constexpr int BQ = ROWS / G;  // query tokens per workgroup
  __shared__ float s_k[BN * KS];
  __shared__ float s_v[BN * VS];

  const int g = blockIdx.x % n_head_kv;
  const int qb = n_qblocks - 1 - static_cast<int>(blockIdx.x / n_head_kv);
  const int q0 = qb * BQ;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = lane >> 5;
  const int j = lane & 31;
  const int row = wave * 32 + j;
  const int tok = q0 + row / G;
  const int head = g * G + row % G;
  const int n_head = n_head_kv * G;
  const bool row_ok = tok < n_q;

  // Q row in registers: qr[u] = Q[tok][head][8u + 4*half .. +3].
  float4 qr[16];
  {
    const float *qp = q + (static_cast<size_t>(row_ok ? tok : 0) * n_head + head) * D + 4 * half;
#pragma unroll
    for (int u = 0; u < 16; ++u)
      qr[u] = row_ok ? *reinterpret_cast<const float4 *>(qp + 8 * u) : make_float4(0.f, 0.f, 0.f, 0.f);
  }

  const int last_tok = min(q0 + BQ, n_q) - 1;
  const int k_end = min(n_kv, n_past + last_tok + 1);
  const int n_tiles = (k_end + BN - 1) / BN;

  floatx16 o0 = {}, o1 = {}, o2 = {}, o3 = {};
  float m_row = -INFINITY, l_row = 0.f;

  // Cooperative tile load: 32 keys x 32 float4 per K (and V) tile, 4 per thread.
  float4 pk[4], pv[4];
  auto load_tile = [&](int tile) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + WG * c;
      const int key = idx >> 5;
      const int c4 = idx & 31;
      const int kk = tile * BN + key;
      if (kk < n_kv) {
        const size_t off = (static_cast<size_t>(kk) * n_head_kv + g) * D + 4 * c4;
        pk[c] = *reinterpret_cast<const float4 *>(k + off);
        pv[c] = *reinterpret_cast<const float4 *>(v + off);
      } else {
        pk[c] = make_float4(0.f, 0.f, 0.f, 0.f);
        pv[c] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + WG * c;
      const int key = idx >> 5;
      const int c4 = idx & 31;
      *reinterpret_cast<float4 *>(&s_k[key * KS + 4 * c4]) = pk[c];
      *reinterpret_cast<float4 *>(&s_v[key * VS + 4 * c4]) = pv[c];
    }
  };

  if (n_tiles > 0) load_tile(0);
  for (int tile = 0; tile < n_tiles; ++tile) {
    __syncthreads();
    store_tile();
    __syncthreads();
    if (tile + 1 < n_tiles) load_tile(tile + 1);

    // S^T[key][row] over this tile.
    floatx16 s = {};
    const float *krow = &s_k[j * KS + 4 * half];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const float4 kv = *reinterpret_cast<const float4 *>(krow + 8 * u);
      s = mfma32(kv.x, qr[u].x, s);
      s = mfma32(kv.y, qr[u].y, s);
      s = mfma32(kv.z, qr[u].z, s);
      s = mfma32(kv.w, qr[u].w, s);
    }

    // Register r of lane holds key (r&3) + 4*half + 8*(r>>2) of the tile.
    const int kbase = tile * BN;
    const bool need_mask = (kbase + BN - 1 > n_past + q0) || (kbase + BN > n_kv);
    float mx = m_row;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float sv = s[r] * scale_log2;
      if (need_mask) {
        const int kk = kbase + (r & 3) + 4 * half + 8 * (r >> 2);
        if (kk > n_past + tok || kk >= n_kv) sv = -INFINITY;
      }
      s[r] = sv;
      mx = fmaxf(mx, sv);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float alpha = ikv::fast_exp2(m_row - mx);
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = ikv::fast_exp2(s[r] - mx);
      s[r] = p;
      psum += p;
    }
    psum += __shfl_xor(psum, 32, 64);
    l_row = l_row * alpha + psum;
    m_row = mx;
    o0 *= alpha;
    o1 *= alpha;
    o2 *= alpha;
    o3 *= alpha;

    // O^T[dim 4i+dt][row] += V^T P^T.
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = (r & 3) + 4 * half + 8 * (r >> 2);
      const float4 vv = *reinterpret_cast<const float4 *>(&s_v[key * VS + 4 * j]);
      o0 = mfma32(vv.x, s[r], o0);
      o1 = mfma32(vv.y, s[r], o1);
      o2 = mfma32(vv.z, s[r], o2);
      o3 = mfma32(vv.w, s[r], o3);
    }
  }

  if (row_ok) {
    const float inv = 1.0f / l_row;
    float *op = out + (static_cast<size_t>(tok) * n_head + head) * D;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = (r & 3) + 4 * half + 8 * (r >> 2);
      *reinterpret_cast<float4 *>(op + 4 * i) =
          make_float4(o0[r] * inv, o1[r] * inv, o2[r] * inv, o3[r] * inv);
    }
  }
}

template <int G>
void launch(const float *q, const float *k, const float *v, float *out, int n_head_kv, int n_q,
            int n_kv, int n_past, float scale_log2, hipStream_t s) {
  constexpr int BQ = ROWS / G;
  const int n_qblocks = (n_q + BQ - 1) / BQ;
  prefill_kernel<G><<<n_head_kv * n_qblocks, WG, 0, s>>>(q, k, v, out, n_head_kv, n_q, n_kv,
                                                         n_past, n_qblocks, scale_log2);
}

}  // namespace

extern "C" int ikv_attn_prefill_f32(const float *q, const float *k, const float *v, float *out,
                                    int n_head, int n_head_kv, int head_dim, int64_t n_q,
                                    int64_t n_kv, int64_t n_past, float scale, void *stream) {
  if (n_q == 0) return 0;
  if (!q || !k || !v || !out) return -EINVAL;
  if (n_head <= 0 || n_head_kv <= 0 || n_head % n_head_kv != 0) return -EINVAL;
  if (n_q < 0 || n_kv <= 0 || n_past < 0) return -EINVAL;
  if (head_dim != D) return -ENOTSUP;
  const int G = n_head / n_head_kv;
  if (G != 1 && G != 2 && G != 4 && G != 8) return -ENOTSUP;
  if (n_q > INT_MAX / 2 || n_kv > INT_MAX / 2 || n_past > INT_MAX / 2) return -EOVERFLOW;
  if (!ikv::aligned16(q) || !ikv::aligned16(k) || !ikv::aligned16(v) || !ikv::aligned16(out))
    return -EINVAL;
  if (!(scale > 0.0f)) scale = 1.0f / sqrtf(static_cast<float>(head_dim));
  const float sl2 = scale * ikv::kLog2e;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nq = static_cast<int>(n_q), nk = static_cast<int>(n_kv), np = static_cast<int>(n_past);
  switch (G) {
    case 1: launch<1>(q, k, v, out, n_head_kv, nq, nk, np, sl2, s); break;
    case 2: launch<2>(q, k, v, out, n_head_kv, nq, nk, np, sl2, s); break;
    case 4: launch<4>(q, k, v, out, n_head_kv, nq, nk, np, sl2, s); break;
    default: launch<8>(q, k, v, out, n_head_kv, nq, nk, np, sl2, s); break;
  }
  return ikv::launch_status();
}
