// attn_decode.hip — GQA decode attention over the contiguous KV cache, split-K
// over the context, with the KV append of the new token fused in.
//
// Replaces the score + softmax kernel pair of CUDA_F32::compute_flash_attn for
// one query token (reference src/kernels/cuda/kernel_f32.cu:330-511), which
// launched one 32-thread block per score, materialised Hq*L scores, and
// allocated, synchronised and freed a buffer on every call. Semantics follow
// CPUBackend::compute_flash_attn (src/backends/cpu_backend.cpp:525-634):
// q head h reads KV head h / (n_head / n_head_kv); softmax(q.k * scale) . v.
//
// Work decomposition (gfx950, 256 CUs in 8 XCDs):
//   * One workgroup = 4 wavefronts = one (KV head g, context split s).
//     blockIdx = s * n_head_kv + g, so with 8 KV heads every split of head g
//     is dispatched to XCD g and shares that XCD's L2.
//   * Within a workgroup each half-wave (32 lanes x float4) owns one 512-byte
//     K or V row at a time: loads are fully coalesced 16-byte accesses along
//     the token-major cache ([token][kv head][128] F32, 4096 B per token at
//     Qwen3 shapes). Each K/V row is read from HBM exactly once and serves all
//     G query heads of the group.
//   * Online softmax (base-2, running max / sum) per half-wave, merged across
//     half-waves by a lane exchange and across the 4 waves through LDS.
//   * Split partials (max, sum, unnormalised output) go to the workspace; the
//     last workgroup of each KV head to finish (device-scope counter) merges
//     them and writes the output, then resets its counter for the next launch.
//   * Fused append: the row of the new token (n_kv-1) is read from k_new/v_new
//     instead of the cache, and the workgroup that owns it stores it into the
//     cache unchanged (a 16-byte copy, bit-exact).
#include "ikv_common.hpp"
#include "../../include/ikv.h"

#include <climits>

namespace {

constexpr int D = 128;         // head_dim supported by this kernel
constexpr int NWAVE = 4;       // wavefronts per workgroup
constexpr int WG = NWAVE * 64;
constexpr int R = 4;           // K and V rows held per lane per iteration
constexpr int TILE = NWAVE * 2 * R;  // tokens per workgroup iteration
constexpr int kMaxSplits = 512;

#ifndef IKV_DECODE_TARGET_WGS
// About two workgroups per CU on MI355X (256 CUs).
#define IKV_DECODE_TARGET_WGS 512
#endif

struct Plan {
  int n_splits;
  int tokens_per_split;
};

Plan plan_for(int n_head_kv, int64_t n_kv) {
  int64_t target = (IKV_DECODE_TARGET_WGS + n_head_kv - 1) / n_head_kv;
  if (target < 1) target = 1;
  if (target > kMaxSplits) target = kMaxSplits;
  const int64_t n_tiles = (n_kv + TILE - 1) / TILE;
  int64_t tiles_per_split = (n_tiles + target - 1) / target;
  if (tiles_per_split < 1) tiles_per_split = 1;
  const int64_t tokens = tiles_per_split * TILE;
  const int64_t splits = (n_kv + tokens - 1) / tokens;
  return {static_cast<int>(splits), static_cast<int>(tokens)};
}

size_t align256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

struct WsLayout {
  size_t counters, part_ml, part_o, total;
};

WsLayout ws_layout(int n_head, int n_head_kv, int n_splits) {
  WsLayout w;
  w.counters = 0;
  w.part_ml = align256(sizeof(unsigned) * static_cast<size_t>(n_head_kv));
  w.part_o = w.part_ml + align256(sizeof(float) * 2 * static_cast<size_t>(n_head) * n_splits);
  w.total = w.part_o + sizeof(float) * static_cast<size_t>(n_head) * n_splits * D;
  return w;
}

template <int G>
__global__ __launch_bounds__(WG) void decode_kernel(
    const float *__restrict__ q, float *kc, float *vc, const float *k_new, const float *v_new,
    float *__restrict__ out, unsigned *__restrict__ counters, float *__restrict__ part_ml,
    float *__restrict__ part_o, int n_head_kv, int n_kv, int tokens_per_split, int n_splits,
    float scale_log2) {
  __shared__ float s_acc[NWAVE][G][D];
  __shared__ float s_m[NWAVE][G];
  __shared__ float s_l[NWAVE][G];
  __shared__ float s_w[G][kMaxSplits];
  __shared__ float s_inv[G];
  __shared__ unsigned s_last;

  const int g = blockIdx.x % n_head_kv;
  const int split = blockIdx.x / n_head_kv;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = lane >> 5;
  const int sub = lane & 31;
  const int t_begin = split * tokens_per_split;
  const int t_end = min(n_kv, t_begin + tokens_per_split);
  const int new_row = k_new ? n_kv - 1 : -1;
  const size_t tok_stride = static_cast<size_t>(n_head_kv) * D;
  const size_t head_off = static_cast<size_t>(g) * D + 4 * sub;

  float4 qv[G];
#pragma unroll
  for (int h = 0; h < G; ++h)
    qv[h] = *reinterpret_cast<const float4 *>(q + static_cast<size_t>(g * G + h) * D + 4 * sub);

  float m[G], l[G];
  float4 acc[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
    acc[h] = make_float4(0.f, 0.f, 0.f, 0.f);
  }

  for (int base = t_begin; base < t_end; base += TILE) {
    float4 kr[R], vr[R];
    int tok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) tok[r] = base + r * (NWAVE * 2) + wave * 2 + half;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int t = tok[r];
      if (t < t_end) {
        const bool fresh = (t == new_row);
        const float *kp = fresh ? k_new + head_off : kc + static_cast<size_t>(t) * tok_stride + head_off;
        const float *vp = fresh ? v_new + head_off : vc + static_cast<size_t>(t) * tok_stride + head_off;
        kr[r] = *reinterpret_cast<const float4 *>(kp);
        vr[r] = *reinterpret_cast<const float4 *>(vp);
      } else {
        kr[r] = make_float4(0.f, 0.f, 0.f, 0.f);
        vr[r] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    if (new_row >= base && new_row < base + TILE) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (tok[r] == new_row && tok[r] < t_end) {
          const size_t off = static_cast<size_t>(new_row) * tok_stride + head_off;
          *reinterpret_cast<float4 *>(kc + off) = kr[r];
          *reinterpret_cast<float4 *>(vc + off) = vr[r];
        }
      }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float sc[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float d = ikv::half_wave_sum(ikv::dot4(qv[h], kr[r]));
        sc[r] = (tok[r] < t_end) ? d * scale_log2 : -INFINITY;
      }
      float mx = m[h];
#pragma unroll
      for (int r = 0; r < R; ++r) mx = fmaxf(mx, sc[r]);
      if (mx != -INFINITY) {
        const float alpha = ikv::fast_exp2(m[h] - mx);
        l[h] *= alpha;
        acc[h] = ikv::scale4(alpha, acc[h]);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float p = ikv::fast_exp2(sc[r] - mx);
          l[h] += p;
          acc[h] = ikv::fma4(p, vr[r], acc[h]);
        }
        m[h] = mx;
      }
    }
  }

  // Merge the two half-waves (they saw different tokens).
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float mo = __shfl_xor(m[h], 32, 64);
    const float lo = __shfl_xor(l[h], 32, 64);
    float4 ao;
    ao.x = __shfl_xor(acc[h].x, 32, 64);
    ao.y = __shfl_xor(acc[h].y, 32, 64);
    ao.z = __shfl_xor(acc[h].z, 32, 64);
    ao.w = __shfl_xor(acc[h].w, 32, 64);
    const float M = fmaxf(m[h], mo);
    const float a = (M == -INFINITY) ? 0.f : ikv::fast_exp2(m[h] - M);
    const float b = (M == -INFINITY) ? 0.f : ikv::fast_exp2(mo - M);
    l[h] = l[h] * a + lo * b;
    acc[h] = make_float4(acc[h].x * a + ao.x * b, acc[h].y * a + ao.y * b,
                         acc[h].z * a + ao.z * b, acc[h].w * a + ao.w * b);
    m[h] = M;
  }
  if (half == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      *reinterpret_cast<float4 *>(&s_acc[wave][h][4 * sub]) = acc[h];
      if (sub == 0) {
        s_m[wave][h] = m[h];
        s_l[wave][h] = l[h];
      }
    }
  }
  __syncthreads();

  // Merge the 4 waves: thread (h, d).
  for (int idx = tid; idx < G * D; idx += WG) {
    const int h = idx / D;
    const int d = idx - h * D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) M = fmaxf(M, s_m[w][h]);
    float O = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
      const float mw = s_m[w][h];
      const float e = (mw == -INFINITY) ? 0.f : ikv::fast_exp2(mw - M);
      O += s_acc[w][h][d] * e;
      L += s_l[w][h] * e;
    }
    const int qh = g * G + h;
    if (n_splits == 1) {
      out[static_cast<size_t>(qh) * D + d] = O / L;
    } else {
      const size_t slot = static_cast<size_t>(qh) * n_splits + split;
      part_o[slot * D + d] = O;
      if (d == 0) {
        part_ml[2 * slot] = M;
        part_ml[2 * slot + 1] = L;
      }
    }
  }
  if (n_splits == 1) return;

  // Last workgroup of this KV head merges the split partials.
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = atomicAdd(&counters[g], 1u);
    s_last = (prev == static_cast<unsigned>(n_splits) - 1u) ? 1u : 0u;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  for (int h = wave; h < G; h += NWAVE) {
    const float *ml = part_ml + static_cast<size_t>(g * G + h) * n_splits * 2;
    float mx = -INFINITY;
    for (int i = lane; i < n_splits; i += 64) mx = fmaxf(mx, ml[2 * i]);
    mx = ikv::wave_max(mx);
    float sum = 0.f;
    for (int i = lane; i < n_splits; i += 64) {
      const float w = ikv::fast_exp2(ml[2 * i] - mx);
      s_w[h][i] = w;
      sum += ml[2 * i + 1] * w;
    }
    sum = ikv::wave_sum(sum);
    if (lane == 0) s_inv[h] = 1.0f / sum;
  }
  __syncthreads();

  for (int idx = tid; idx < G * D; idx += WG) {
    const int h = idx / D;
    const int d = idx - h * D;
    const int qh = g * G + h;
    const float *po = part_o + static_cast<size_t>(qh) * n_splits * D + d;
    float O0 = 0.f, O1 = 0.f, O2 = 0.f, O3 = 0.f;
    int i = 0;
    for (; i + 4 <= n_splits; i += 4) {
      O0 += po[static_cast<size_t>(i) * D] * s_w[h][i];
      O1 += po[static_cast<size_t>(i + 1) * D] * s_w[h][i + 1];
      O2 += po[static_cast<size_t>(i + 2) * D] * s_w[h][i + 2];
      O3 += po[static_cast<size_t>(i + 3) * D] * s_w[h][i + 3];
    }
    for (; i < n_splits; ++i) O0 += po[static_cast<size_t>(i) * D] * s_w[h][i];
    out[static_cast<size_t>(qh) * D + d] = ((O0 + O1) + (O2 + O3)) * s_inv[h];
  }
  if (tid == 0) atomicExch(&counters[g], 0u);
}

template <int G>
void launch(const float *q, float *kc, float *vc, const float *kn, const float *vn, float *out,
            char *ws, const WsLayout &L, int n_head_kv, int n_kv, const Plan &p, float scale_log2,
            hipStream_t s) {
  decode_kernel<G><<<n_head_kv * p.n_splits, WG, 0, s>>>(
      q, kc, vc, kn, vn, out, reinterpret_cast<unsigned *>(ws + L.counters),
      reinterpret_cast<float *>(ws + L.part_ml), reinterpret_cast<float *>(ws + L.part_o),
      n_head_kv, n_kv, p.tokens_per_split, p.n_splits, scale_log2);
}

}  // namespace

extern "C" size_t ikv_attn_decode_workspace_bytes(int n_head, int n_head_kv, int head_dim,
                                                  int64_t n_kv) {
  if (n_head <= 0 || n_head_kv <= 0 || head_dim != D || n_kv <= 0) return 0;
  const Plan p = plan_for(n_head_kv, n_kv);
  return ws_layout(n_head, n_head_kv, p.n_splits).total;
}

extern "C" int ikv_attn_decode_f32(const float *q, float *k_cache, float *v_cache,
                                   const float *k_new, const float *v_new, float *out, int n_head,
                                   int n_head_kv, int head_dim, int64_t n_kv, float scale,
                                   void *workspace, size_t workspace_bytes, void *stream) {
  if (!q || !k_cache || !v_cache || !out) return -EINVAL;
  if ((k_new == nullptr) != (v_new == nullptr)) return -EINVAL;
  if (n_head <= 0 || n_head_kv <= 0 || n_head % n_head_kv != 0) return -EINVAL;
  if (n_kv <= 0) return -EINVAL;
  if (head_dim != D) return -ENOTSUP;
  const int G = n_head / n_head_kv;
  if (G != 1 && G != 2 && G != 4 && G != 8) return -ENOTSUP;
  if (n_kv > INT_MAX - TILE) return -EOVERFLOW;
  if (!ikv::aligned16(q) || !ikv::aligned16(k_cache) || !ikv::aligned16(v_cache) ||
      !ikv::aligned16(out) || (k_new && (!ikv::aligned16(k_new) || !ikv::aligned16(v_new))))
    return -EINVAL;
  const Plan p = plan_for(n_head_kv, n_kv);
  const WsLayout L = ws_layout(n_head, n_head_kv, p.n_splits);
  if (p.n_splits > 1 && (!workspace || workspace_bytes < L.total || !ikv::aligned16(workspace)))
    return -EINVAL;
  if (!(scale > 0.0f)) scale = 1.0f / sqrtf(static_cast<float>(head_dim));
  const float scale_log2 = scale * ikv::kLog2e;
  char *ws = static_cast<char *>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nk = static_cast<int>(n_kv);
  switch (G) {
    case 1: launch<1>(q, k_cache, v_cache, k_new, v_new, out, ws, L, n_head_kv, nk, p, scale_log2, s); break;
    case 2: launch<2>(q, k_cache, v_cache, k_new, v_new, out, ws, L, n_head_kv, nk, p, scale_log2, s); break;
    case 4: launch<4>(q, k_cache, v_cache, k_new, v_new, out, ws, L, n_head_kv, nk, p, scale_log2, s); break;
    default: launch<8>(q, k_cache, v_cache, k_new, v_new, out, ws, L, n_head_kv, nk, p, scale_log2, s); break;
  }
  return ikv::launch_status();
}
