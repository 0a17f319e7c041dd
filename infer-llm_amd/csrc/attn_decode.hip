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
// Two launches, no device-scope fences or atomics:
//   split kernel  one workgroup (4 wavefronts) per (KV head g, context split).
//                 blockIdx = split * n_head_kv + g, so with 8 KV heads every
//                 split of head g lands on XCD g. Each half-wave (32 lanes x
//                 float4) owns one 512-byte K or V row at a time: coalesced
//                 16-byte non-temporal loads along the token-major cache
//                 ([token][kv head][128] F32, 4096 B per token at Qwen3
//                 shapes), every row read from HBM once and used by all G
//                 query heads of the group. The next R rows per lane are
//                 prefetched into registers while the current ones are
//                 scored. Online softmax in base 2 per half-wave, merged
//                 across half-waves by lane exchange and across waves through
//                 LDS. With one split the output is written directly;
//                 otherwise (max, sum, unnormalised output) per split goes to
//                 the workspace.
//   merge kernel  four workgroups per query head rescale and sum the split
//                 partials in one memory round trip.
// Why a second launch: the kernel boundary makes the partials of all 8 XCDs
// visible. Merging inside the split kernel ("last workgroup to arrive merges")
// was measured on MI355X and is slower than the extra launch at every context
// length: agent-scope release/acquire fences write back / invalidate the
// XCD's L2 (buffer_wbl2 / buffer_inv), and device-scope atomics on one
// counter serialise at about 0.14 us per arriving workgroup, while a kernel
// boundary in a HIP graph costs about 1.6 us.
// Fused append: the row of the new token (n_kv-1) is read from k_new/v_new
// instead of the cache, and the workgroup that owns it stores it into the
// cache unchanged (a 16-byte copy, bit-exact).
#include "ikv_common.hpp"
#include "../../include/ikv.h"

#include <climits>

namespace {

constexpr int D = 128;         // head_dim supported by this kernel
constexpr int NWAVE = 4;       // wavefronts per workgroup
constexpr int WG = NWAVE * 64;
#ifndef IKV_DECODE_R
#define IKV_DECODE_R 4
#endif
constexpr int R = IKV_DECODE_R;      // K and V rows per lane per iteration
constexpr int TILE = NWAVE * 2 * R;  // tokens per workgroup iteration
constexpr int kMaxSplits = 1024;

#ifndef IKV_DECODE_TARGET_WGS
// Split-kernel workgroups aimed for: four per CU on MI355X (256 CUs).
#define IKV_DECODE_TARGET_WGS 1024
#endif
#ifndef IKV_DECODE_NT
#define IKV_DECODE_NT 1  // 1: K/V history read with non-temporal (streaming) loads
#endif

struct Plan {
  int n_splits;
  int tokens_per_split;
};

Plan plan_for(int n_head_kv, int64_t n_kv) {
  // Whole tiles per split, as few per split as the target allows: at ctx 4096
  // (129 tiles per head) every split is one tile and all workgroups are
  // resident at once. Splits stay below 2*target <= kMaxSplits.
  int64_t target = (IKV_DECODE_TARGET_WGS + n_head_kv - 1) / n_head_kv;
  if (target < 1) target = 1;
  if (target > kMaxSplits / 2) target = kMaxSplits / 2;
  const int64_t n_tiles = (n_kv + TILE - 1) / TILE;
  int64_t tiles_per_split = n_tiles / target;
  if (tiles_per_split < 1) tiles_per_split = 1;
  const int64_t tokens = tiles_per_split * TILE;
  const int64_t splits = (n_kv + tokens - 1) / tokens;
  return {static_cast<int>(splits), static_cast<int>(tokens)};
}

size_t align256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

struct WsLayout {
  size_t part_ml, part_o, total;
};

// [n_head x n_splits x (max, sum)][n_head x n_splits x D]
WsLayout ws_layout(int n_head, int n_splits) {
  WsLayout w;
  w.part_ml = 0;
  w.part_o = align256(sizeof(float) * 2 * static_cast<size_t>(n_head) * n_splits);
  w.total = w.part_o + sizeof(float) * static_cast<size_t>(n_head) * n_splits * D;
  return w;
}

template <int G>
__device__ __forceinline__ void load_rows(float4 (&kr)[R], float4 (&vr)[R], int base, int t_end,
                                          int wave, int half, int new_row, const float *kc,
                                          const float *vc, const float *k_new, const float *v_new,
                                          size_t tok_stride, size_t head_off) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int t = base + r * (NWAVE * 2) + wave * 2 + half;
    if (t < t_end) {
      const bool fresh = (t == new_row);
      const float *kp = fresh ? k_new + head_off : kc + static_cast<size_t>(t) * tok_stride + head_off;
      const float *vp = fresh ? v_new + head_off : vc + static_cast<size_t>(t) * tok_stride + head_off;
#if IKV_DECODE_NT
      typedef float f4v __attribute__((ext_vector_type(4)));
      const f4v a = __builtin_nontemporal_load(reinterpret_cast<const f4v *>(kp));
      const f4v b = __builtin_nontemporal_load(reinterpret_cast<const f4v *>(vp));
      kr[r] = make_float4(a.x, a.y, a.z, a.w);
      vr[r] = make_float4(b.x, b.y, b.z, b.w);
#else
      kr[r] = *reinterpret_cast<const float4 *>(kp);
      vr[r] = *reinterpret_cast<const float4 *>(vp);
#endif
    } else {
      kr[r] = make_float4(0.f, 0.f, 0.f, 0.f);
      vr[r] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
}

// Combines the online-softmax states of the 4 waves (in LDS) for query head
// h of the group, dim d: unnormalised output O, sum L, max M.
template <int G>
__device__ __forceinline__ void merge_waves(const float (&s_acc)[NWAVE][G][D],
                                            const float (&s_m)[NWAVE][G],
                                            const float (&s_l)[NWAVE][G], int h, int d, float &O,
                                            float &L, float &M) {
  M = -INFINITY;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) M = fmaxf(M, s_m[w][h]);
  O = 0.f;
  L = 0.f;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) {
    const float mw = s_m[w][h];
    const float e = (mw == -INFINITY) ? 0.f : ikv::fast_exp2(mw - M);
    O += s_acc[w][h][d] * e;
    L += s_l[w][h] * e;
  }
}

template <int G>
__global__ __launch_bounds__(WG) void decode_split_kernel(
    const float *__restrict__ q, float *kc, float *vc, const float *k_new, const float *v_new,
    float *__restrict__ out, float *__restrict__ part_ml, float *__restrict__ part_o,
    int n_head_kv, int n_kv, int tokens_per_split, int n_splits, float scale_log2) {
  __shared__ float s_acc[NWAVE][G][D];
  __shared__ float s_m[NWAVE][G];
  __shared__ float s_l[NWAVE][G];

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

  float4 kr[R], vr[R];
  load_rows<G>(kr, vr, t_begin, t_end, wave, half, new_row, kc, vc, k_new, v_new, tok_stride,
               head_off);

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
    float4 kn[R], vn[R];
    const bool more = base + TILE < t_end;
    if (more)
      load_rows<G>(kn, vn, base + TILE, t_end, wave, half, new_row, kc, vc, k_new, v_new,
                   tok_stride, head_off);

    if (new_row >= base && new_row < base + TILE) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int t = base + r * (NWAVE * 2) + wave * 2 + half;
        if (t == new_row) {
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
        const int t = base + r * (NWAVE * 2) + wave * 2 + half;
        const float d = ikv::half_wave_sum(ikv::dot4(qv[h], kr[r]));
        sc[r] = (t < t_end) ? d * scale_log2 : -INFINITY;
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
    if (more) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        kr[r] = kn[r];
        vr[r] = vn[r];
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

  // Merge the 4 waves. With one split the result is final.
  if (n_splits == 1) {
    for (int idx = tid; idx < G * D; idx += WG) {
      const int h = idx / D;
      const int d = idx - h * D;
      float O, L, M;
      merge_waves<G>(s_acc, s_m, s_l, h, d, O, L, M);
      out[static_cast<size_t>(g * G + h) * D + d] = O / L;
    }
    return;
  }
  for (int idx = tid; idx < G * D; idx += WG) {
    const int h = idx / D;
    const int d = idx - h * D;
    float O, L, M;
    merge_waves<G>(s_acc, s_m, s_l, h, d, O, L, M);
    const size_t slot = static_cast<size_t>(g * G + h) * n_splits + split;
    part_o[slot * D + d] = O;
    if (d == 0) {
      part_ml[2 * slot] = M;
      part_ml[2 * slot + 1] = L;
    }
  }
}

// Merge of the split partials: 4 workgroups per query head, each owning 32
// dims. Thread (grp, dd) of 8 x 32 sums splits grp, grp+8, ... for dim dd.
// All partial loads of a chunk of 256 splits are issued before any is used,
// so a chunk costs one memory round trip.
constexpr int kMergeThreads = 256;
constexpr int kMergeDims = 32;
constexpr int kMergeGroups = kMergeThreads / kMergeDims;  // 8
constexpr int kMergeChunk = 256;                          // splits per round trip
constexpr int kMergeJ = kMergeChunk / kMergeGroups;       // 32 loads per thread

__global__ __launch_bounds__(kMergeThreads) void decode_merge_kernel(
    const float *__restrict__ part_ml, const float *__restrict__ part_o, float *__restrict__ out,
    int n_splits) {
  __shared__ float s_w[kMaxSplits];
  __shared__ float s_red[kMergeGroups][kMergeDims];
  __shared__ float s_stat[4];
  const int qh = blockIdx.x / (D / kMergeDims);
  const int d0 = (blockIdx.x % (D / kMergeDims)) * kMergeDims;
  const int tid = threadIdx.x;
  const int grp = tid / kMergeDims;
  const int dd = tid % kMergeDims;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const float *ml = part_ml + static_cast<size_t>(qh) * n_splits * 2;
  const float *po = part_o + static_cast<size_t>(qh) * n_splits * D + d0 + dd;

  float v[kMergeJ];
#pragma unroll
  for (int j = 0; j < kMergeJ; ++j) {
    const int s = grp + kMergeGroups * j;
    v[j] = (s < n_splits) ? po[static_cast<size_t>(s) * D] : 0.f;
  }
  // Split statistics, one (max, sum) pair per split, loaded together with the
  // partials above: weights 2^(m - M) and the weighted sum of l.
  float2 st[kMergeChunk / kMergeThreads];
#pragma unroll
  for (int k = 0; k < kMergeChunk / kMergeThreads; ++k) {
    const int i = tid + k * kMergeThreads;
    st[k] = (i < n_splits) ? reinterpret_cast<const float2 *>(ml)[i] : make_float2(-INFINITY, 0.f);
  }
  float mloc = -INFINITY;
  for (int i = tid + kMergeChunk; i < n_splits; i += kMergeThreads) mloc = fmaxf(mloc, ml[2 * i]);
#pragma unroll
  for (int k = 0; k < kMergeChunk / kMergeThreads; ++k) mloc = fmaxf(mloc, st[k].x);
  mloc = ikv::wave_max(mloc);
  if (lane == 0) s_stat[wave] = mloc;
  __syncthreads();
  const float M = fmaxf(fmaxf(s_stat[0], s_stat[1]), fmaxf(s_stat[2], s_stat[3]));
  float lsum = 0.f;
#pragma unroll
  for (int k = 0; k < kMergeChunk / kMergeThreads; ++k) {
    const int i = tid + k * kMergeThreads;
    if (i < n_splits) {
      const float w = ikv::fast_exp2(st[k].x - M);
      s_w[i] = w;
      lsum += st[k].y * w;
    }
  }
  for (int i = tid + kMergeChunk; i < n_splits; i += kMergeThreads) {
    const float w = ikv::fast_exp2(ml[2 * i] - M);
    s_w[i] = w;
    lsum += ml[2 * i + 1] * w;
  }
  lsum = ikv::wave_sum(lsum);
  __syncthreads();
  if (lane == 0) s_stat[wave] = lsum;
  __syncthreads();
  const float inv = 1.0f / ((s_stat[0] + s_stat[1]) + (s_stat[2] + s_stat[3]));

  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < kMergeJ; ++j) {
    const int s = grp + kMergeGroups * j;
    if (s < n_splits) acc += v[j] * s_w[s];
  }
  for (int base = kMergeChunk; base < n_splits; base += kMergeChunk) {
#pragma unroll
    for (int j = 0; j < kMergeJ; ++j) {
      const int s = base + grp + kMergeGroups * j;
      v[j] = (s < n_splits) ? po[static_cast<size_t>(s) * D] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < kMergeJ; ++j) {
      const int s = base + grp + kMergeGroups * j;
      if (s < n_splits) acc += v[j] * s_w[s];
    }
  }
  s_red[grp][dd] = acc;
  __syncthreads();
  if (grp == 0) {
    float o = 0.f;
#pragma unroll
    for (int k = 0; k < kMergeGroups; ++k) o += s_red[k][dd];
    out[static_cast<size_t>(qh) * D + d0 + dd] = o * inv;
  }
}

template <int G>
void launch_split(const float *q, float *kc, float *vc, const float *kn, const float *vn,
                  float *out, float *part_ml, float *part_o, int n_head_kv, int n_kv,
                  const Plan &p, float scale_log2, hipStream_t s) {
  decode_split_kernel<G><<<n_head_kv * p.n_splits, WG, 0, s>>>(
      q, kc, vc, kn, vn, out, part_ml, part_o, n_head_kv, n_kv, p.tokens_per_split, p.n_splits,
      scale_log2);
}

}  // namespace

extern "C" size_t ikv_attn_decode_workspace_bytes(int n_head, int n_head_kv, int head_dim,
                                                  int64_t n_kv) {
  if (n_head <= 0 || n_head_kv <= 0 || head_dim != D || n_kv <= 0) return 0;
  const Plan p = plan_for(n_head_kv, n_kv);
  return ws_layout(n_head, p.n_splits).total;
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
  if (n_kv > INT_MAX - 2 * TILE) return -EOVERFLOW;
  if (!ikv::aligned16(q) || !ikv::aligned16(k_cache) || !ikv::aligned16(v_cache) ||
      !ikv::aligned16(out) || (k_new && (!ikv::aligned16(k_new) || !ikv::aligned16(v_new))))
    return -EINVAL;
  const Plan p = plan_for(n_head_kv, n_kv);
  const WsLayout L = ws_layout(n_head, p.n_splits);
  float *part_ml = nullptr, *part_o = nullptr;
  if (p.n_splits > 1) {
    if (!workspace || workspace_bytes < L.total || !ikv::aligned16(workspace)) return -EINVAL;
    part_ml = reinterpret_cast<float *>(static_cast<char *>(workspace) + L.part_ml);
    part_o = reinterpret_cast<float *>(static_cast<char *>(workspace) + L.part_o);
  }
  if (!(scale > 0.0f)) scale = 1.0f / sqrtf(static_cast<float>(head_dim));
  const float sl2 = scale * ikv::kLog2e;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nk = static_cast<int>(n_kv);
  switch (G) {
    case 1: launch_split<1>(q, k_cache, v_cache, k_new, v_new, out, part_ml, part_o, n_head_kv, nk, p, sl2, s); break;
    case 2: launch_split<2>(q, k_cache, v_cache, k_new, v_new, out, part_ml, part_o, n_head_kv, nk, p, sl2, s); break;
    case 4: launch_split<4>(q, k_cache, v_cache, k_new, v_new, out, part_ml, part_o, n_head_kv, nk, p, sl2, s); break;
    default: launch_split<8>(q, k_cache, v_cache, k_new, v_new, out, part_ml, part_o, n_head_kv, nk, p, sl2, s); break;
  }
  if (p.n_splits > 1)
    decode_merge_kernel<<<n_head * (D / kMergeDims), kMergeThreads, 0, s>>>(part_ml, part_o, out,
                                                                          p.n_splits);
  return ikv::launch_status();
}
