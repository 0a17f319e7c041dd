// attn_prefill.hip — causal GQA flash attention for n_q >= 1 query tokens on
// F32 MFMA (v_mfma_f32_16x16x4_f32), never materialising the score matrix.
//
// Replaces CUDA_F32::compute_flash_attn for prefill (reference
// src/kernels/cuda/kernel_f32.cu:452-511), which allocated Hq*n_q*n_kv floats
// of scores per call. Semantics: CPUBackend::compute_flash_attn
// (src/backends/cpu_backend.cpp:525-634): key j is visible to query t iff
// j <= n_past + t; q head h reads KV head h / G, G = n_head / n_head_kv.
//
// Decomposition:
//   * A query block is NW*16 rows of one KV head's group: NW*16/G tokens x G
//     query heads. K/V tiles (32 keys x 128 dims) of that KV head are staged
//     in LDS once per block and shared by its NW wavefronts, i.e. by all G
//     query heads. blockIdx % n_head_kv is the KV head, so with 8 KV heads each
//     XCD (and its L2) serves one KV head.
//   * Causal balance: a workgroup processes the pair of query blocks (i,
//     n_blocks-1-i) of its KV head one after the other, so every workgroup
//     walks the same number of key tiles (the heaviest block alone is twice
//     the average).
//   * Key split: where a block per CU leaves SIMDs idle, a block's waves form
//     NG groups holding the same rows that take interleaved key tiles and
//     merge their softmax states through LDS at the end: two 4-wave groups
//     (long prompts), or for short prompts two or four one-wave groups, so
//     that the longest causal rows take 1/NG of the serial MFMA steps.
//   * Each wavefront owns 16 rows and computes, per 32-key tile,
//       S^T = K Q^T    (2 x [16 keys x 16 rows], contraction over 128 dims)
//       O^T += V^T P^T (8 x [16 dims x 16 rows], contraction over 32 keys)
//     so a lane holds one query row (lane % 16) in both products. Operands
//     come from registers (Q, P) or 16-byte LDS reads (one ds_read_b128 of K
//     feeds 4 MFMAs); output tile t, register r of lane l holds dim
//     64*(t/4) + 16*(l/16) + 4r + t%4.
//   * Tiles move global -> LDS with buffer_load_dwordx4 ... lds (no VGPR
//     staging) into two LDS buffers: tile t+1 loads while tile t is used.
//     Each tile's K and V rows are a buffer resource built from scalars (the
//     tile's first row, or its paged block's) and each lane's byte offsets
//     are the same for every tile, so issuing a tile costs no vector
//     address arithmetic (with 64-bit per-lane addresses: P = 4096 520 ->
//     501 us, P = 2048 ~1-4% faster, outputs bit-identical).
//     The DMA writes each wave's 64 x 16 bytes contiguously, so K rows are
//     stored with 16-byte chunk c at slot c ^ (key % 16): the 16 lanes that
//     read one chunk index from 16 keys then hit 16 different bank groups.
//     Keys past n_kv lie outside the tile's buffer range and read as zeros
//     (finite data, masked out).
//   * Softmax runs in base 2 on a per-row reference max that only moves when
//     a score exceeds it by 2^8 (checked with one wave vote), so most tiles
//     skip the cross-lane max and the O rescale; row sums stay per lane until
//     the end. Cross-lane row reductions use v_permlane{32,16}_swap.
//   * LDS fragment reads run one MFMA group ahead; sched_group_barrier keeps
//     the compiler from sinking them next to their uses.
//   * A wave raises its issue priority (s_setprio 1) for its two MFMA
//     sections and drops it for the softmax between them, so that on a SIMD
//     shared by two waves the one with MFMAs to issue goes first and the
//     other's softmax fills the matrix pipe's gaps (P = 2048: 147.3 ->
//     145.8 us, alternated runs on one box).
//   * Two 4-wave key-split groups use their own double buffers, so a round
//     of tiles needs only the waves of one group to agree: each group passes
//     an LDS arrival counter instead of the workgroup barrier, and the
//     groups drift apart (P = 2048: 144.4 -> 141.4 us, alternated runs).
#include "attn_generic.hpp"
#include "coherent.hpp"
#include "ikv_common.hpp"
#include "../../include/ikv.h"

#include <algorithm>
#include <climits>

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void *lds_ptr;

constexpr int D = 128;
constexpr int BN = 32;              // keys per tile
constexpr int TILE = BN * D;        // floats of K (or V) per tile
constexpr int kMaxKvHeads = 1 << 16;  // tile rows addressed with 32-bit offsets
constexpr float kRescale = 8.0f;    // log2 headroom before the running max is moved
#ifndef IKV_PREFILL_PAIR_MIN_WGS
#define IKV_PREFILL_PAIR_MIN_WGS 256  // one workgroup per CU
#endif
#ifndef IKV_PREFILL_NW
#define IKV_PREFILL_NW 0  // waves per workgroup; 0 = chosen per launch
#endif
#ifndef IKV_PREFILL_SPLIT
#define IKV_PREFILL_SPLIT 1  // 8-wave workgroups (two key-split groups) at one block per CU
#endif
constexpr int kCUs = 256;  // MI355X compute units

// 16 bytes per lane from a buffer resource at byte offset voff into LDS at
// dst (the wave's 64 x 16 bytes contiguous from dst)
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, float *dst, unsigned voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)dst, 16, voff, 0, 0, 0);
}

__device__ __forceinline__ floatx4 mfma16(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// max / sum over the 4 lanes l, l^16, l^32, l^48 (one query row); every lane
// gets the same bits.
__device__ __forceinline__ float row_max4(float x) {
  auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float row_sum4(float x) {
  auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

template <int G, int NW, int NG, bool PAGED>
__global__ __launch_bounds__(NW * 64) void prefill_kernel(const float *__restrict__ q,
                                                          const float *__restrict__ k,
                                                          const float *__restrict__ v,
                                                          float *__restrict__ out, int n_head_kv,
                                                          int n_q, int n_kv, int n_past,
                                                          int n_blocks, int paired,
                                                          float scale_log2, ikv::Pages pages) {
  // NG > 1: NG groups of NW / NG waves hold the same query rows and take
  // interleaved key tiles (group r: tiles r, r + NG, ...), merging their
  // softmax states at the end: two groups of 4 waves so that each SIMD runs
  // two; four one-wave groups (one per SIMD) so that a short prompt's
  // longest causal rows take a quarter of the serial MFMA steps.
  // One-wave groups (ONE) keep a single K and V buffer each, 4 x 32 KB of
  // LDS: the next tile's K is issued once this tile's Q K^T has read K, its
  // V once P V has read V, with this wave's own waits and no barriers.
  static_assert(NG == 1 || NG == 2 || NG == 4, "one, two or four wave groups");
  static_assert(NW % NG == 0, "whole groups");
  constexpr int WPG = NW / NG;         // waves per group
  constexpr bool ONE = NG == 4;
  static_assert(!ONE || WPG == 1, "four groups are one wave each");
  constexpr int BQ = WPG * 16 / G;

  const int g = blockIdx.x % n_head_kv;
  const int item = blockIdx.x / n_head_kv;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int grp = 0, w = wave;  // group, wave within the group
  if constexpr (NG > 1) {
    grp = wave / WPG;
    w = wave - grp * WPG;
  }
  // K and V tile buffers of this group: two of each, or with ONE one of each
  // in separate arrays (so that the compiler's LDS-DMA waits can tell the
  // next tile's K from this tile's V). K rows hold 16-byte chunk c at slot
  // c ^ (key & 15). xch: where the groups' states meet at the end.
  float *k0, *v0, *k1, *v1, *xch0;
  if constexpr (ONE) {
    __shared__ __attribute__((aligned(16))) float s_k[NG][TILE];
    __shared__ __attribute__((aligned(16))) float s_v[NG][TILE];
    k0 = k1 = s_k[grp];
    v0 = v1 = s_v[grp];
    xch0 = s_k[0];
  } else {
    __shared__ __attribute__((aligned(16))) float s_buf[NG][2][2 * TILE];
    k0 = s_buf[grp][0];
    v0 = k0 + TILE;
    k1 = s_buf[grp][1];
    v1 = k1 + TILE;
    xch0 = s_buf[0][0];
  }
  // Group barrier of the two-group tile loop: an LDS counter per group that
  // each of its waves raises by one per round; a wave waits for WPG arrivals
  // per round so far. Every wave of a group runs the same rounds (the loop
  // bounds are per workgroup), so every wait ends.
  __shared__ unsigned s_arrive[NG];
  unsigned rounds = 0;
  if constexpr (NG == 2) {
    if (threadIdx.x < NG) s_arrive[threadIdx.x] = 0;
  }
  auto group_sync = [&]() {
    if constexpr (NG == 2) {
      ++rounds;
      if (lane == 0)
        __hip_atomic_fetch_add(&s_arrive[grp], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      const unsigned target = WPG * rounds;
      while (static_cast<int>(__hip_atomic_load(&s_arrive[grp], __ATOMIC_ACQUIRE,
                                                __HIP_MEMORY_SCOPE_WORKGROUP) -
                              target) < 0)
        __builtin_amdgcn_s_sleep(1);
    } else {
      __syncthreads();
    }
  };
  const int kk = lane >> 4;
  const int j = lane & 15;
  const int row = w * 16 + j;
  const int n_head = n_head_kv * G;

  // this wave's share of one tile: chunks c = w + WPG*i, 1 KB (2 keys) each.
  // A paged cache's block (a multiple of 64 keys) holds every tile whole, so
  // one block offset serves the tile.
  // parts: 1 = K, 2 = V, 3 = both (interleaved)
  // Per tile, one buffer resource over its K rows and one over its V rows
  // (this KV head's 512 bytes of each of the tile's keys, the range ending
  // at the last key inside the cache: keys past n_kv read zeros, which the
  // mask drops); each lane's byte offsets within a tile are fixed.
  constexpr int NI = 16 / WPG;
  unsigned kvo[NI], vvo[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int c = w + WPG * i;
    const int key = 2 * c + (lane >> 5);
    const int slot = lane & 31;
    kvo[i] = static_cast<unsigned>((key * n_head_kv * D + 4 * (slot ^ (key & 15))) * 4);
    vvo[i] = static_cast<unsigned>((key * n_head_kv * D + 4 * slot) * 4);
  }
  auto issue = [&](float *kbuf, float *vbuf, int tile, int parts = 3) {
    int64_t shift = 0;
    if constexpr (PAGED) shift = ikv::page_shift(pages, tile * BN);
    const int rows = min(BN, n_kv - tile * BN);
    const size_t base = (static_cast<size_t>(tile * BN + shift) * n_head_kv + g) * D;
    const int bytes = ((rows - 1) * n_head_kv * D + D) * 4;
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(k + base), 0, bytes, ikv::kBufWord3);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(v + base), 0, bytes, ikv::kBufWord3);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int c = w + WPG * i;
      if (parts & 1)
        dma16(rk, kbuf + c * 256, kvo[i]);
      if (parts & 2)
        dma16(rv, vbuf + c * 256, vvo[i]);
    }
  };
  // s_waitcnt vmcnt(n) (lgkmcnt and expcnt not waited for); with ONE, a
  // tile's 16 K loads are issued before its 16 V loads
  constexpr int kWaitVm0 = 0x0F70, kWaitVm16 = 0x4F70;

  int koff[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) koff[u] = j * D + 4 * ((4 * u + kk) ^ j);
  const int voff = 4 * kk * D + 4 * j;

  const int n_items = paired ? 2 : 1;
  for (int it = 0; it < n_items; ++it) {
    const int blk = paired ? (it == 0 ? item : n_blocks - 1 - item) : n_blocks - 1 - item;
    if (it == 1 && blk == item) break;
    const int q0 = blk * BQ;
    const int tok = q0 + row / G;
    const int head = g * G + row % G;
    const bool row_ok = tok < n_q;
    const int last_tok = min(q0 + BQ, n_q) - 1;
    const int k_end = min(n_kv, n_past + last_tok + 1);
    const int n_tiles = (k_end + BN - 1) / BN;

    __syncthreads();  // the previous item's readers are done with the buffers
    if (grp < n_tiles) {
      if constexpr (ONE) {
        issue(k0, v0, grp, 1);
        issue(k0, v0, grp, 2);
      } else {
        issue(k0, v0, grp);
      }
    }

    float4 qr[8];
    {
      const float *qp = q + (static_cast<size_t>(row_ok ? tok : 0) * n_head + head) * D + 4 * kk;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        qr[u] = row_ok ? *reinterpret_cast<const float4 *>(qp + 16 * u) : make_float4(0.f, 0.f, 0.f, 0.f);
    }

    floatx4 o[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) o[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_row = -INFINITY, l_part = 0.f;

    auto step = [&](const float *kbuf, const float *vbuf, int tile, float *nk, float *nv, bool more,
                    int next) {
      floatx4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
      __builtin_amdgcn_s_setprio(1);  // Q K^T
      // K fragments are read one step ahead so LDS latency hides under MFMAs
      float4 ka0 = *reinterpret_cast<const float4 *>(kbuf + koff[0]);
      float4 ka1 = *reinterpret_cast<const float4 *>(kbuf + 16 * D + koff[0]);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float4 a0 = ka0, a1 = ka1;
        if (u < 7) {
          ka0 = *reinterpret_cast<const float4 *>(kbuf + koff[u + 1]);
          ka1 = *reinterpret_cast<const float4 *>(kbuf + 16 * D + koff[u + 1]);
        }
        s0 = mfma16(a0.x, qr[u].x, s0);
        s1 = mfma16(a1.x, qr[u].x, s1);
        s0 = mfma16(a0.y, qr[u].y, s0);
        s1 = mfma16(a1.y, qr[u].y, s1);
        s0 = mfma16(a0.z, qr[u].z, s0);
        s1 = mfma16(a1.z, qr[u].z, s1);
        s0 = mfma16(a0.w, qr[u].w, s0);
        s1 = mfma16(a1.w, qr[u].w, s1);
      }
      const float *vb = vbuf + voff;
      float4 va_n, vc_n;
      if constexpr (!ONE) {  // (with ONE, V may land only after Q K^T: read below)
        va_n = *reinterpret_cast<const float4 *>(vb);
        vc_n = *reinterpret_cast<const float4 *>(vb + 64);
      }
      // schedule: K(0) K(1) | MMA(0) K(2) | MMA(1) K(3) | ... | MMA(6) V(0) | MMA(7)
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int u = 0; u < 7; ++u) {
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
      if constexpr (ONE) {
        // this buffer's K reads are done (their MFMAs ran): the next
        // tile's K may land in it; this tile's V must have landed
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        if (more) issue(nk, nv, next, 1);
        if (more)
          __builtin_amdgcn_s_waitcnt(kWaitVm16);
        else
          __builtin_amdgcn_s_waitcnt(kWaitVm0);
        __builtin_amdgcn_sched_barrier(0);
        va_n = *reinterpret_cast<const float4 *>(vb);
        vc_n = *reinterpret_cast<const float4 *>(vb + 64);
      } else {
        if (more) issue(nk, nv, next);
      }
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(0);  // softmax
      const int kbase = tile * BN;
      float p[8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[r] = s0[r] * scale_log2;
        p[4 + r] = s1[r] * scale_log2;
      }
      if ((kbase + BN - 1 > n_past + q0) || (kbase + BN > n_kv)) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int kg = kbase + 16 * (i >> 2) + 4 * kk + (i & 3);
          if (kg > n_past + tok || kg >= n_kv) p[i] = -INFINITY;
        }
      }
      float mt = p[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) mt = fmaxf(mt, p[i]);
      // move the row's reference max only when a score exceeds it by 2^8
      if (__builtin_amdgcn_ballot_w64(mt > m_row + kRescale) != 0) {
        const float m_new = fmaxf(m_row, row_max4(mt));
        float alpha = ikv::fast_exp2(m_row - m_new);
        // a later group's row can see only masked keys in its first tiles
        // (its tile lies past an early query): keep -inf - -inf out
        if constexpr (NG > 1) alpha = (m_new == -INFINITY) ? 1.f : alpha;
        m_row = m_new;
        l_part *= alpha;
#pragma unroll
        for (int t = 0; t < 8; ++t) o[t] *= alpha;
      }
      float ref = m_row;
      if constexpr (NG > 1) ref = (m_row == -INFINITY) ? 0.f : m_row;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        p[i] = ikv::fast_exp2(p[i] - ref);
        l_part += p[i];
      }
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(1);  // P V
#pragma unroll
      for (int st = 0; st < 2; ++st) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float4 va = va_n, vc = vc_n;
          if (4 * st + r < 7) {
            const int nx = 4 * st + r + 1;
            va_n = *reinterpret_cast<const float4 *>(vb + (16 * (nx >> 2) + (nx & 3)) * D);
            vc_n = *reinterpret_cast<const float4 *>(vb + (16 * (nx >> 2) + (nx & 3)) * D + 64);
          }
          const float pp = p[4 * st + r];
          o[0] = mfma16(va.x, pp, o[0]);
          o[1] = mfma16(va.y, pp, o[1]);
          o[2] = mfma16(va.z, pp, o[2]);
          o[3] = mfma16(va.w, pp, o[3]);
          o[4] = mfma16(vc.x, pp, o[4]);
          o[5] = mfma16(vc.y, pp, o[5]);
          o[6] = mfma16(vc.z, pp, o[6]);
          o[7] = mfma16(vc.w, pp, o[7]);
        }
      }
      // schedule: V(1) | MMA(0) V(2) | ... | MMA(6) | MMA(7)
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
#pragma unroll
      for (int r = 0; r < 6; ++r) {
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 1);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 16, 1);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(0);
      if constexpr (ONE) {
        // this buffer's V reads are done: the next tile's V may land in it
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        if (more) issue(nk, nv, next, 2);
        __builtin_amdgcn_sched_barrier(0);
      }
    };

    if constexpr (ONE) {
      // this group's tiles, one buffer, no barriers (the group is this wave)
      for (int t = grp; t < n_tiles; t += NG) {
        __builtin_amdgcn_s_waitcnt(kWaitVm16);  // this tile's K landed (its V may not have)
        step(k0, v0, t, k0, v0, t + NG < n_tiles, t + NG);
      }
    } else
    // Rounds of NG tiles, one per group, alternating the buffers.
    for (int t0 = 0; t0 < n_tiles; t0 += 2 * NG) {
      const int ta = t0 + grp;
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's loads of its tile landed
      group_sync();                         // the group's landed; its other buffers are free
      if (ta < n_tiles) step(k0, v0, ta, k1, v1, ta + NG < n_tiles, ta + NG);
      if (t0 + NG >= n_tiles) break;
      const int tb = t0 + NG + grp;
      __builtin_amdgcn_s_waitcnt(0x0F70);
      group_sync();
      if (tb < n_tiles) step(k1, v1, tb, k0, v0, tb + NG < n_tiles, tb + NG);
    }

    if constexpr (NG > 1) {
      // Groups 1 .. NG-1 hand their (O, max, per-lane sum) to group 0
      // through LDS (the tile buffers are free now); group 0 merges them in
      // group order and writes.
      __syncthreads();
      float *const xbase = xch0 + (w * 64 + lane) * 34;
      constexpr int kXchStride = WPG * 64 * 34;  // floats per group
      if (grp > 0) {
        float *xch = xbase + (grp - 1) * kXchStride;
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) xch[4 * t + r] = o[t][r];
        xch[32] = m_row;
        xch[33] = l_part;
      }
      __syncthreads();
      if (grp == 0) {
#pragma unroll
        for (int src = 1; src < NG; ++src) {
          const float *xch = xbase + (src - 1) * kXchStride;
          const float mb = xch[32];
          const float M = fmaxf(m_row, mb);
          const float a = (m_row == -INFINITY) ? 0.f : ikv::fast_exp2(m_row - M);
          const float b = (mb == -INFINITY) ? 0.f : ikv::fast_exp2(mb - M);
          l_part = l_part * a + xch[33] * b;
#pragma unroll
          for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[t][r] = o[t][r] * a + xch[4 * t + r] * b;
          m_row = M;
        }
      }
    }

    const float l_row = row_sum4(l_part);
    if (row_ok && grp == 0) {
      const float inv = 1.0f / l_row;
      float *op = out + (static_cast<size_t>(tok) * n_head + head) * D;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int d0 = 64 * hh + 16 * kk + 4 * r;
          *reinterpret_cast<float4 *>(op + d0) =
              make_float4(o[4 * hh][r] * inv, o[4 * hh + 1][r] * inv, o[4 * hh + 2][r] * inv,
                          o[4 * hh + 3][r] * inv);
        }
      }
    }
  }
}

template <int G, int NW, int NG>
void launch_nw(const float *q, const float *k, const float *v, float *out, int n_head_kv, int n_q,
               int n_kv, int n_past, float scale_log2, int paired, const ikv::Pages *pg,
               hipStream_t s) {
  constexpr int BQ = (NW / NG) * 16 / G;
  const int n_blocks = (n_q + BQ - 1) / BQ;
  const int items = paired ? (n_blocks + 1) / 2 : n_blocks;
  if (pg)
    prefill_kernel<G, NW, NG, true><<<n_head_kv * items, NW * 64, 0, s>>>(
        q, k, v, out, n_head_kv, n_q, n_kv, n_past, n_blocks, paired, scale_log2, *pg);
  else
    prefill_kernel<G, NW, NG, false><<<n_head_kv * items, NW * 64, 0, s>>>(
        q, k, v, out, n_head_kv, n_q, n_kv, n_past, n_blocks, paired, scale_log2, ikv::Pages{});
}

// Shape choice: 4-wave blocks (64 rows) share each staged K/V tile among the
// most rows; 2-wave blocks are used when 4-wave blocks would leave CUs idle.
// Pairing balances the causal triangle but halves the workgroup count, so it
// is used only when the paired grid still gives every CU a workgroup.
template <int G>
void launch(const float *q, const float *k, const float *v, float *out, int n_head_kv, int n_q,
            int n_kv, int n_past, float scale_log2, const ikv::Pages *pg, hipStream_t s) {
  int nw = IKV_PREFILL_NW;
  auto blocks = [&](int w) { return (n_q + w * 16 / G - 1) / (w * 16 / G); };
  // Short prompts: one 16-row block per workgroup, when that still fits one
  // workgroup per CU, its key tiles split among four one-wave groups (one
  // per SIMD; four single buffers, 128 KB of LDS) when the longest causal
  // row spans 3 tiles or more, else between two (two double buffers). At
  // the Qwen3-0.6B shape: P = 256 11.4 us with four groups against 15.0
  // with two, P = 128 8.0 against 9.1; P = 32 and 64 (one or two tiles)
  // 6.2 / 6.4 with two against 7.2 / 7.5 with four.
  if (nw == 0 && IKV_PREFILL_SPLIT && blocks(1) * n_head_kv <= kCUs) {
    const int64_t longest = std::min<int64_t>(n_kv, static_cast<int64_t>(n_past) + n_q);
    if (longest > 2 * BN)
      launch_nw<G, 4, 4>(q, k, v, out, n_head_kv, n_q, n_kv, n_past, scale_log2, 0, pg, s);
    else
      launch_nw<G, 2, 2>(q, k, v, out, n_head_kv, n_q, n_kv, n_past, scale_log2, 0, pg, s);
    return;
  }
  if (nw == 0) nw = blocks(4) * n_head_kv >= IKV_PREFILL_PAIR_MIN_WGS ? 4 : 2;
  const int nb = blocks(nw);
  const int paired = (nb >= 2 && (nb + 1) / 2 * n_head_kv >= IKV_PREFILL_PAIR_MIN_WGS) ? 1 : 0;
  // With at most one 4-wave workgroup per CU, each SIMD would run one wave:
  // give every block a second wave group instead (NW = 8).
  if (nw == 4 && IKV_PREFILL_SPLIT && n_head_kv * (paired ? (nb + 1) / 2 : nb) <= kCUs) nw = 8;
  if (nw == 8)
    launch_nw<G, 8, 2>(q, k, v, out, n_head_kv, n_q, n_kv, n_past, scale_log2, paired, pg, s);
  else if (nw == 4)
    launch_nw<G, 4, 1>(q, k, v, out, n_head_kv, n_q, n_kv, n_past, scale_log2, paired, pg, s);
  else
    launch_nw<G, 2, 1>(q, k, v, out, n_head_kv, n_q, n_kv, n_past, scale_log2, paired, pg, s);
}

}  // namespace

namespace {

int prefill_common(const float *q, const float *k, const float *v, const ikv_kv_pages *pages,
                   float *out, int n_head, int n_head_kv, int head_dim, int64_t n_q,
                   int64_t n_kv, int64_t n_past, float scale, void *stream) {
  if (n_q == 0) return 0;
  if (!q || !k || !v || !out) return -EINVAL;
  ikv::Pages pgv;
  const ikv::Pages *pg = nullptr;
  if (pages) {
    if (const int rc = ikv::pages_arg(pages, pgv)) return rc;
    pg = &pgv;
  }
  if (n_head <= 0 || n_head_kv <= 0 || n_head % n_head_kv != 0) return -EINVAL;
  if (n_q < 0 || n_kv <= 0 || n_past < 0) return -EINVAL;
  const int G = n_head / n_head_kv;
  if (head_dim != D || (G != 1 && G != 2 && G != 4 && G != 8)) {
    // other head sizes and groupings: the generic path
    if (!ikv::generic_attn_shape(n_head, n_head_kv, head_dim)) return -ENOTSUP;
    return ikv::attn_generic(q, k, v, pg, out, n_head, n_head_kv, head_dim, n_q, n_kv, n_past,
                             scale, static_cast<hipStream_t>(stream));
  }
  if (n_q > INT_MAX / 2 || n_kv > INT_MAX / 2 || n_past > INT_MAX / 2) return -EOVERFLOW;
  // a tile's 32 key rows (n_head_kv x 512 bytes each) are one buffer range
  if (n_head_kv > kMaxKvHeads) return -EOVERFLOW;
  if (!ikv::aligned16(q) || !ikv::aligned16(k) || !ikv::aligned16(v) || !ikv::aligned16(out))
    return -EINVAL;
  if (!(scale > 0.0f)) scale = 1.0f / sqrtf(static_cast<float>(head_dim));
  const float sl2 = scale * ikv::kLog2e;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nq = static_cast<int>(n_q), nk = static_cast<int>(n_kv), np = static_cast<int>(n_past);
  switch (G) {
    case 1: launch<1>(q, k, v, out, n_head_kv, nq, nk, np, sl2, pg, s); break;
    case 2: launch<2>(q, k, v, out, n_head_kv, nq, nk, np, sl2, pg, s); break;
    case 4: launch<4>(q, k, v, out, n_head_kv, nq, nk, np, sl2, pg, s); break;
    default: launch<8>(q, k, v, out, n_head_kv, nq, nk, np, sl2, pg, s); break;
  }
  return ikv::launch_status();
}

}  // namespace

extern "C" int ikv_attn_prefill_f32(const float *q, const float *k, const float *v, float *out,
                                    int n_head, int n_head_kv, int head_dim, int64_t n_q,
                                    int64_t n_kv, int64_t n_past, float scale, void *stream) {
  return prefill_common(q, k, v, nullptr, out, n_head, n_head_kv, head_dim, n_q, n_kv, n_past,
                        scale, stream);
}

extern "C" int ikv_attn_prefill_paged_f32(const float *q, const float *k_pool,
                                          const float *v_pool, const ikv_kv_pages *pages,
                                          float *out, int n_head, int n_head_kv, int head_dim,
                                          int64_t n_q, int64_t n_kv, int64_t n_past, float scale,
                                          void *stream) {
  if (!pages) return -EINVAL;
  return prefill_common(q, k_pool, v_pool, pages, out, n_head, n_head_kv, head_dim, n_q, n_kv,
                        n_past, scale, stream);
}
