// attn_decode.hip — GQA decode attention over the contiguous KV cache, split-K
// over the context, with the KV append of the new token fused in. One launch.
//
// Replaces the score + softmax kernel pair of CUDA_F32::compute_flash_attn for
// one query token (reference src/kernels/cuda/kernel_f32.cu:330-511), which
// launched one 32-thread block per score, materialised Hq*L scores, and
// allocated, synchronised and freed a buffer on every call. Semantics follow
// CPUBackend::compute_flash_attn (src/backends/cpu_backend.cpp:525-634):
// q head h reads KV head h / (n_head / n_head_kv); softmax(q.k * scale) . v.
//
// One workgroup (8 wavefronts) per (KV head g, context split).
// blockIdx = split * n_head_kv + g, so with 8 KV heads every split of head g
// lands on XCD g (workgroups are dealt to the 8 XCDs round-robin) and shares
// that XCD's L2. Each half-wave (32 lanes x float4) owns one 512-byte K or V
// row at a time: coalesced 16-byte non-temporal loads along the token-major
// cache ([token][kv head][128] F32, 4096 B per token at Qwen3 shapes), every
// row read from HBM once and used by all G query heads of the group. The next
// R rows per lane are prefetched into registers while the current ones are
// scored. Online softmax in base 2 per half-wave, merged across half-waves by
// lane exchange and across waves through LDS.
//
// Split merge, inside the same launch: every split publishes (max, sum,
// unnormalised output) for its G query heads with agent-coherent stores, waits
// for them to complete, and counts itself in the KV head's arrival counter
// (an agent-scope atomic; one counter per KV head, 256 bytes apart, so the 8
// heads never contend). The split that arrives last rescales and sums all
// partials of its head, loading every partial of a chunk of splits before
// using any (one memory round trip per chunk), writes the output, and resets
// the counter to zero for the next launch. Nothing waits or spins: every
// workgroup runs to completion whatever the arrival order. The workspace's
// counters must be zero before the first launch; each launch leaves them zero.
//
// Fused append: the row of the new token (n_kv-1) is read from k_new/v_new
// instead of the cache, and the workgroup that owns it stores it into the
// cache unchanged (a 16-byte copy, bit-exact).
//
// Fused qk-RMSNorm + RoPE (ikv_attn_decode_rope_f32): q and k_new arrive as
// projected; every workgroup stages its G query rows and the KV head's new
// key row in LDS, one lane per row adds the float squares in double in index
// order (the reference's loop), and all lanes then normalise and rotate the
// RoPE pairs with the resident sin/cos tables — the arithmetic of
// ikv_qk_norm_rope_f32 with contraction off, so the key row appended to the
// cache is bit-identical to the one the separate ops produce. The prologue's
// loads are issued first and the first tile's K/V loads right after them, so
// the prologue's arithmetic runs while the tile is in flight.
#include "attn_generic.hpp"
#include "coherent.hpp"
#include "gemv_dev.hpp"
#include "ikv_common.hpp"
#include "../../include/ikv.h"

#include <climits>
#include <mutex>

namespace {

// Phase timeline of the split decode, for the bench-only build of this file
// (IKV_DECODE_TIMELINE=1, libikv_bench.so; the product library has none of
// it): per workgroup, the 100 MHz s_memrealtime count at its entry, its first
// tile scored, its last tile scored (wave 0, and every wave), the waves
// merged in LDS, its partial published, the arrival counted, and (the
// merging workgroup) the merge done and its output stored.
#ifndef IKV_DECODE_TIMELINE
#define IKV_DECODE_TIMELINE 0
#endif
#if IKV_DECODE_TIMELINE
constexpr int kTimelineWgs = 1024;
constexpr int kTimelineWords = 16;
__device__ unsigned long long g_timeline[kTimelineWgs * kTimelineWords];
#endif
struct Timeline {
#if IKV_DECODE_TIMELINE
  unsigned long long t[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  bool first_done = false;
  __device__ void stamp(int i) { t[i] = __builtin_amdgcn_s_memrealtime(); }
  __device__ void first() {
    if (!first_done) stamp(1);
    first_done = true;
  }
  __device__ void wave_done(int slot, int wave) {
    if ((threadIdx.x & 63) == 0 && slot < kTimelineWgs)
      g_timeline[static_cast<size_t>(slot) * kTimelineWords + 8 + wave] = t[2];
  }
  // thread 0 writes the record; role 0 published, 1 merged, 2 one split
  __device__ void flush(int slot, int role) {
    if (threadIdx.x != 0 || slot >= kTimelineWgs) return;
    const unsigned xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20) & 15;  // HW_REG_XCC_ID
    t[7] = xcc | (static_cast<unsigned long long>(role) << 8);
    for (int i = 0; i < 8; ++i) g_timeline[static_cast<size_t>(slot) * kTimelineWords + i] = t[i];
  }
#else
  __device__ void stamp(int) {}
  __device__ void first() {}
  __device__ void wave_done(int, int) {}
  __device__ void flush(int, int) {}
#endif
};

constexpr int D = 128;  // head_dim supported by this kernel
#ifndef IKV_DECODE_NWAVE
#define IKV_DECODE_NWAVE 8
#endif
constexpr int NWAVE = IKV_DECODE_NWAVE;  // wavefronts per workgroup
constexpr int WG = NWAVE * 64;
#ifndef IKV_DECODE_R
// 2 (32-token tiles) against 4: ctx 4096 11.3 against 11.9 us per layer,
// the Qwen3-8B shape 12.2 against 13.2 us (27.1 against 30.5 at ctx 16384),
// faster at every context measured on MI355X (1: slower again)
#define IKV_DECODE_R 2
#endif
constexpr int R = IKV_DECODE_R;      // K and V rows per lane per iteration
constexpr int TILE = NWAVE * 2 * R;  // tokens per workgroup iteration
static_assert(64 % TILE == 0, "a paged block (a multiple of 64 tokens) must hold each tile whole");

#ifndef IKV_DECODE_TARGET_WGS
// Workgroups aimed for over all KV heads: one 8-wave workgroup per CU of
// MI355X's 256 (32 splits per head with 8 KV heads). One more split per
// head (264 workgroups) puts a second full split on 8 CUs, and those set
// the kernel's end: measured ctx 20000 40.9 against 31.1 us, ctx 4096 11.35
// against 10.16 us (the plan then takes 26 splits of 5 tiles), equal or
// slower at no context measured. Fewer splits keep the merge short (it
// reads G x splits x 512 B in one workgroup).
#define IKV_DECODE_TARGET_WGS 256
#endif
#ifndef IKV_DECODE_NT
#define IKV_DECODE_NT 1  // 1: K/V history read with non-temporal (streaming) loads
#endif

// Splits per KV head are capped so that G * n_splits <= kMergeCap.
constexpr int kMergeCap = 1024;
// Arrival counters: one int per KV head, kCounterStride ints apart.
constexpr int kCounterStride = 64;


// MI355X compute units.
constexpr int kCUs = 256;

// Waves per SIMD that decode_kernel<G> is built for (the second launch
// bound): 4 caps it at 128 VGPRs, which fits G <= 2; wider query groups need
// more registers (G = 4: ~172), so they get 2 (256 VGPRs) instead of spilling.
constexpr int waves_per_simd(int G) { return G <= 2 ? 4 : 2; }
// 8-wave workgroups resident per CU (4 SIMDs) at that bound.
constexpr int resident_wgs(int G) { return waves_per_simd(G) * 4 / NWAVE; }

struct Plan {
  int n_splits;
  int tokens_per_split;
};

// qk-RMSNorm + RoPE folded into the launch (all pointers device memory).
struct Prologue {
  const float *q_norm_w = nullptr, *k_norm_w = nullptr;
  float eps = 0.f;
  const int32_t *pos = nullptr;  // pos[0]: the new token's position
  const float *sin_tab = nullptr, *cos_tab = nullptr;
  int64_t n_ctx = 0;
  int *status = nullptr;
  // > 0: a launch recorded once and replayed at successive positions; the
  // context is pos[0] + 1, read on the device, and the launch was planned
  // for dyn_max keys (splits past pos[0] + 1 are empty).
  int dyn_max = 0;
  // 0, as a kernel argument: an offset the compiler cannot fold, so that a
  // load through it is a per-lane value that need not be waited for at once
  int zero = 0;
};

// The context of a launch: n_kv, or with pro.dyn_max, pos[0] + 1. A
// position outside [0, dyn_max) raises IKV_STATUS_POSITION and runs as
// dyn_max keys, inside the planned splits, with no append (*append false):
// the cache keeps every committed row.
// p: pos[0] when the launch is a replay form (loaded early by the caller).
__device__ __forceinline__ int launch_n_kv(const Prologue &pro, int n_kv, int p, bool &append) {
  append = true;
  if (pro.dyn_max <= 0) return n_kv;
  if (p >= 0 && p < pro.dyn_max) return p + 1;
  if (threadIdx.x == 0) ikv::raise_status(pro.status, IKV_STATUS_POSITION);
  append = false;
  return pro.dyn_max;
}

// Contexts this short run as one split per KV head (and can fold into the
// q/k/v projection's launch).
constexpr int kOneSplitTokens = 128;
static_assert(kOneSplitTokens % TILE == 0, "whole tiles");

#ifndef IKV_DECODE_MIN_SPLIT_TOKENS
// One tile per split at short contexts: 32 against 64 took 129 keys from
// 6.35 to 5.88 us per layer, 200..511 keys 0.55 us faster, equal from 1500
// keys on (MI355X, Qwen3-0.6B shape).
#define IKV_DECODE_MIN_SPLIT_TOKENS 32
#endif

// Most splits per KV head any context gets: `target` workgroups over the KV
// heads, at most kMergeCap / G so that the merge's weights fit in LDS.
int max_splits(int n_head, int n_head_kv) {
  const int G = n_head / n_head_kv;
  // With one resident workgroup per CU, the workgroups past 256 would run as
  // a second wave behind the first: stay at one per CU.
  const int target_wgs = resident_wgs(G) >= 2 ? IKV_DECODE_TARGET_WGS : kCUs;
  int target = (target_wgs + n_head_kv - 1) / n_head_kv;
  if (target > kMergeCap / G) target = kMergeCap / G;
  return target;
}

Plan plan_for(int n_head, int n_head_kv, int64_t n_kv) {
  // Whole tiles per split; at most max_splits per KV head and at least
  // IKV_DECODE_MIN_SPLIT_TOKENS tokens per split.
  int64_t target = max_splits(n_head, n_head_kv);
  const int64_t by_min = (n_kv + IKV_DECODE_MIN_SPLIT_TOKENS - 1) / IKV_DECODE_MIN_SPLIT_TOKENS;
  if (target > by_min) target = by_min;
  // Up to kOneSplitTokens keys one workgroup per KV head is faster than any
  // split: the further tiles cost less than the merge (measured on MI355X:
  // 127 tokens take 5.4 us in one split, 6.7 us in two).
  if (n_kv <= kOneSplitTokens) target = 1;
  if (target < 1) target = 1;
  const int64_t n_tiles = (n_kv + TILE - 1) / TILE;
  int64_t tiles_per_split = (n_tiles + target - 1) / target;
  // Splits of exactly 4 tiles (128 keys, 512 KB of cache rows apart) run
  // slower than 5-tile ones with fewer splits: measured on MI355X over 3073
  // to 4096 keys, 0.3..1.1 us per layer (Qwen3-0.6B shape) and 0.1..0.7 us
  // (Qwen3-8B shape) in favour of 5; no other length measured showed it.
  if (tiles_per_split == 4) tiles_per_split = 5;
  const int64_t tokens = tiles_per_split * TILE;
  const int64_t splits = (n_kv + tokens - 1) / tokens;
  return {static_cast<int>(splits), static_cast<int>(tokens)};
}

size_t align256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

struct WsLayout {
  size_t counters, part_ml, part_o, total;
};

// [n_head_kv counters, 256 B apart][n_head x n_splits x (max, sum)]
// [n_head x n_splits x D]. Every launch leaves the counters at zero, so one
// workspace serves every context length of a shape.
WsLayout ws_layout(int n_head, int n_head_kv, int n_splits) {
  WsLayout w;
  w.counters = 0;
  w.part_ml = align256(sizeof(int) * kCounterStride * static_cast<size_t>(n_head_kv));
  w.part_o = w.part_ml + align256(sizeof(float) * 2 * static_cast<size_t>(n_head) * n_splits);
  w.total = w.part_o + sizeof(float) * static_cast<size_t>(n_head) * n_splits * D;
  return w;
}

using ikv::f2v;
using ikv::f4v;
using ikv::load2_agent;
using ikv::load4_agent;
using ikv::load_agent;
using ikv::partial_rsrc;
using ikv::store2_agent;
using ikv::store4_agent;
using ikv::store_agent;

// Loads the K and V rows of tile `base` for this lane: row r of the lane is
// token base + r*2*NWAVE + 2*wave + half. Rows past the split (t > t_last)
// are clamped to t_last and scored -inf by the caller, so every lane issues
// the same unconditional loads (no branch between a load and its use, which
// keeps the next tile's loads in flight while this one is scored). The new
// token's row comes from k_new / v_new. Token t is read from cache row
// t + shift (shift = 0 for a contiguous cache; a paged cache's block offset,
// the same for the whole tile).
//
// With COH (k_new / v_new written by other workgroups of the same launch)
// the new token's row is loaded from the cache like the others (stale, in
// bounds) and the caller substitutes the new row it loaded coherently.
template <bool COH = false>
__device__ __forceinline__ void load_tile(float4 (&kr)[R], float4 (&vr)[R], int base, int t_last,
                                          int wave, int half, int new_row, const float *kc,
                                          const float *vc, const float *k_new, const float *v_new,
                                          size_t tok_stride, size_t head_off, int64_t shift) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int t = min(base + r * (NWAVE * 2) + wave * 2 + half, t_last);
    const bool fresh = !COH && (t == new_row);
    const size_t row = static_cast<size_t>(t + shift) * tok_stride + head_off;
    const float *kp = fresh ? k_new + head_off : kc + row;
    const float *vp = fresh ? v_new + head_off : vc + row;
#if IKV_DECODE_NT
    const f4v ka = __builtin_nontemporal_load(reinterpret_cast<const f4v *>(kp));
    const f4v va = __builtin_nontemporal_load(reinterpret_cast<const f4v *>(vp));
    kr[r] = make_float4(ka.x, ka.y, ka.z, ka.w);
    vr[r] = make_float4(va.x, va.y, va.z, va.w);
#else
    kr[r] = *reinterpret_cast<const float4 *>(kp);
    vr[r] = *reinterpret_cast<const float4 *>(vp);
#endif
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

// merge_waves for output columns 4c .. 4c + 3 of query head h.
template <int G>
__device__ __forceinline__ void merge_waves4(const float (&s_acc)[NWAVE][G][D],
                                             const float (&s_m)[NWAVE][G],
                                             const float (&s_l)[NWAVE][G], int h, int c, float4 &O,
                                             float &L, float &M) {
  M = -INFINITY;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) M = fmaxf(M, s_m[w][h]);
  O = make_float4(0.f, 0.f, 0.f, 0.f);
  L = 0.f;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) {
    const float mw = s_m[w][h];
    const float e = (mw == -INFINITY) ? 0.f : ikv::fast_exp2(mw - M);
    O = ikv::fma4(e, *reinterpret_cast<const float4 *>(&s_acc[w][h][4 * c]), O);
    L = fmaf(s_l[w][h], e, L);
  }
}

// The register stage of the folded qk-norm + RoPE prologue: this thread's
// elements of q rows g*G .. g*G+G-1 and of the new key row of KV head g, and
// for its RoPE pairs the norm weights and the sin/cos of row n_kv - 1 (the
// new token's position whenever the caller's positions follow the cache, as
// in a decode step). The kernel issues these loads before those of its first
// K/V tile, so that waiting for them does not wait for the tile, and the
// prologue's arithmetic runs while the tile is in flight.
// Row stride of the prologue's LDS rows: 4 floats of padding put the G+1
// rows that the summing lanes read in lockstep on different banks.
constexpr int kRowPad = D + 4;

template <int G>
struct ProStage {
  static constexpr int hd = D / 2;
  static constexpr int n_el = (G + 1) * D;
  static constexpr int EPT = (n_el + WG - 1) / WG;
  static constexpr int n_pairs = (G + 1) * hd;
  static constexpr int PPT = (n_pairs + WG - 1) / WG;
  float el[EPT];
  float w0[PPT], w1[PPT], cs[PPT], sn[PPT];
  int32_t p;
  int spec;
};

template <int G, bool COH>
__device__ __forceinline__ void qk_prologue_load(const Prologue &pro, const float *q, const float *k_new,
                                                 int g, int n_kv, ProStage<G> &st) {
  using S = ProStage<G>;
  const int tid = threadIdx.x;
#pragma unroll
  for (int u = 0; u < S::EPT; ++u) {
    const int i = tid + u * WG;
    if (i < S::n_el) {
      const int r = i / D;
      const int d = i - r * D;
      const float *p = r < G ? q + static_cast<size_t>(g * G + r) * D + d
                             : k_new + static_cast<size_t>(g) * D + d;
      if constexpr (COH)
        st.el[u] = load_agent(p);
      else
        st.el[u] = *p;
    }
  }
  st.spec = min(n_kv - 1, static_cast<int>(min(pro.n_ctx, static_cast<int64_t>(INT_MAX))) - 1);
#pragma unroll
  for (int u = 0; u < S::PPT; ++u) {
    const int i = tid + u * WG;
    if (i < S::n_pairs) {
      const int r = i / S::hd;
      const int j = i - r * S::hd;
      const float *w = r < G ? pro.q_norm_w : pro.k_norm_w;
      st.w0[u] = w[j];
      st.w1[u] = w[j + S::hd];
      st.cs[u] = pro.cos_tab[static_cast<int64_t>(st.spec) * S::hd + j];
      st.sn[u] = pro.sin_tab[static_cast<int64_t>(st.spec) * S::hd + j];
    }
  }
  st.p = pro.pos[0];
}

// Completes the prologue from the register stage: s[h] = rope(norm(q_h)),
// s[G] = rope(norm(k_g)), RMSNorm with an ordered double sum per row (one
// lane per row) and NeoX RoPE at position pos[0]; if pos[0] is not the row
// staged, that row's sin/cos are loaded here. A position outside
// [0, n_ctx) reads row 0 (in bounds), gives zero rows and raises *status.
template <int G>
__device__ __forceinline__ void qk_prologue(const Prologue &pro, ProStage<G> &st,
                                            float (&s)[G + 1][kRowPad], float (&scl)[G + 1]) {
#pragma clang fp contract(off)
  using S = ProStage<G>;
  const int tid = threadIdx.x;
  constexpr int hd = S::hd;
  constexpr int n_pairs = S::n_pairs;
  constexpr int PPT = S::PPT;
  float(&w0)[PPT] = st.w0;
  float(&w1)[PPT] = st.w1;
  float(&cs)[PPT] = st.cs;
  float(&sn)[PPT] = st.sn;
  const int32_t p = st.p;
  const bool ok = p >= 0 && p < pro.n_ctx;
  const int prow = ok ? p : 0;
  if (prow != st.spec) {
#pragma unroll
    for (int u = 0; u < PPT; ++u) {
      const int i = tid + u * WG;
      if (i < n_pairs) {
        const int j = i - (i / hd) * hd;
        cs[u] = pro.cos_tab[static_cast<int64_t>(prow) * hd + j];
        sn[u] = pro.sin_tab[static_cast<int64_t>(prow) * hd + j];
      }
    }
    // These loads were issued after the first tile's. Waiting for them here
    // (vmcnt(0); expcnt and lgkmcnt left at their maxima) keeps that wait on
    // this rare path: otherwise the compiler's wait where the paths join
    // would also hold the common path until its tile has landed.
    __builtin_amdgcn_s_waitcnt(0x0F70);
  }
#pragma unroll
  for (int u = 0; u < S::EPT; ++u) {
    const int i = tid + u * WG;
    if (i < S::n_el) s[i / D][i - (i / D) * D] = st.el[u];
  }
  __syncthreads();
  {
    // Row r's sum of squares by half-wave r: lane c adds the squares of
    // elements 4c..4c+3, a xor butterfly over the half-wave adds the lanes
    // (8 roundings on any term's path), and the scale is certified against
    // the reference's index-order sum (127 roundings); lane 0 redoes the sum
    // in index order when it is not certain. The ordered sum alone is a
    // chain of 128 dependent double adds, about 1.1 us on MI355X.
    static_assert((G + 1) * 32 <= WG, "a half-wave per row");
    const int r = tid >> 5;
    const int c = tid & 31;
    if (r <= G) {
      const float4 v = *reinterpret_cast<const float4 *>(&s[r][4 * c]);
      const float a = v.x * v.x, b = v.y * v.y, e = v.z * v.z, f = v.w * v.w;
      double part = static_cast<double>(a);
      part += static_cast<double>(b);
      part += static_cast<double>(e);
      part += static_cast<double>(f);
      part = ikv::half_wave_sum_f64(part);
      float sc = 0.f;
      const bool certain = ikv::certified_rms_scale(part, D, pro.eps, (D - 1) + 8, sc);
      if (c == 0) scl[r] = certain ? sc : ikv::ordered_rms_scale(&s[r][0], D, pro.eps);
    }
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < PPT; ++u) {
    const int i = tid + u * WG;
    if (i >= n_pairs) break;
    const int r = i / hd;
    const int j = i - r * hd;
    const float sc = scl[r];
    const float t0 = s[r][j] * sc;
    const float t1 = s[r][j + hd] * sc;
    const float x0 = t0 * w0[u];
    const float x1 = t1 * w1[u];
    float o0 = 0.f, o1 = 0.f;
    if (ok) {
      const float a = x0 * cs[u];
      const float b = x1 * sn[u];
      const float e = x0 * sn[u];
      const float f = x1 * cs[u];
      o0 = a - b;
      o1 = e + f;
    }
    s[r][j] = o0;
    s[r][j + hd] = o1;
  }
  if (!ok && tid == 0) ikv::raise_status(pro.status, IKV_STATUS_POSITION);
  __syncthreads();
}

// The merging workgroup's 16 half-waves ("units") split the work: unit u
// serves query head u % G of the group and sums the splits s = k, k + U,
// k + 2U, ... (k = u / G, U = 16 / G units per head), lane c of the unit
// owning output columns 4c .. 4c + 3. A unit loads the (max, sum) record and
// its 16-byte piece of the partial output of every split it sums, J splits
// per round, all loads of a round issued before any is used and none behind
// a branch (one memory round trip for up to J * U splits per head: J = 4 / 8
// / 16 for G <= 2 / 4 / 8, so a round covers 32 splits at G >= 2), and folds
// them into its own (max, sum, output) in registers. The units of a head
// then combine through LDS. (Fewer units with more loads each, a wavefront
// per query head combining its halves by lane swaps, measured slower: the
// merge is bound by how fast one CU issues its loads.)
constexpr int kMergeUnits = WG / 32;

struct MergeLds {
  float4 acc[kMergeUnits][32];  // per unit and lane: unnormalised output
  float m[kMergeUnits];         // per unit: max
  float l[kMergeUnits];         // per unit: sum
};

// Run by the last split of KV head g to arrive: out = sum_s w_s O_s / sum_s w_s l_s
// over the n_splits partials of each of the G query heads, w_s = 2^(m_s - max).
template <int G>
__device__ __forceinline__ void merge_splits(const float *part_ml, const float *part_o, float *out,
                                             int g, int n_splits, MergeLds &lds) {
  constexpr int U = kMergeUnits / G;  // units per query head
  // rounds of J splits per unit until every split is summed:
  // ceil(n_splits / (U * J)), one for the plans of the Qwen3 shapes
  constexpr int J = G <= 2 ? 4 : (G == 4 ? 8 : 16);
  const int tid = threadIdx.x;
  const int u = tid >> 5;
  const int c = tid & 31;
  const int hh = u % G;
  const int k = u / G;
  const int S = n_splits;
  // This KV head's partials: G x S (max, sum) pairs and G x S x D outputs.
  // Raw buffer loads past the end of a range return zeros; a split index past
  // S inside the range reads another head's record, which the mask drops.
  const __amdgpu_buffer_rsrc_t rml =
      partial_rsrc(part_ml + static_cast<size_t>(g * G) * S * 2, sizeof(float) * 2 * G * S);
  const __amdgpu_buffer_rsrc_t ro =
      partial_rsrc(part_o + static_cast<size_t>(g * G) * S * D, sizeof(float) * G * S * D);
  float M = -INFINITY, L = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = k; s0 < S; s0 += U * J) {
    float mj[J], lj[J], ox[J], oy[J], oz[J], ow[J];
    // The partials were published with agent-coherent stores before their
    // workgroups were counted; agent-coherent loads observe them.
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const unsigned r = static_cast<unsigned>(hh * S + s0 + j * U);
      const float2 st = load2_agent(rml, r * static_cast<unsigned>(sizeof(float) * 2));
      const float4 v = load4_agent(ro, r * static_cast<unsigned>(sizeof(float) * D) + 16u * c);
      mj[j] = (s0 + j * U < S) ? st.x : -INFINITY;
      lj[j] = st.y;
      ox[j] = v.x;
      oy[j] = v.y;
      oz[j] = v.z;
      ow[j] = v.w;
    }
    float mx = M;
#pragma unroll
    for (int j = 0; j < J; ++j) mx = fmaxf(mx, mj[j]);
    // with every record so far masked (mx = -inf) nothing is added
    const float ref = (mx == -INFINITY) ? 0.f : mx;
    const float alpha = ikv::fast_exp2(M - ref);
    L *= alpha;
    acc = ikv::scale4(alpha, acc);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const float e = ikv::fast_exp2(mj[j] - ref);
      L = fmaf(e, lj[j], L);
      acc = make_float4(fmaf(e, ox[j], acc.x), fmaf(e, oy[j], acc.y), fmaf(e, oz[j], acc.z),
                        fmaf(e, ow[j], acc.w));
    }
    M = mx;
  }
  lds.acc[u][c] = acc;
  if (c == 0) {
    lds.m[u] = M;
    lds.l[u] = L;
  }
  __syncthreads();
  if (tid < G * 32) {
    // tid < G * 32: unit tid >> 5 = hh is this head's first unit
    float Mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < U; ++q) Mx = fmaxf(Mx, lds.m[hh + q * G]);
    float Ls = 0.f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int q = 0; q < U; ++q) {
      const int uu = hh + q * G;
      const float mq = lds.m[uu];
      const float w = (mq == -INFINITY) ? 0.f : ikv::fast_exp2(mq - Mx);
      Ls = fmaf(w, lds.l[uu], Ls);
      o = ikv::fma4(w, lds.acc[uu][c], o);
    }
    *reinterpret_cast<float4 *>(out + static_cast<size_t>(g * G + hh) * D + 4 * c) =
        make_float4(o.x / Ls, o.y / Ls, o.z / Ls, o.w / Ls);
  }
}

// One workgroup's share of a decode: KV head g, split `split`. COH: q, k_new
// and v_new were written by other workgroups of the same launch (the folded
// q/k/v projection) and are read with agent-coherent loads.
template <int G, bool PRO, bool PAGED, bool COH>
__device__ __forceinline__ void decode_body(
    const float *q, float *kc, float *vc, const float *k_new, const float *v_new,
    float *__restrict__ out, int *counters, float *part_ml, float *part_o, int n_head_kv, int n_kv,
    int tokens_per_split, int n_splits, float scale_log2, const Prologue &pro,
    const ikv::Pages &pages, int g, int split, bool append = true) {
  static_assert(!COH || PRO, "the coherent form is the one with the prologue folded in");
  // Arrays read or written as float4 are declared 16-byte aligned.
  __shared__ __attribute__((aligned(16))) float s_acc[NWAVE][G][D];
  __shared__ float s_m[NWAVE][G];
  __shared__ float s_l[NWAVE][G];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = lane >> 5;
  const int sub = lane & 31;
  Timeline tl;
  tl.stamp(0);
  const int tl_slot = split * n_head_kv + g;
  const int t_begin = split * tokens_per_split;
  const int t_end = min(n_kv, t_begin + tokens_per_split);
  // the new token's row: read from k_new / v_new and appended (none when the
  // launch's position was rejected: then row n_kv - 1 is read from the cache)
  const int new_row = (k_new && append) ? n_kv - 1 : -1;
  const size_t tok_stride = static_cast<size_t>(n_head_kv) * D;
  const size_t head_off = static_cast<size_t>(g) * D + 4 * sub;

  // Cache row offset of the tile at token `base`: tiles start at multiples
  // of TILE from a split start (itself a multiple of TILE), so a paged
  // cache's block (a multiple of 64 tokens) holds each tile whole. The
  // offsets of the first kSplitBlocks blocks the split reads are loaded
  // together at its start (their table loads overlap each other and the
  // prologue), so no tile's loads wait on a table load; a longer split looks
  // the later blocks up as it reaches them. Only entries of blocks that hold
  // keys of [t_begin, t_end) are read (an empty split of a replay launch
  // reads the block of the context's last key).
  constexpr int kSplitBlocks = 4;
  int64_t blk_shift[kSplitBlocks] = {};
  int first_block = 0;
  if constexpr (PAGED) {
    first_block = min(t_begin, t_end - 1) / pages.bt;
    const int last_block = (t_end - 1) / pages.bt;
#pragma unroll
    for (int i = 0; i < kSplitBlocks; ++i)
      if (first_block + i <= last_block)
        blk_shift[i] = ikv::page_shift(pages, (first_block + i) * pages.bt);
  }
  auto shift_of = [&](int base) -> int64_t {
    if constexpr (PAGED) {
      const int i = base / pages.bt - first_block;
      int64_t sh = 0;
      bool hit = false;
#pragma unroll
      for (int j = 0; j < kSplitBlocks; ++j)
        if (i == j) {
          sh = blk_shift[j];
          hit = true;
        }
      return hit ? sh : ikv::page_shift(pages, base);
    } else {
      return 0;
    }
  };

  // Two register buffers of K/V rows: tile t+1 loads into one while tile t
  // is scored from the other.
  float4 ka[R], va[R], kb[R], vb[R];
  ProStage<G> st;
  if constexpr (PRO) qk_prologue_load<G, COH>(pro, q, k_new, g, n_kv, st);
  // the new token's V piece of this lane, when it cannot be read with the tiles
  float4 vnew = make_float4(0.f, 0.f, 0.f, 0.f);
  if constexpr (COH) {
    const float *p = v_new + head_off;
    vnew = make_float4(load_agent(p), load_agent(p + 1), load_agent(p + 2), load_agent(p + 3));
  }
  // (an empty split of a replay launch, past the context, clamps every row
  // onto the context's last one: its block, not the unallocated one at
  // t_begin)
  load_tile<COH>(ka, va, t_begin, t_end - 1, wave, half, new_row, kc, vc, k_new, v_new, tok_stride,
                 head_off, shift_of(min(t_begin, t_end - 1)));

  float4 qv[G];
  float4 knew_rot = make_float4(0.f, 0.f, 0.f, 0.f);  // this lane's piece of rope(norm(k_new))
  if constexpr (PRO) {
    __shared__ __attribute__((aligned(16))) float s_qk[G + 1][kRowPad];
    __shared__ float s_scl[G + 1];
    qk_prologue<G>(pro, st, s_qk, s_scl);
#pragma unroll
    for (int h = 0; h < G; ++h) qv[h] = *reinterpret_cast<const float4 *>(&s_qk[h][4 * sub]);
    knew_rot = *reinterpret_cast<const float4 *>(&s_qk[G][4 * sub]);
  } else {
#pragma unroll
    for (int h = 0; h < G; ++h)
      qv[h] = *reinterpret_cast<const float4 *>(q + static_cast<size_t>(g * G + h) * D + 4 * sub);
  }

  float m[G], l[G];
  float4 acc[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
    acc[h] = make_float4(0.f, 0.f, 0.f, 0.f);
  }

  // Scores and accumulates one tile. Branch-free: masked rows are -inf
  // scores, and with the folded RoPE the new token's key is swapped for the
  // rotated one by a select.
  auto process = [&](float4 (&kr)[R], float4 (&vr)[R], int base) {
    if constexpr (PRO) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        // The row this lane loaded: rows past the split were clamped onto
        // its last, which may be the new token's. Its cache row is not yet
        // written (its bytes are whatever the memory held): a masked row
        // still multiplies its V by a zero weight, so it must get the new
        // row's finite values too.
        const bool fresh = min(base + r * (NWAVE * 2) + wave * 2 + half, t_end - 1) == new_row;
        kr[r].x = fresh ? knew_rot.x : kr[r].x;
        kr[r].y = fresh ? knew_rot.y : kr[r].y;
        kr[r].z = fresh ? knew_rot.z : kr[r].z;
        kr[r].w = fresh ? knew_rot.w : kr[r].w;
        if constexpr (COH) {
          vr[r].x = fresh ? vnew.x : vr[r].x;
          vr[r].y = fresh ? vnew.y : vr[r].y;
          vr[r].z = fresh ? vnew.z : vr[r].z;
          vr[r].w = fresh ? vnew.w : vr[r].w;
        }
      }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float sc[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int t = base + r * (NWAVE * 2) + wave * 2 + half;
        const float dq = ikv::dot4(qv[h], kr[r]);
        const float d = G <= 2 ? ikv::half_wave_sum_valu(dq) : ikv::half_wave_sum(dq);
        sc[r] = (t < t_end) ? d * scale_log2 : -INFINITY;
      }
      float mx = m[h];
#pragma unroll
      for (int r = 0; r < R; ++r) mx = fmaxf(mx, sc[r]);
      // No branch on mx: with every score so far masked (mx = -inf) the
      // reference point is 0, so alpha and every p are exactly 0.
      const float ref = (mx == -INFINITY) ? 0.f : mx;
      const float alpha = ikv::fast_exp2(m[h] - ref);
      l[h] *= alpha;
      acc[h] = ikv::scale4(alpha, acc[h]);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float p = ikv::fast_exp2(sc[r] - ref);
        l[h] += p;
        acc[h] = ikv::fma4(p, vr[r], acc[h]);
      }
      m[h] = mx;
    }
    tl.first();
  };
  // Ping-pong over the split's tiles. The tail cases get their own calls so
  // that on every path the next tile's loads are issued unconditionally
  // before the current tile is scored: the compiler's wait then covers only
  // the current tile's loads.
  for (int base = t_begin;; base += 2 * TILE) {
    if (base + TILE >= t_end) {
      process(ka, va, base);
      break;
    }
    load_tile<COH>(kb, vb, base + TILE, t_end - 1, wave, half, new_row, kc, vc, k_new, v_new,
                   tok_stride, head_off, shift_of(base + TILE));
    process(ka, va, base);
    if (base + 2 * TILE >= t_end) {
      process(kb, vb, base + TILE);
      break;
    }
    load_tile<COH>(ka, va, base + 2 * TILE, t_end - 1, wave, half, new_row, kc, vc, k_new, v_new,
                   tok_stride, head_off, shift_of(base + 2 * TILE));
    process(kb, vb, base + TILE);
  }

  tl.stamp(2);
  tl.wave_done(tl_slot, wave);
  // The append: the split holding the new token writes its K (rotated when
  // RoPE is folded in) and V rows into the caches, 16 bytes per lane of the
  // first half-wave.
  bool append_here = new_row >= t_begin && new_row < t_end && wave == 0 && half == 0;
  if constexpr (PAGED) append_here = append_here && ikv::page_ok(pages, new_row);
  if (append_here) {
    const size_t off = static_cast<size_t>(new_row + shift_of(new_row)) * tok_stride + head_off;
    float4 kw;
    if constexpr (PRO)
      kw = knew_rot;
    else
      kw = *reinterpret_cast<const float4 *>(k_new + head_off);
    *reinterpret_cast<float4 *>(kc + off) = kw;
    if constexpr (COH)
      *reinterpret_cast<float4 *>(vc + off) = vnew;
    else
      *reinterpret_cast<float4 *>(vc + off) = *reinterpret_cast<const float4 *>(v_new + head_off);
  }

  // Merge the two half-waves (they saw different tokens): lanes i and i ^ 32
  // swap values (v_permlane32_swap), and every lane combines the pair in the
  // same order, so both halves hold the same bits.
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float2 mm = ikv::halves(m[h]);
    const float2 ll = ikv::halves(l[h]);
    const float2 ax = ikv::halves(acc[h].x), ay = ikv::halves(acc[h].y);
    const float2 az = ikv::halves(acc[h].z), aw = ikv::halves(acc[h].w);
    const float M = fmaxf(mm.x, mm.y);
    const float a = (M == -INFINITY) ? 0.f : ikv::fast_exp2(mm.x - M);
    const float b = (M == -INFINITY) ? 0.f : ikv::fast_exp2(mm.y - M);
    l[h] = ll.x * a + ll.y * b;
    acc[h] = make_float4(ax.x * a + ax.y * b, ay.x * a + ay.y * b, az.x * a + az.y * b,
                         aw.x * a + aw.y * b);
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
  tl.stamp(3);

  // Merge the waves. With one split the result is final.
  if (n_splits == 1) {
    for (int idx = tid; idx < G * D; idx += WG) {
      const int h = idx / D;
      const int d = idx - h * D;
      float O, L, M;
      merge_waves<G>(s_acc, s_m, s_l, h, d, O, L, M);
      out[static_cast<size_t>(g * G + h) * D + d] = O / L;
    }
    tl.flush(tl_slot, 2);
    return;
  }
  // Publish: wave 0 merges the waves and stores the workgroup's (max, sum,
  // unnormalised output) agent-coherently, 16 bytes per lane and column;
  // once its stores have completed (vmcnt counts stores on CDNA) it counts
  // the workgroup in the KV head's arrival counter. The split that arrives
  // last merges the head and resets the counter for the next launch.
  __shared__ int s_last;
  if (wave == 0) {
    const __amdgpu_buffer_rsrc_t ro = partial_rsrc(
        part_o + static_cast<size_t>(g * G) * n_splits * D, sizeof(float) * G * n_splits * D);
#pragma unroll
    for (int i = lane; i < G * 32; i += 64) {
      const int h = i >> 5;
      const int c = i & 31;
      float4 O;
      float L, M;
      merge_waves4<G>(s_acc, s_m, s_l, h, c, O, L, M);
      const int slot = h * n_splits + split;  // within this KV head's partials
      store4_agent(ro, static_cast<unsigned>(sizeof(float) * (slot * D + 4 * c)), O);
      if (c == 0) store2_agent(part_ml + 2 * (static_cast<size_t>(g * G) * n_splits + slot), M, L);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    tl.stamp(4);
    if (lane == 0) {
      int *ctr = counters + static_cast<size_t>(g) * kCounterStride;
      const int before =
          __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = (before == n_splits - 1);
      if (s_last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  tl.stamp(5);
  if (!s_last) {
    tl.flush(tl_slot, 0);
    return;
  }
  __shared__ __attribute__((aligned(16))) MergeLds s_merge;
  merge_splits<G>(part_ml, part_o, out, g, n_splits, s_merge);
#if IKV_DECODE_TIMELINE
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  tl.stamp(6);
  tl.flush(tl_slot, 1);
#endif
}

template <int G, bool PRO, bool PAGED>
__global__ __launch_bounds__(WG, waves_per_simd(G)) void decode_kernel(
    const float *__restrict__ q, float *kc, float *vc, const float *k_new, const float *v_new,
    float *__restrict__ out, int *counters, float *part_ml, float *part_o, int n_head_kv, int n_kv,
    int tokens_per_split, int n_splits, float scale_log2, Prologue pro, ikv::Pages pages) {
  bool append = true;
  if constexpr (PRO) n_kv = launch_n_kv(pro, n_kv, pro.dyn_max > 0 ? pro.pos[0] : 0, append);
  decode_body<G, PRO, PAGED, false>(q, kc, vc, k_new, v_new, out, counters, part_ml, part_o,
                                    n_head_kv, n_kv, tokens_per_split, n_splits, scale_log2, pro,
                                    pages, static_cast<int>(blockIdx.x) % n_head_kv,
                                    static_cast<int>(blockIdx.x) / n_head_kv, append);
}

// ---------------------------------------------------------------------------
// The q/k/v projection of a one-token step with the short-context decode
// folded in (ikv_qkv_attn_decode_f32). Every workgroup first computes 16 rows
// of [q | k | v] = [w_q | w_k | w_v] x (with the attn_norm of x folded in),
// 2 per wave, exactly as the q/k/v product ikv_gemv3_f32 does (the same
// device code), and stores them agent-coherently. The 16 rows of a workgroup
// belong to one KV head g (D and the group's G * D q rows are multiples of
// 16); a per-head arrival counter finds the last of the head's workgroups to
// finish, and that workgroup runs the head's decode (qk-norm + RoPE + append
// + attention over n_kv <= kOneSplitTokens keys, one split) with the decode
// kernel's device code, reading the head's q, k and v rows back coherently. The
// outputs are bit-identical to the separate launches; the decode's launch,
// its ramp and its wait for the projection's last wave are gone.
constexpr int kQkvRpw = 2;                        // rows per wave
constexpr int kQkvRowsPerWg = NWAVE * kQkvRpw;    // 16
static_assert(D % kQkvRowsPerWg == 0, "a workgroup's rows stay within one head");

// Built for 2 waves per SIMD (256 VGPRs): the projection's and the decode's
// registers together do not fit 128, and one 8-wave workgroup per CU is the
// launch's occupancy anyway at the widths it serves (Qwen3-0.6B: 256
// workgroups).
template <int G>
__global__ __launch_bounds__(WG, 2) void qkv_attn_kernel(
    const float *__restrict__ wq, const float *__restrict__ wk, const float *__restrict__ wv,
    const float *__restrict__ x, const float *attn_norm_w, float attn_eps, float *q_out,
    float *k_out, float *v_out, int K, float *kc, float *vc, float *out, int *counters,
    int n_head_kv, int n_kv, int tokens_per_split, float scale_log2, Prologue pro) {
  // A replay form's position, loaded before the projection's weights: the
  // decode that needs it then does not wait for it. Through a per-lane
  // address (an offset of pro.zero): a uniform load would be waited for at
  // once, to move it to a scalar register.
  const int pos_lane = pro.pos[threadIdx.x & pro.zero];
  const int n0 = n_head_kv * G * D;  // q rows
  const int n1 = n_head_kv * D;      // k rows, v rows
  const int lane = threadIdx.x & 63;
  const int wg_row0 = static_cast<int>(blockIdx.x) * kQkvRowsPerWg;
  int row0 = wg_row0 + (static_cast<int>(threadIdx.x) >> 6) * kQkvRpw;
  const float *w;
  float *o;
  int g;
  if (wg_row0 < n0) {
    w = wq;
    o = q_out;
    g = wg_row0 / (G * D);
  } else if (wg_row0 < n0 + n1) {
    w = wk;
    o = k_out;
    row0 -= n0;
    g = (wg_row0 - n0) / D;
  } else {
    w = wv;
    o = v_out;
    row0 -= n0 + n1;
    g = (wg_row0 - n0 - n1) / D;
  }
  const float *rows[kQkvRpw];
#pragma unroll
  for (int r = 0; r < kQkvRpw; ++r) rows[r] = w + static_cast<size_t>(row0 + r) * K;
  float sums[kQkvRpw];
  ikv::gemv::wave_dots<kQkvRpw>(rows, x, K, sums, attn_norm_w, attn_eps);
  if (lane < kQkvRpw) {
    float v = sums[0];
#pragma unroll
    for (int r = 1; r < kQkvRpw; ++r)
      if (lane == r) v = sums[r];
    store_agent(o + row0 + lane, v);
  }
  // Publish: the row stores have completed (vmcnt counts stores) before the
  // workgroup's arrival is counted.
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  __shared__ int s_last_qkv;
  if (threadIdx.x == 0) {
    constexpr int per_head = (G + 2) * D / kQkvRowsPerWg;
    int *ctr = counters + static_cast<size_t>(g) * kCounterStride;
    const int before = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last_qkv = (before == per_head - 1);
    if (s_last_qkv) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last_qkv) return;
  bool append = true;
  const int n_kv_launch =
      launch_n_kv(pro, n_kv, __builtin_amdgcn_readfirstlane(pos_lane), append);
  decode_body<G, true, false, true>(q_out, kc, vc, k_out, v_out, out, counters, nullptr, nullptr,
                                    n_head_kv, n_kv_launch, tokens_per_split, 1, scale_log2, pro,
                                    ikv::Pages{}, g, 0, append);
}

bool supported_group(int G) { return G == 1 || G == 2 || G == 4 || G == 8; }

template <int G, bool PRO, bool PAGED>
void launch_one(const float *q, float *kc, float *vc, const float *kn, const float *vn, float *out,
                int *counters, float *part_ml, float *part_o, int n_head_kv, int n_kv,
                const Plan &p, float scale_log2, const Prologue &pro, const ikv::Pages &pg,
                hipStream_t s) {
  decode_kernel<G, PRO, PAGED><<<n_head_kv * p.n_splits, WG, 0, s>>>(
      q, kc, vc, kn, vn, out, counters, part_ml, part_o, n_head_kv, n_kv, p.tokens_per_split,
      p.n_splits, scale_log2, pro, pg);
}

template <int G>
void launch(const float *q, float *kc, float *vc, const float *kn, const float *vn, float *out,
            int *counters, float *part_ml, float *part_o, int n_head_kv, int n_kv, const Plan &p,
            float scale_log2, const Prologue *pro, const ikv::Pages *pg, hipStream_t s) {
  const Prologue none{};
  const ikv::Pages flat{};
  if (pro && pg)
    launch_one<G, true, true>(q, kc, vc, kn, vn, out, counters, part_ml, part_o, n_head_kv, n_kv,
                              p, scale_log2, *pro, *pg, s);
  else if (pro)
    launch_one<G, true, false>(q, kc, vc, kn, vn, out, counters, part_ml, part_o, n_head_kv,
                               n_kv, p, scale_log2, *pro, flat, s);
  else if (pg)
    launch_one<G, false, true>(q, kc, vc, kn, vn, out, counters, part_ml, part_o, n_head_kv,
                               n_kv, p, scale_log2, none, *pg, s);
  else
    launch_one<G, false, false>(q, kc, vc, kn, vn, out, counters, part_ml, part_o, n_head_kv,
                                n_kv, p, scale_log2, none, flat, s);
}

// Zeroes the n arrival counters (kCounterStride ints apart) a launch starts
// from: a kernel, not a memset, so that a caller may capture it in a graph.
__global__ void clear_counters_kernel(int *counters, int n) {
  const int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
  if (i < n) counters[static_cast<size_t>(i) * kCounterStride] = 0;
}

// 0 when decode supports the shape, else the code it is rejected with.
int shape_status(int n_head, int n_head_kv, int head_dim, int64_t n_kv) {
  if (n_head <= 0 || n_head_kv <= 0 || n_head % n_head_kv != 0) return -EINVAL;
  if (n_kv <= 0) return -EINVAL;
  if (head_dim != D) return -ENOTSUP;
  if (!supported_group(n_head / n_head_kv)) return -ENOTSUP;
  if (n_kv > INT_MAX - 2 * TILE) return -EOVERFLOW;
  return 0;
}

// The workspace of the generic path (attn_generic.hpp) with qk-norm + RoPE
// folded in: the new token's rotated q and k rows.
// [rotated q rows][rotated k row][the split partials of the generic decode]
size_t generic_pro_bytes(int n_head, int n_head_kv, int head_dim) {
  return align256(sizeof(float) * static_cast<size_t>(n_head) * head_dim) +
         align256(sizeof(float) * static_cast<size_t>(n_head_kv) * head_dim);
}
size_t generic_ws_bytes(int n_head, int n_head_kv, int head_dim, int64_t n_kv) {
  return generic_pro_bytes(n_head, n_head_kv, head_dim) +
         ikv::generic_decode_ws_bytes(n_head, n_head_kv, head_dim, n_kv);
}

// A decode step on the generic attention path, for head sizes and query
// groupings the decode kernel does not take: the prologue (qk-RMSNorm + RoPE
// of the new token, into the workspace) and the append run as the separate
// kernels, then the attention of the one query over n_kv keys. No replay
// form (-ENOTSUP).
int decode_generic(const float *q, float *k_cache, float *v_cache, const float *k_new,
                   const float *v_new, float *out, int n_head, int n_head_kv, int head_dim,
                   int64_t n_kv, float scale, void *workspace, size_t workspace_bytes,
                   const Prologue *pro, const ikv_kv_pages *pages, const ikv::Pages *pg,
                   hipStream_t s) {
  if (pro && pro->dyn_max > 0) return -ENOTSUP;
  if (n_kv > INT_MAX / 2) return -EOVERFLOW;
  const size_t row_bytes = sizeof(float) * static_cast<size_t>(n_head_kv) * head_dim;
  if (k_new && pages && row_bytes % 16 != 0) return -ENOTSUP;
  if (pro) {
    if (!workspace || workspace_bytes < generic_pro_bytes(n_head, n_head_kv, head_dim))
      return -EINVAL;
    float *q_rot = static_cast<float *>(workspace);
    float *k_rot = reinterpret_cast<float *>(
        static_cast<char *>(workspace) +
        align256(sizeof(float) * static_cast<size_t>(n_head) * head_dim));
    int rc = ikv_qk_norm_rope_f32(q, pro->q_norm_w, q_rot, pro->pos, 1, n_head, head_dim,
                                  pro->eps, pro->sin_tab, pro->cos_tab, pro->n_ctx, pro->status,
                                  s);
    if (!rc)
      rc = ikv_qk_norm_rope_f32(k_new, pro->k_norm_w, k_rot, pro->pos, 1, n_head_kv, head_dim,
                                pro->eps, pro->sin_tab, pro->cos_tab, pro->n_ctx, pro->status, s);
    if (rc) return rc;
    q = q_rot;
    k_new = k_rot;
  }
  if (k_new) {
    int rc;
    if (pages) {
      rc = ikv_append_paged_f32(k_cache, k_new, pages, n_kv - 1, 1, row_bytes, s);
      if (!rc) rc = ikv_append_paged_f32(v_cache, v_new, pages, n_kv - 1, 1, row_bytes, s);
    } else {
      const size_t at = static_cast<size_t>(n_kv - 1) * (row_bytes / sizeof(float));
      rc = ikv_append_f32(k_cache + at, k_new, 1, row_bytes, s);
      if (!rc) rc = ikv_append_f32(v_cache + at, v_new, 1, row_bytes, s);
    }
    if (rc) return rc;
  }
  // the split form's partials after the prologue's rows (a smaller or no
  // workspace runs the one-workgroup-per-head form)
  const size_t pro_bytes = generic_pro_bytes(n_head, n_head_kv, head_dim);
  void *split_ws = nullptr;
  size_t split_bytes = 0;
  if (workspace && workspace_bytes > pro_bytes) {
    split_ws = static_cast<char *>(workspace) + pro_bytes;
    split_bytes = workspace_bytes - pro_bytes;
  }
  return ikv::attn_generic_decode(q, k_cache, v_cache, pg, out, n_head, n_head_kv, head_dim, n_kv,
                                  scale, split_ws, split_bytes, s);
}

int decode_common(const float *q, float *k_cache, float *v_cache, const float *k_new,
                  const float *v_new, float *out, int n_head, int n_head_kv, int head_dim,
                  int64_t n_kv, float scale, void *workspace, size_t workspace_bytes,
                  const Prologue *pro, const ikv_kv_pages *pages, void *stream,
                  bool clear_counters = false) {
  if (!q || !k_cache || !v_cache || !out) return -EINVAL;
  ikv::Pages pg;
  if (pages) {
    if (const int rc = ikv::pages_arg(pages, pg)) return rc;
  }
  if ((k_new == nullptr) != (v_new == nullptr)) return -EINVAL;
  if (const int rc = shape_status(n_head, n_head_kv, head_dim, n_kv)) {
    if (rc == -ENOTSUP && ikv::generic_attn_shape(n_head, n_head_kv, head_dim))
      return decode_generic(q, k_cache, v_cache, k_new, v_new, out, n_head, n_head_kv, head_dim,
                            n_kv, scale, workspace, workspace_bytes, pro, pages,
                            pages ? &pg : nullptr, static_cast<hipStream_t>(stream));
    return rc;
  }
  const int G = n_head / n_head_kv;
  if (!ikv::aligned16(q) || !ikv::aligned16(k_cache) || !ikv::aligned16(v_cache) ||
      !ikv::aligned16(out) || (k_new && (!ikv::aligned16(k_new) || !ikv::aligned16(v_new))))
    return -EINVAL;
  const Plan p = plan_for(n_head, n_head_kv, n_kv);
  const WsLayout L = ws_layout(n_head, n_head_kv, p.n_splits);
  int *counters = nullptr;
  float *part_ml = nullptr, *part_o = nullptr;
  if (p.n_splits > 1) {
    if (!workspace || workspace_bytes < L.total || !ikv::aligned16(workspace)) return -EINVAL;
    char *base = static_cast<char *>(workspace);
    counters = reinterpret_cast<int *>(base + L.counters);
    part_ml = reinterpret_cast<float *>(base + L.part_ml);
    part_o = reinterpret_cast<float *>(base + L.part_o);
  }
  if (!(scale > 0.0f)) scale = 1.0f / sqrtf(static_cast<float>(head_dim));
  const float sl2 = scale * ikv::kLog2e;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nk = static_cast<int>(n_kv);
  if (clear_counters && p.n_splits > 1) {
    clear_counters_kernel<<<(n_head_kv + 255) / 256, 256, 0, s>>>(counters, n_head_kv);
    if (const int rc = ikv::launch_status()) return rc;
  }
  switch (G) {
    case 1: launch<1>(q, k_cache, v_cache, k_new, v_new, out, counters, part_ml, part_o, n_head_kv, nk, p, sl2, pro, pages ? &pg : nullptr, s); break;
    case 2: launch<2>(q, k_cache, v_cache, k_new, v_new, out, counters, part_ml, part_o, n_head_kv, nk, p, sl2, pro, pages ? &pg : nullptr, s); break;
    case 4: launch<4>(q, k_cache, v_cache, k_new, v_new, out, counters, part_ml, part_o, n_head_kv, nk, p, sl2, pro, pages ? &pg : nullptr, s); break;
    default: launch<8>(q, k_cache, v_cache, k_new, v_new, out, counters, part_ml, part_o, n_head_kv, nk, p, sl2, pro, pages ? &pg : nullptr, s); break;
  }
  return ikv::launch_status();
}

}  // namespace

extern "C" size_t ikv_attn_decode_workspace_bytes(int n_head, int n_head_kv, int head_dim,
                                                  int64_t n_kv) {
  if (const int rc = shape_status(n_head, n_head_kv, head_dim, n_kv))
    return rc == -ENOTSUP && ikv::generic_attn_shape(n_head, n_head_kv, head_dim)
               ? generic_ws_bytes(n_head, n_head_kv, head_dim, n_kv)
               : 0;
  const Plan p = plan_for(n_head, n_head_kv, n_kv);
  return ws_layout(n_head, n_head_kv, p.n_splits).total;
}

extern "C" int ikv_attn_decode_f32(const float *q, float *k_cache, float *v_cache,
                                   const float *k_new, const float *v_new, float *out, int n_head,
                                   int n_head_kv, int head_dim, int64_t n_kv, float scale,
                                   void *workspace, size_t workspace_bytes, void *stream) {
  return decode_common(q, k_cache, v_cache, k_new, v_new, out, n_head, n_head_kv, head_dim, n_kv,
                       scale, workspace, workspace_bytes, nullptr, nullptr, stream);
}

extern "C" int ikv_attn_decode_paged_f32(const float *q, float *k_pool, float *v_pool,
                                         const ikv_kv_pages *pages, const float *k_new,
                                         const float *v_new, float *out, int n_head,
                                         int n_head_kv, int head_dim, int64_t n_kv, float scale,
                                         void *workspace, size_t workspace_bytes, void *stream) {
  if (!pages) return -EINVAL;
  return decode_common(q, k_pool, v_pool, k_new, v_new, out, n_head, n_head_kv, head_dim, n_kv,
                       scale, workspace, workspace_bytes, nullptr, pages, stream);
}

namespace {

int decode_rope_common(const float *q_raw, const float *k_raw, const float *v_new, float *k_cache,
                       float *v_cache, const ikv_kv_pages *pages, float *out, int n_head,
                       int n_head_kv, int head_dim, int64_t n_kv, float scale,
                       const float *q_norm_w, const float *k_norm_w, float eps,
                       const int32_t *pos, const float *sin_tab, const float *cos_tab,
                       int64_t n_ctx, int *status, void *workspace, size_t workspace_bytes,
                       void *stream, bool replay = false) {
  if (!k_raw || !v_new || !q_norm_w || !k_norm_w || !pos || !sin_tab || !cos_tab || n_ctx <= 0)
    return -EINVAL;
  Prologue pro;
  pro.q_norm_w = q_norm_w;
  pro.k_norm_w = k_norm_w;
  pro.eps = eps;
  pro.pos = pos;
  pro.sin_tab = sin_tab;
  pro.cos_tab = cos_tab;
  pro.n_ctx = n_ctx;
  pro.status = status;
  if (replay) {
    if (n_kv <= 0 || n_kv > INT_MAX - 2 * TILE) return n_kv <= 0 ? -EINVAL : -EOVERFLOW;
    pro.dyn_max = static_cast<int>(n_kv);
  }
  return decode_common(q_raw, k_cache, v_cache, k_raw, v_new, out, n_head, n_head_kv, head_dim,
                       n_kv, scale, workspace, workspace_bytes, &pro, pages, stream);
}

}  // namespace

extern "C" int ikv_attn_decode_rope_f32(const float *q_raw, const float *k_raw, const float *v_new,
                                        float *k_cache, float *v_cache, float *out, int n_head,
                                        int n_head_kv, int head_dim, int64_t n_kv, float scale,
                                        const float *q_norm_w, const float *k_norm_w, float eps,
                                        const int32_t *pos, const float *sin_tab,
                                        const float *cos_tab, int64_t n_ctx, int *status,
                                        void *workspace, size_t workspace_bytes, void *stream) {
  return decode_rope_common(q_raw, k_raw, v_new, k_cache, v_cache, nullptr, out, n_head,
                            n_head_kv, head_dim, n_kv, scale, q_norm_w, k_norm_w, eps, pos,
                            sin_tab, cos_tab, n_ctx, status, workspace, workspace_bytes, stream);
}

extern "C" int ikv_attn_decode_rope_paged_f32(
    const float *q_raw, const float *k_raw, const float *v_new, float *k_pool, float *v_pool,
    const ikv_kv_pages *pages, float *out, int n_head, int n_head_kv, int head_dim, int64_t n_kv,
    float scale, const float *q_norm_w, const float *k_norm_w, float eps, const int32_t *pos,
    const float *sin_tab, const float *cos_tab, int64_t n_ctx, int *status, void *workspace,
    size_t workspace_bytes, void *stream) {
  if (!pages) return -EINVAL;
  return decode_rope_common(q_raw, k_raw, v_new, k_pool, v_pool, pages, out, n_head, n_head_kv,
                            head_dim, n_kv, scale, q_norm_w, k_norm_w, eps, pos, sin_tab, cos_tab,
                            n_ctx, status, workspace, workspace_bytes, stream);
}

namespace {

int qkv_attn_common(
    const float *w_q, const float *w_k, const float *w_v, const float *x, const float *attn_norm_w,
    float attn_eps, float *q_out, float *k_out, float *v_out, int64_t n_embd, float *k_cache,
    float *v_cache, float *out, int n_head, int n_head_kv, int head_dim, int64_t n_kv, float scale,
    const float *q_norm_w, const float *k_norm_w, float eps, const int32_t *pos,
    const float *sin_tab, const float *cos_tab, int64_t n_ctx, int *status, void *workspace,
    size_t workspace_bytes, void *stream, bool replay) {
  if (const int rc = shape_status(n_head, n_head_kv, head_dim, n_kv)) return rc;
  if (n_embd <= 0 || n_embd > INT_MAX) return -EINVAL;
  // one split: the short contexts this launch is for; longer ones take the
  // projection and the split decode as two launches
  const Plan p = plan_for(n_head, n_head_kv, n_kv);
  if (p.n_splits != 1 || n_embd % ikv::gemv::kBatchCols != 0) return -ENOTSUP;
  if (!w_q || !w_k || !w_v || !x || !q_out || !k_out || !v_out || !k_cache || !v_cache || !out ||
      !q_norm_w || !k_norm_w || !pos || !sin_tab || !cos_tab || n_ctx <= 0 || !workspace)
    return -EINVAL;
  if (!ikv::aligned16(w_q) || !ikv::aligned16(w_k) || !ikv::aligned16(w_v) || !ikv::aligned16(x) ||
      !ikv::aligned16(k_cache) || !ikv::aligned16(v_cache) || !ikv::aligned16(out) ||
      !ikv::aligned16(q_out) || !ikv::aligned16(k_out) || !ikv::aligned16(v_out) ||
      (attn_norm_w && !ikv::aligned16(attn_norm_w)) || !ikv::aligned16(workspace))
    return -EINVAL;
  // the arrival counters, at the start of a decode workspace
  if (workspace_bytes < ws_layout(n_head, n_head_kv, 1).part_ml) return -EINVAL;
  Prologue pro;
  pro.q_norm_w = q_norm_w;
  pro.k_norm_w = k_norm_w;
  pro.eps = eps;
  pro.pos = pos;
  pro.sin_tab = sin_tab;
  pro.cos_tab = cos_tab;
  pro.n_ctx = n_ctx;
  pro.status = status;
  if (replay) pro.dyn_max = static_cast<int>(n_kv);
  if (!(scale > 0.0f)) scale = 1.0f / sqrtf(static_cast<float>(head_dim));
  const float sl2 = scale * ikv::kLog2e;
  const int G = n_head / n_head_kv;
  const int total_rows = (G + 2) * n_head_kv * D;
  const unsigned grid = static_cast<unsigned>(total_rows / kQkvRowsPerWg);
  hipStream_t s = static_cast<hipStream_t>(stream);
  int *counters = static_cast<int *>(workspace);
  const int K = static_cast<int>(n_embd);
  const int nk = static_cast<int>(n_kv);
#define IKV_QKV_ATTN(GG)                                                                          \
  qkv_attn_kernel<GG><<<grid, WG, 0, s>>>(w_q, w_k, w_v, x, attn_norm_w, attn_eps, q_out, k_out,   \
                                          v_out, K, k_cache, v_cache, out, counters, n_head_kv,   \
                                          nk, p.tokens_per_split, sl2, pro)
  switch (G) {
    case 1: IKV_QKV_ATTN(1); break;
    case 2: IKV_QKV_ATTN(2); break;
    case 4: IKV_QKV_ATTN(4); break;
    default: IKV_QKV_ATTN(8); break;
  }
#undef IKV_QKV_ATTN
  return ikv::launch_status();
}

// Whether launches planned for m keys give, at n keys, the results of the
// launch planned for n: one split for both, or splits of the same length
// (the launch for m then only adds empty splits, whose zero weights leave
// every sum unchanged).
bool replay_compatible(int n_head, int n_head_kv, int64_t n, int64_t m) {
  const Plan a = plan_for(n_head, n_head_kv, n), b = plan_for(n_head, n_head_kv, m);
  if (a.n_splits == 1 || b.n_splits == 1) return a.n_splits == 1 && b.n_splits == 1;
  return a.tokens_per_split == b.tokens_per_split;
}

}  // namespace

extern "C" int ikv_qkv_attn_decode_f32(
    const float *w_q, const float *w_k, const float *w_v, const float *x, const float *attn_norm_w,
    float attn_eps, float *q_out, float *k_out, float *v_out, int64_t n_embd, float *k_cache,
    float *v_cache, float *out, int n_head, int n_head_kv, int head_dim, int64_t n_kv, float scale,
    const float *q_norm_w, const float *k_norm_w, float eps, const int32_t *pos,
    const float *sin_tab, const float *cos_tab, int64_t n_ctx, int *status, void *workspace,
    size_t workspace_bytes, void *stream) {
  return qkv_attn_common(w_q, w_k, w_v, x, attn_norm_w, attn_eps, q_out, k_out, v_out, n_embd,
                         k_cache, v_cache, out, n_head, n_head_kv, head_dim, n_kv, scale, q_norm_w,
                         k_norm_w, eps, pos, sin_tab, cos_tab, n_ctx, status, workspace,
                         workspace_bytes, stream, false);
}

extern "C" int ikv_qkv_attn_decode_replay_f32(
    const float *w_q, const float *w_k, const float *w_v, const float *x, const float *attn_norm_w,
    float attn_eps, float *q_out, float *k_out, float *v_out, int64_t n_embd, float *k_cache,
    float *v_cache, float *out, int n_head, int n_head_kv, int head_dim, int64_t n_kv_max,
    float scale, const float *q_norm_w, const float *k_norm_w, float eps, const int32_t *pos,
    const float *sin_tab, const float *cos_tab, int64_t n_ctx, int *status, void *workspace,
    size_t workspace_bytes, void *stream) {
  return qkv_attn_common(w_q, w_k, w_v, x, attn_norm_w, attn_eps, q_out, k_out, v_out, n_embd,
                         k_cache, v_cache, out, n_head, n_head_kv, head_dim, n_kv_max, scale,
                         q_norm_w, k_norm_w, eps, pos, sin_tab, cos_tab, n_ctx, status, workspace,
                         workspace_bytes, stream, true);
}

extern "C" int ikv_attn_decode_rope_replay_f32(
    const float *q_raw, const float *k_raw, const float *v_new, float *k_cache, float *v_cache,
    float *out, int n_head, int n_head_kv, int head_dim, int64_t n_kv_max, float scale,
    const float *q_norm_w, const float *k_norm_w, float eps, const int32_t *pos,
    const float *sin_tab, const float *cos_tab, int64_t n_ctx, int *status, void *workspace,
    size_t workspace_bytes, void *stream) {
  return decode_rope_common(q_raw, k_raw, v_new, k_cache, v_cache, nullptr, out, n_head,
                            n_head_kv, head_dim, n_kv_max, scale, q_norm_w, k_norm_w, eps, pos,
                            sin_tab, cos_tab, n_ctx, status, workspace, workspace_bytes, stream,
                            true);
}

extern "C" int ikv_attn_decode_rope_paged_replay_f32(
    const float *q_raw, const float *k_raw, const float *v_new, float *k_pool, float *v_pool,
    const ikv_kv_pages *pages, float *out, int n_head, int n_head_kv, int head_dim,
    int64_t n_kv_max, float scale, const float *q_norm_w, const float *k_norm_w, float eps,
    const int32_t *pos, const float *sin_tab, const float *cos_tab, int64_t n_ctx, int *status,
    void *workspace, size_t workspace_bytes, void *stream) {
  if (!pages) return -EINVAL;
  return decode_rope_common(q_raw, k_raw, v_new, k_pool, v_pool, pages, out, n_head, n_head_kv,
                            head_dim, n_kv_max, scale, q_norm_w, k_norm_w, eps, pos, sin_tab,
                            cos_tab, n_ctx, status, workspace, workspace_bytes, stream, true);
}

extern "C" int64_t ikv_attn_decode_replay_limit(int n_head, int n_head_kv, int head_dim,
                                                int64_t n_kv, int64_t width) {
  if (width < 1 || shape_status(n_head, n_head_kv, head_dim, n_kv)) return 0;
  int64_t m = n_kv;
  while (m - n_kv + 1 < width && m + 1 <= INT_MAX - 2 * TILE &&
         replay_compatible(n_head, n_head_kv, n_kv, m + 1))
    ++m;
  return m;
}

// ---------------------------------------------------------------------------
// Decode without a caller workspace (for callers that cannot allocate: code
// under stream capture, serving loops that forbid allocation). The split
// partials and arrival counters live in a file-scope device array,
// kNoAllocScratchBytes per device: every call on a device shares that
// device's copy, so calls that overlap on one device race (order them on one
// stream). Nothing is allocated or freed: the array's address on each device
// is looked up on the first call there (hipGetSymbolAddress) and kept.
// ---------------------------------------------------------------------------
namespace {

constexpr size_t kNoAllocScratchBytes = IKV_DECODE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device (host code must not
// use the symbol itself as a pointer).
int scratch_ptr(void **out) {
  int dev = 0;
  if (const hipError_t e = hipGetDevice(&dev); e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return -ENODEV;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    if (const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); e != hipSuccess)
      return static_cast<int>(e);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace

extern "C" int ikv_attn_decode_noalloc_f32(const float *q, float *k_cache, float *v_cache,
                                           const float *k_new, const float *v_new, float *out,
                                           int n_head, int n_head_kv, int head_dim, int64_t n_kv,
                                           float scale, void *stream) {
  if (const int rc = shape_status(n_head, n_head_kv, head_dim, n_kv)) return rc;
  if (ikv_attn_decode_workspace_bytes(n_head, n_head_kv, head_dim, n_kv) > kNoAllocScratchBytes)
    return -ENOSPC;
  void *ws = nullptr;
  if (const int rc = scratch_ptr(&ws)) return rc;
  // The counters are cleared on every call: a call of another shape may have
  // left split partials where this shape's counters sit.
  return decode_common(q, k_cache, v_cache, k_new, v_new, out, n_head, n_head_kv, head_dim, n_kv,
                       scale, ws, kNoAllocScratchBytes, nullptr, nullptr, stream,
                       /*clear_counters=*/true);
}

#if IKV_DECODE_TIMELINE
// Copies the phase records of the last decode launch (kTimelineWgs x 16
// words, workgroup split * n_head_kv + g) to host memory, or zeroes them.
extern "C" int ikv_bench_timeline_read(unsigned long long *dst, size_t n_words) {
  if (!dst || n_words > static_cast<size_t>(kTimelineWgs) * kTimelineWords) return -EINVAL;
  return static_cast<int>(hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_timeline), n_words * 8));
}
extern "C" int ikv_bench_timeline_clear() {
  static unsigned long long zeros[kTimelineWgs * kTimelineWords];
  return static_cast<int>(hipMemcpyToSymbol(HIP_SYMBOL(g_timeline), zeros, sizeof(zeros)));
}
#endif
