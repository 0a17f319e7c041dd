// attn_generic.hip — causal GQA attention for the shapes the tuned kernels
// (attn_decode.hip, attn_prefill.hip: head_dim 128, query groups of 1, 2, 4
// or 8) do not take: any head_dim up to kGenericMaxDim and any ratio of query
// to KV heads, contiguous or paged caches. The semantics are
// CPUBackend::compute_flash_attn's (src/backends/cpu_backend.cpp:525-634):
// key j is visible to query t iff j <= n_past + t and j < n_kv; q head h
// reads KV head h / (n_head / n_head_kv).
//
// Prompts (and any n_q): a workgroup of 4 wavefronts owns 16 query rows of
// one KV head g (row r = token * G + query head in the group, so a block of
// rows covers every query head of its tokens and each K / V tile serves all
// of them). Key tiles of KT rows (64 keys for head_dim <= 128, fewer for
// wider heads so a tile stays about 34 KB) are staged in LDS (16-byte loads
// when rows are 16-byte aligned) with rows padded by 4 floats (16-byte reads
// from 16 rows hit distinct banks). A wave
// holds 4 rows: for the scores each lane takes a key (and, with KT < 64, a
// part of its dims, the parts summed by lane swaps) and forms its dot with
// the 4 query rows, broadcast from LDS; online softmax in base 2 per row
// over the wave; the weights go through LDS and every lane then adds the
// tile's V rows for its output dims (lane, lane + 64, ...), once per key for
// all 4 rows.
//
// One query token (a decode step): the split form below.
#include "attn_generic.hpp"
#include "ikv_common.hpp"

#include <algorithm>
#include <climits>

namespace {

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

constexpr int kTileRowsPerWave = 4;  // 8 measured slower (fewer workgroups, more registers)
constexpr int kTileRows = 4 * kTileRowsPerWave;  // query rows per workgroup

template <int DL>  // dims per lane: head_dim <= 64 * DL
__global__ __launch_bounds__(256) void generic_tile_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    float *__restrict__ out, int n_head, int n_head_kv, int dim, int n_q, int n_kv, int n_past,
    float scale_log2, bool paged, ikv::Pages pg, bool vec4) {
  constexpr int KT = DL <= 2 ? 64 : 128 / DL;  // keys per tile: 64, 64, 32, 16
  constexpr int LPK = 64 / KT;                 // lanes per key in the score phase
  constexpr int DA = 64 * DL;                  // dims held (zeros past head_dim)
  constexpr int DP = DA + 4;                   // padded LDS row
  constexpr int DPART = DA / LPK;              // dims of a lane's score part
  constexpr int RW = kTileRowsPerWave;
  __shared__ __attribute__((aligned(16))) float s_k[KT * DP];
  __shared__ __attribute__((aligned(16))) float s_v[KT * DP];
  __shared__ __attribute__((aligned(16))) float s_q[kTileRows * DP];
  __shared__ __attribute__((aligned(16))) float s_p[4][RW][KT];
  const int G = n_head / n_head_kv;
  const int g = static_cast<int>(blockIdx.x) % n_head_kv;
  const int blk = static_cast<int>(blockIdx.x) / n_head_kv;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n_rows = n_q * G;
  const int r0 = blk * kTileRows;
  const size_t tok_stride = static_cast<size_t>(n_head_kv) * dim;
  const size_t head_off = static_cast<size_t>(g) * dim;

  // the block's query rows, pre-scaled, zero past head_dim and past the rows
  for (int i = tid; i < kTileRows * DA; i += 256) {
    const int rr = i / DA, d = i - rr * DA;
    const int r = r0 + rr;
    float x = 0.f;
    if (r < n_rows && d < dim) {
      const int t = r / G, hh = r - t * G;
      x = q[(static_cast<size_t>(t) * n_head + g * G + hh) * dim + d] * scale_log2;
    }
    s_q[rr * DP + d] = x;
  }
  const int r_last = min(r0 + kTileRows, n_rows) - 1;
  const int kv_end = min(n_kv, n_past + r_last / G + 1);  // keys any row of the block sees

  int tok[RW];
  bool rok[RW];
  float m[RW], l[RW], o[RW][DL];
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    const int r = r0 + wave * RW + i;
    rok[i] = r < n_rows;
    tok[i] = rok[i] ? r / G : 0;
    m[i] = -INFINITY;
    l[i] = 0.f;
#pragma unroll
    for (int t = 0; t < DL; ++t) o[i][t] = 0.f;
  }
  const int jl = lane % KT;    // this lane's key in the score phase
  const int part = lane / KT;  // and its part of the dims
  for (int kb = 0; kb < kv_end; kb += KT) {
    __syncthreads();  // the previous tile's readers are done (and q is staged)
    if (vec4) {
      // 16-byte pieces: thread tid takes piece c = tid + 256 i of the tile
      constexpr int P4 = DA / 4;  // pieces per padded row
#pragma unroll
      for (int i = 0; i < KT * P4 / 256; ++i) {
        const int c = tid + 256 * i;
        const int jj = c / P4, d = 4 * (c - jj * P4);
        const int j = kb + jj;
        float4 kx = make_float4(0.f, 0.f, 0.f, 0.f), vx = kx;
        if (j < kv_end && d < dim) {
          const int64_t row = key_row(pg, paged, j);
          kx = *reinterpret_cast<const float4 *>(k + row * tok_stride + head_off + d);
          vx = *reinterpret_cast<const float4 *>(v + row * tok_stride + head_off + d);
        }
        *reinterpret_cast<float4 *>(s_k + jj * DP + d) = kx;
        *reinterpret_cast<float4 *>(s_v + jj * DP + d) = vx;
      }
    } else {
      for (int i = tid; i < KT * DA; i += 256) {
        const int jj = i / DA, d = i - jj * DA;
        const int j = kb + jj;
        float kx = 0.f, vx = 0.f;
        if (j < kv_end && d < dim) {
          const int64_t row = key_row(pg, paged, j);
          kx = k[row * tok_stride + head_off + d];
          vx = v[row * tok_stride + head_off + d];
        }
        s_k[jj * DP + d] = kx;
        s_v[jj * DP + d] = vx;
      }
    }
    __syncthreads();
    // scores of key kb + jl with the wave's 4 rows, over this lane's part
    float sc[RW];
#pragma unroll
    for (int i = 0; i < RW; ++i) sc[i] = 0.f;
    const float *kp = s_k + jl * DP + part * DPART;
    const float *qp = s_q + (wave * RW) * DP + part * DPART;
#pragma unroll 4
    for (int d4 = 0; d4 < DPART; d4 += 4) {
      const float4 kx = *reinterpret_cast<const float4 *>(kp + d4);
#pragma unroll
      for (int i = 0; i < RW; ++i) {
        const float4 qx = *reinterpret_cast<const float4 *>(qp + i * DP + d4);
        sc[i] = fmaf(qx.x, kx.x, sc[i]);
        sc[i] = fmaf(qx.y, kx.y, sc[i]);
        sc[i] = fmaf(qx.z, kx.z, sc[i]);
        sc[i] = fmaf(qx.w, kx.w, sc[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      if constexpr (LPK >= 2) {  // parts at lanes l, l ^ 32 (and l ^ 16)
        auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(sc[i]), __float_as_uint(sc[i]),
                                                  false, false);
        sc[i] = __uint_as_float(a[0]) + __uint_as_float(a[1]);
      }
      if constexpr (LPK >= 4) {
        auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(sc[i]), __float_as_uint(sc[i]),
                                                  false, false);
        sc[i] = __uint_as_float(b[0]) + __uint_as_float(b[1]);
      }
    }
    const int j = kb + jl;
    float alpha[RW];
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      const bool vis = rok[i] && j < kv_end && j <= n_past + tok[i];
      const float s = vis ? sc[i] : -INFINITY;
      const float m_new = fmaxf(m[i], ikv::wave_max(s));
      // a row that has seen no key yet keeps a zero state (reference 0)
      const float ref = (m_new == -INFINITY) ? 0.f : m_new;
      alpha[i] = ikv::fast_exp2(m[i] - ref);
      const float p = ikv::fast_exp2(s - ref);
      l[i] = fmaf(l[i], alpha[i], ikv::wave_sum(part == 0 ? p : 0.f));
      if (part == 0) s_p[wave][i][jl] = p;
      m[i] = m_new;
    }
    // the wave's weights are in LDS (its own writes, in order): add V
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int t = 0; t < DL; ++t) o[i][t] *= alpha[i];
    for (int j4 = 0; j4 < KT; j4 += 4) {  // 4 keys: the rows' weights as one 16-byte read
      float vd[4][DL];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int t = 0; t < DL; ++t) vd[u][t] = s_v[(j4 + u) * DP + lane + 64 * t];
#pragma unroll
      for (int i = 0; i < RW; ++i) {
        const float4 pj = *reinterpret_cast<const float4 *>(&s_p[wave][i][j4]);
#pragma unroll
        for (int t = 0; t < DL; ++t) {
          o[i][t] = fmaf(pj.x, vd[0][t], o[i][t]);
          o[i][t] = fmaf(pj.y, vd[1][t], o[i][t]);
          o[i][t] = fmaf(pj.z, vd[2][t], o[i][t]);
          o[i][t] = fmaf(pj.w, vd[3][t], o[i][t]);
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    if (!rok[i]) continue;
    const int r = r0 + wave * RW + i;
    const int hh = r - tok[i] * G;
    float *orow = out + (static_cast<size_t>(tok[i]) * n_head + g * G + hh) * dim;
    const float inv = 1.0f / l[i];
#pragma unroll
    for (int t = 0; t < DL; ++t) {
      const int d = lane + 64 * t;
      if (d < dim) orow[d] = o[i][t] * inv;
    }
  }
}

// ---------------------------------------------------------------------------
// One query token (a decode step), split over the context: workgroup
// (KV head g, split) serves all G query heads of g over keys [t_begin,
// t_end), so every K and V row is read once. Its 4 wavefronts take keys
// t_begin + wave, + 4, ...; a key's row is spread over the lanes (dims lane,
// lane + 64, ...: DL per lane, head_dim <= 64 DL), loaded 4 keys ahead, and
// each query head's score is a wave sum. Online softmax in base 2 per head;
// the waves meet in LDS and the split's (max, sum, unnormalised output) per
// head goes to the workspace; a second launch merges the splits in split
// order. Registers hold G x DL query and output values per lane: G * DL <=
// kSplitHeadDims.
constexpr int kSplitHeadDims = 32;
constexpr int kSplitWaves = 4;
// keys per wave in flight: 16 dims' worth of registers per lane for K and V
constexpr int split_ahead(int dl) { return dl >= 8 ? 2 : 16 / dl; }
constexpr int kSplitMinKeys = 64;
constexpr int kSplitTargetWgs = 256;  // one per MI355X compute unit

template <int DL>
__global__ __launch_bounds__(kSplitWaves * 64) void generic_split_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    float *__restrict__ part_ml, float *__restrict__ part_o, int n_head_kv, int G, int dim,
    int n_kv, int keys_per_split, int n_splits, float scale_log2, bool paged, ikv::Pages pg) {
  constexpr int GM = kSplitHeadDims / DL;  // most query heads per KV head
  constexpr int kSplitAhead = split_ahead(DL);
  __shared__ float s_m[kSplitWaves][GM], s_l[kSplitWaves][GM];
  __shared__ float s_o[kSplitWaves][GM][64 * DL];
  const int g = static_cast<int>(blockIdx.x) % n_head_kv;
  const int split = static_cast<int>(blockIdx.x) / n_head_kv;
  const int t_begin = split * keys_per_split;
  const int t_end = min(n_kv, t_begin + keys_per_split);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const size_t tok_stride = static_cast<size_t>(n_head_kv) * dim;
  const size_t head_off = static_cast<size_t>(g) * dim;

  float qv[GM][DL], o[GM][DL], m[GM], l[GM];
#pragma unroll
  for (int h = 0; h < GM; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int t = 0; t < DL; ++t) {
      const int d = lane + 64 * t;
      qv[h][t] = (h < G && d < dim)
                     ? q[(static_cast<size_t>(g) * G + h) * dim + d] * scale_log2
                     : 0.f;
      o[h][t] = 0.f;
    }
  }
  for (int j0 = t_begin + wave; j0 < t_end; j0 += kSplitWaves * kSplitAhead) {
    float kr[kSplitAhead][DL], vr[kSplitAhead][DL];
#pragma unroll
    for (int u = 0; u < kSplitAhead; ++u) {
      const int j = j0 + kSplitWaves * u;
      const bool ok = j < t_end;
      const int64_t row = key_row(pg, paged, ok ? j : t_begin);
      const float *kp = k + row * tok_stride + head_off;
      const float *vp = v + row * tok_stride + head_off;
#pragma unroll
      for (int t = 0; t < DL; ++t) {
        const int d = lane + 64 * t;
        kr[u][t] = (ok && d < dim) ? kp[d] : 0.f;
        vr[u][t] = (ok && d < dim) ? vp[d] : 0.f;
      }
    }
    // per query head: the chunk's scores (independent wave sums), then one
    // online-softmax step over them (the chunk's first key is always valid)
#pragma unroll
    for (int h = 0; h < GM; ++h) {
      if (h < G) {  // (guards, not breaks: the register arrays stay unrolled)
        float sc[kSplitAhead];
#pragma unroll
        for (int u = 0; u < kSplitAhead; ++u) {
          float part = 0.f;
#pragma unroll
          for (int t = 0; t < DL; ++t) part = fmaf(qv[h][t], kr[u][t], part);
          const float w = ikv::wave_sum(part);
          sc[u] = (j0 + kSplitWaves * u < t_end) ? w : -INFINITY;
        }
        float mx = m[h];
#pragma unroll
        for (int u = 0; u < kSplitAhead; ++u) mx = fmaxf(mx, sc[u]);
        const float alpha = ikv::fast_exp2(m[h] - mx);  // 0 on the first chunk
        float psum = 0.f;
#pragma unroll
        for (int t = 0; t < DL; ++t) o[h][t] *= alpha;
#pragma unroll
        for (int u = 0; u < kSplitAhead; ++u) {
          const float pu = ikv::fast_exp2(sc[u] - mx);  // 0 for a key past the split
          psum += pu;
#pragma unroll
          for (int t = 0; t < DL; ++t) o[h][t] = fmaf(pu, vr[u][t], o[h][t]);
        }
        l[h] = fmaf(l[h], alpha, psum);
        m[h] = mx;
      }
    }
  }
  // the waves meet in LDS (a wave with no key holds m = -inf, l = 0, o = 0)
#pragma unroll
  for (int h = 0; h < GM; ++h) {
    if (h < G) {
      if (lane == 0) {
        s_m[wave][h] = m[h];
        s_l[wave][h] = l[h];
      }
#pragma unroll
      for (int t = 0; t < DL; ++t) s_o[wave][h][lane + 64 * t] = o[h][t];
    }
  }
  __syncthreads();
  const size_t rec0 = static_cast<size_t>(g) * G * n_splits + split;  // record of head 0
  for (int idx = threadIdx.x; idx < G * dim; idx += kSplitWaves * 64) {
    const int h = idx / dim, d = idx - h * dim;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kSplitWaves; ++w) M = fmaxf(M, s_m[w][h]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kSplitWaves; ++w) {
      const float mw = s_m[w][h];
      const float e = (mw == -INFINITY) ? 0.f : ikv::fast_exp2(mw - M);
      L = fmaf(e, s_l[w][h], L);
      O = fmaf(e, s_o[w][h][d], O);
    }
    const size_t rec = rec0 + static_cast<size_t>(h) * n_splits;
    part_o[rec * dim + d] = O;
    if (d == 0) {
      part_ml[2 * rec] = M;
      part_ml[2 * rec + 1] = L;
    }
  }
}

// out[head][d] = sum_s e_s O_s[d] / sum_s e_s L_s, e_s = 2^(M_s - max_s M_s):
// one workgroup per query head. Wave 0 forms the weights (lanes over splits)
// and the sum; then every thread takes output dims and adds the splits'
// parts in split order.
constexpr int kMergeThreads = 256;
__global__ __launch_bounds__(kMergeThreads) void generic_merge_kernel(
    const float *__restrict__ part_ml, const float *__restrict__ part_o, float *__restrict__ out,
    int dim, int n_splits) {
  __shared__ float s_e[kSplitTargetWgs];
  __shared__ float s_L;
  const int head = blockIdx.x;
  const size_t rec0 = static_cast<size_t>(head) * n_splits;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    float M = -INFINITY;
    for (int sp = lane; sp < n_splits; sp += 64) M = fmaxf(M, part_ml[2 * (rec0 + sp)]);
    M = ikv::wave_max(M);
    float L = 0.f;
    for (int sp = lane; sp < n_splits; sp += 64) {
      const float ms = part_ml[2 * (rec0 + sp)];
      const float e = ms == -INFINITY ? 0.f : ikv::fast_exp2(ms - M);
      s_e[sp] = e;
      L = fmaf(e, part_ml[2 * (rec0 + sp) + 1], L);
    }
    L = ikv::wave_sum(L);
    if (lane == 0) s_L = L;
  }
  __syncthreads();
  const float inv = 1.0f / s_L;
  for (int d = threadIdx.x; d < dim; d += kMergeThreads) {
    float O = 0.f;
#pragma unroll 8
    for (int sp = 0; sp < n_splits; ++sp) O = fmaf(s_e[sp], part_o[(rec0 + sp) * dim + d], O);
    out[static_cast<size_t>(head) * dim + d] = O * inv;
  }
}

struct SplitPlan {
  int dl = 0;  // dims per lane; 0: the shape does not fit the split kernel
  int n_splits = 0, keys_per_split = 0;
};

SplitPlan split_plan(int n_head, int n_head_kv, int head_dim, int64_t n_kv) {
  SplitPlan p;
  const int G = n_head / n_head_kv;
  const int dl = head_dim <= 64 ? 1 : head_dim <= 128 ? 2 : head_dim <= 256 ? 4 : 8;
  if (G * dl > kSplitHeadDims || n_kv < 1 || n_kv > INT_MAX / 2) return p;
  const int64_t target = std::max<int64_t>(1, (kSplitTargetWgs + n_head_kv - 1) / n_head_kv);
  int64_t per = (n_kv + target - 1) / target;
  if (per < kSplitMinKeys) per = kSplitMinKeys;
  p.dl = dl;
  p.keys_per_split = static_cast<int>(per);
  p.n_splits = static_cast<int>((n_kv + per - 1) / per);
  return p;
}

size_t split_ws_bytes(int n_head, int head_dim, int n_splits) {
  const size_t ml = (sizeof(float) * 2 * static_cast<size_t>(n_head) * n_splits + 255) & ~size_t(255);
  return ml + sizeof(float) * static_cast<size_t>(n_head) * n_splits * head_dim;
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
  const int dl = head_dim <= 64 ? 1 : head_dim <= 128 ? 2 : head_dim <= 256 ? 4 : 8;
  const int64_t rows = n_q * (n_head / n_head_kv);
  const int64_t blocks = (rows + kTileRows - 1) / kTileRows;
  if (blocks * n_head_kv > INT_MAX) return -EOVERFLOW;
  const unsigned grid = static_cast<unsigned>(blocks * n_head_kv);
  const float sl2 = scale * kLog2e;
  const Pages pgv = pages ? *pages : Pages{};
  // K and V rows staged 16 bytes at a time when every row starts 16-byte
  // aligned
  const bool vec4 = head_dim % 4 == 0 && aligned16(k) && aligned16(v);
#define IKV_GENERIC_TILE(DD)                                                                  \
  generic_tile_kernel<DD><<<grid, 256, 0, s>>>(q, k, v, out, n_head, n_head_kv, head_dim,     \
                                               static_cast<int>(n_q), static_cast<int>(n_kv), \
                                               static_cast<int>(n_past), sl2, pages != nullptr, pgv, \
                                               vec4)
  switch (dl) {
    case 1: IKV_GENERIC_TILE(1); break;
    case 2: IKV_GENERIC_TILE(2); break;
    case 4: IKV_GENERIC_TILE(4); break;
    default: IKV_GENERIC_TILE(8); break;
  }
#undef IKV_GENERIC_TILE
  return launch_status();
}

}  // namespace ikv

namespace ikv {

size_t generic_decode_ws_bytes(int n_head, int n_head_kv, int head_dim, int64_t n_kv) {
  if (!generic_attn_shape(n_head, n_head_kv, head_dim)) return 0;
  const SplitPlan p = split_plan(n_head, n_head_kv, head_dim, n_kv);
  return p.dl ? split_ws_bytes(n_head, head_dim, p.n_splits) : 0;
}

int attn_generic_decode(const float *q, const float *k, const float *v, const Pages *pages,
                        float *out, int n_head, int n_head_kv, int head_dim, int64_t n_kv,
                        float scale, void *workspace, size_t workspace_bytes, hipStream_t s) {
  if (!generic_attn_shape(n_head, n_head_kv, head_dim)) return -ENOTSUP;
  if (n_kv <= 0) return -EINVAL;
  const SplitPlan p = split_plan(n_head, n_head_kv, head_dim, n_kv);
  if (!p.dl || !workspace || !aligned16(workspace) ||
      workspace_bytes < split_ws_bytes(n_head, head_dim, p.n_splits))
    return attn_generic(q, k, v, pages, out, n_head, n_head_kv, head_dim, 1, n_kv, n_kv - 1,
                        scale, s);
  if (!(scale > 0.0f)) scale = 1.0f / sqrtf(static_cast<float>(head_dim));
  float *part_ml = static_cast<float *>(workspace);
  float *part_o = reinterpret_cast<float *>(
      static_cast<char *>(workspace) +
      ((sizeof(float) * 2 * static_cast<size_t>(n_head) * p.n_splits + 255) & ~size_t(255)));
  const unsigned grid = static_cast<unsigned>(n_head_kv) * static_cast<unsigned>(p.n_splits);
  const int G = n_head / n_head_kv;
  const float sl2 = scale * kLog2e;
  const Pages pg = pages ? *pages : Pages{};
#define IKV_GENERIC_SPLIT(DD)                                                                \
  generic_split_kernel<DD><<<grid, kSplitWaves * 64, 0, s>>>(                                \
      q, k, v, part_ml, part_o, n_head_kv, G, head_dim, static_cast<int>(n_kv),              \
      p.keys_per_split, p.n_splits, sl2, pages != nullptr, pg)
  switch (p.dl) {
    case 1: IKV_GENERIC_SPLIT(1); break;
    case 2: IKV_GENERIC_SPLIT(2); break;
    case 4: IKV_GENERIC_SPLIT(4); break;
    default: IKV_GENERIC_SPLIT(8); break;
  }
#undef IKV_GENERIC_SPLIT
  generic_merge_kernel<<<static_cast<unsigned>(n_head), kMergeThreads, 0, s>>>(
      part_ml, part_o, out, head_dim, p.n_splits);
  return launch_status();
}

}  // namespace ikv
