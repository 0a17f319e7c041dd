// gemm.hip — the prefill projections: out[m][n] = sum_k x[m][k] w[n][k]
// (+ residual[m][n]) on F32 MFMA (v_mfma_f32_16x16x4_f32), used by
// ikv_mul_mat_f32 for every product of more than one token that its
// few-token kernel does not take.
//
// Replaces CPUBackend::compute_mul_mat (src/backends/cpu_backend.cpp:386-424)
// and CUDA_F32 mul_mat (src/kernels/cuda/kernel_f32.cu:142-205) for prompts;
// both operands are K-contiguous rows (GGUF weights [n][k], activations
// [m][k]), the "NT" product.
//
// Decomposition:
//   * A workgroup owns a BM x BN output tile (BM tokens x BN outputs) and is
//     WM x WN wavefronts, each TM x TN MFMA tiles of 16 x 16 (4
//     accumulators per lane per tile): 128 x 128 as 2 x 2 waves of 4 x 4
//     tiles for large products, 64 x 64 as 2 x 2 waves of 2 x 2 tiles
//     otherwise.
//   * The K loop stages BK = 64 columns of the tile's x rows and w rows in
//     LDS per step, in two buffers: while step s multiplies, the chunks of
//     step s+1 (loaded into registers during step s-2) are written to the
//     other buffer and those of step s+3 are loaded, a few per MFMA group.
//     (Global -> LDS DMA instead cost a tenth of the time even with every
//     load hitting L2.) A row's 64 columns are sixteen 16-byte chunks,
//     XOR-swizzled per row (chunk_slot) so that the 16 lanes of one LDS
//     read cycle hit distinct banks.
//   * One MFMA contracts 4 columns: lane l supplies row l % 16 and column
//     slot l / 16. The pairing of columns to slots is free as long as A and
//     B agree, so lane l reads chunk 4q + l / 16 of its row and its four
//     floats feed the four MFMAs of group q: per tile, MFMA e of group q
//     adds columns 16q + e, 16q + 4 + e, 16q + 8 + e, 16q + 12 + e. One
//     ds_read_b128 per operand tile per 4 MFMAs.
//   * Each group's MFMAs are interleaved with its memory instructions
//     (interleave_group): the wave is alone on its SIMD and issues in
//     order, so a burst of LDS / global instructions would idle the MFMA
//     pipe.
//   * Tiles are ordered so that each XCD (blockIdx % 8) walks a contiguous
//     run of a grouped order (8 tile rows walked column by column):
//     neighbouring tiles share x and w panels in that XCD's L2.
//   * Tokens past m are clamped to row m-1 for the loads and not stored.
//   * Split K: when even the smallest tiles leave CUs idle (few tokens, few
//     outputs, long k) the K loop of each tile is cut into n_split ranges of
//     whole steps, one workgroup each. The splits of a tile run on one XCD
//     (the same blockIdx % 8). Each stores its partial tile to a workspace
//     at the device's coherence point, waits for the stores and counts
//     itself on the tile's counter; the workgroup that counts last adds the
//     partials in split order (0, 1, ..., its own from registers), writes
//     the tile and sets the counter back to 0.
//   * Tile shape and split (gemm_plan) come from a cost model fitted to a
//     sweep of the Qwen3 projections on MI355X: rounds of tiles over the
//     256 CUs times a measured time per tile of each shape.
//   * Results are deterministic (fixed order per output for a given shape;
//     the split depends only on n_out, k and m).
#include "coherent.hpp"
#include "ikv_common.hpp"
#include "gemm.hpp"

#include <algorithm>
#include <climits>
#include <mutex>
#include <type_traits>

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int BK = 64;      // columns per step: 16 chunks of 16 bytes per row
constexpr int kChunks = BK / 4;
constexpr int kXcds = 8;
constexpr int64_t kMaxK = INT_MAX / (128 * 4);  // columns of a panel addressed in 32 bits
constexpr int kGroupM = 8;  // tile rows per group of the tile order

// Slot of 16-byte chunk c in staged row r (a row is 256 bytes, the width of
// MI355X's 64 banks). A ds_read_b128 of one chunk index by 32 lanes (32
// consecutive rows) is served 16 lanes at a time: every row starts on the
// same bank, so the slots of 16 consecutive rows must all differ, which the
// XOR key r & 15 gives. (With 128-byte rows and the key r & 7, rows 8 apart
// collided: 3.4e7 bank-conflict cycles per 4096^3 product.)
__device__ __forceinline__ int chunk_slot(int r, int c) { return c ^ (r & 15); }
constexpr int kCUs = 256;   // MI355X compute units

// f(std::integral_constant<int, i>) for i = 0 .. N-1, in order.
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

// Issue order of one MFMA group's region: its NR operand reads for the next
// group spread over the first half of its NM MFMAs, then NW LDS writes and
// NW global loads over the rest. A wave is alone on its SIMD here, and
// it issues in order: a burst of memory instructions stalls on full LDS /
// texture queues while the matrix core, which only ever holds the previous
// MFMA, runs dry.
template <int NM, int NR, int NW>
__device__ __forceinline__ void interleave_group() {
  constexpr int half = NR > 0 ? NM / 2 : 0;
  constexpr int per_read = NR > 0 ? half / NR : 0;
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);         // DS read
    __builtin_amdgcn_sched_group_barrier(0x008, per_read, 0);  // MFMA
  }
  // the NW LDS writes first, then the NW loads that refill the registers
  // they wrote from (a load right behind the write of the same registers
  // measured ~0.6% slower at the 8B shapes)
  constexpr int per_half = NW > 0 ? (NM - half) / (2 * NW) : 0;
#pragma unroll
  for (int j = 0; j < NW; ++j) {
    __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
    __builtin_amdgcn_sched_group_barrier(0x008, per_half, 0);
  }
#pragma unroll
  for (int j = 0; j < NW; ++j) {
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
    __builtin_amdgcn_sched_group_barrier(0x008, per_half, 0);
  }
}

// TM x TN MFMA tiles of 16 x 16 per wave, WM x WN waves per workgroup.
template <int TM, int TN, int WM, int WN>
__global__ __launch_bounds__(WM * WN * 64) void gemm_nt_kernel(const float *__restrict__ w,
                                                               const float *__restrict__ x,
                                                               float *out, const float *residual,
                                                               int n_out, int k, int m,
                                                               int tiles_n, int n_tiles,
                                                               int n_split, float *part,
                                                               int *counters) {
  constexpr int NT = WM * WN * 64;  // threads
  constexpr int BM = 16 * TM * WM, BN = 16 * TN * WN;
  constexpr int ROWS = BM + BN;     // staged rows per step: x rows, then w rows
  constexpr int CHUNKS = ROWS * kChunks;
  static_assert(CHUNKS % NT == 0, "whole chunks per thread");
  constexpr int CPT = CHUNKS / NT;  // 16-byte chunks per thread per step
  constexpr int NQ = kChunks / 4;   // MFMA groups per step: 4 chunks (16 columns) each
  __shared__ __attribute__((aligned(16))) float s_buf[2][ROWS * BK];
  __shared__ int s_last;

  // Tile order: XCD x (blockIdx % 8) takes positions [x * per, (x + 1) *
  // per) of a grouped order in which kGroupM tile rows are walked column by
  // column, so that the workgroups an XCD holds at once form a square block
  // of tiles sharing few x and w panels in its L2. Its j-th workgroup (j =
  // blockIdx / 8) takes split j / per of tile x * per + j % per.
  const int b = static_cast<int>(blockIdx.x);
  const int per = (n_tiles + kXcds - 1) / kXcds;
  const int j = b / kXcds;
  const int t = (b % kXcds) * per + j % per;
  const int sp = j / per;
  if (t >= n_tiles) return;
  const int tiles_m = n_tiles / tiles_n;
  const int grp = t / (kGroupM * tiles_n);
  const int first_m = grp * kGroupM;
  const int gsize = min(kGroupM, tiles_m - first_m);
  const int in_grp = t - grp * kGroupM * tiles_n;
  const int tm = first_m + in_grp % gsize, tn = in_grp / gsize;
  const int m0 = tm * BM, n0 = tn * BN;

  // This split's steps of BK columns: [lo, hi) of k / BK, in equal shares.
  const int all_steps = k / BK;
  const int s_lo = static_cast<int>(static_cast<int64_t>(sp) * all_steps / n_split);
  const int s_hi = static_cast<int>(static_cast<int64_t>(sp + 1) * all_steps / n_split);
  const int k_lo = s_lo * BK;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave - (wave / WN) * WN;

  // This thread's chunks: chunk q = tid + NT*i is column chunk c = q %
  // kChunks of staged row r = q / kChunks (16 consecutive threads read one
  // row's 256 contiguous bytes), stored at slot chunk_slot(r, c) of row r.
  // Rows r = tid / 16 + 16 i, so chunks i < CPT_X are x rows and the rest w
  // rows for every thread. Loads go through a buffer resource over the
  // tile's x panel and one over its w panel: a fixed 32-bit byte offset per
  // chunk and the step's column offset as the scalar offset, so the loop
  // issues no address arithmetic (with 64-bit pointers it added a VALU op
  // per load and ran ~1.7% slower).
  constexpr int CPT_X = BM * kChunks / NT;
  static_assert(BM % (NT / kChunks) == 0, "x and w chunks split at a whole i");
  const int x_rows = min(BM, m - m0);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(x + static_cast<size_t>(m0) * k), 0, x_rows * k * 4, ikv::kBufWord3);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(w + static_cast<size_t>(n0) * k), 0, BN * k * 4, ikv::kBufWord3);
  unsigned voff[CPT];
  int dst[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int q = tid + NT * i;
    const int r = q / kChunks;
    const int c = q % kChunks;
    const int row = r < BM ? min(r, x_rows - 1) : r - BM;  // within the panel
    voff[i] = static_cast<unsigned>((row * k + k_lo + 4 * c) * 4);
    dst[i] = r * BK + 4 * chunk_slot(r, c);
  }
  // chunk i of the step whose columns start at kb
  auto gload = [&](int i, int kb) -> floatx4 {
    return __builtin_amdgcn_raw_buffer_load_b128(i < CPT_X ? rx : rw, voff[i], kb * 4, 0);
  };
  // The chunks of the next two steps, global -> registers -> LDS: at the
  // start of step s, stage[(s + 1) & 1] holds step s + 1 and stage[s & 1]
  // step s + 2 (loads in flight), so a load has two steps to land.
  floatx4 stage[2][CPT];

  floatx4 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int c = 0; c < TN; ++c) acc[a][c] = floatx4{};

  // LDS read offsets (floats): lane l supplies row l % 16 of each 16-row
  // tile and reads chunk 4q + l / 16 of it, whose four floats feed the four
  // MFMAs of group q (one column each, the same for A and B). Tiles are 16
  // rows apart, a constant offset.
  const int r16 = lane & 15;
  const int h4 = lane >> 4;
  int aoff[NQ], boff[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int ra = wm * 16 * TM + r16;
    const int rb = BM + wn * 16 * TN + r16;
    aoff[q] = ra * BK + 4 * chunk_slot(ra, 4 * q + h4);
    boff[q] = rb * BK + 4 * chunk_slot(rb, 4 * q + h4);
  }

  // Operand chunks of one group: tile ti of A at aoff[q] + 16 * BK * ti.
  auto read_ops = [&](const float *buf, int q, floatx4 *a, floatx4 *b) {
#pragma unroll
    for (int ti = 0; ti < TM; ++ti)
      a[ti] = *reinterpret_cast<const floatx4 *>(buf + aoff[q] + 16 * BK * ti);
#pragma unroll
    for (int tj = 0; tj < TN; ++tj)
      b[tj] = *reinterpret_cast<const floatx4 *>(buf + boff[q] + 16 * BK * tj);
  };
  floatx4 av[TM], bv[TN];  // operands of the group being multiplied

  // One step, on the chunks in buffer s & 1 (P = s & 1): NQ groups of 4 x
  // TM*TN MFMAs, each group's operands read during the group before. With
  // NEXT, groups 0 .. NQ-2 write the staged chunks of step s + 1 to the
  // other buffer and load those of step s + 3 in their place; the barrier
  // then comes before the last group (every read of this buffer and every
  // write of the other is done), so that the last group's MFMAs cover the
  // reads of the next step's first operands instead of the step opening
  // on an LDS round trip.
  const int n_steps = s_hi - s_lo;
  auto step = [&](int s, auto next, auto par) {
    constexpr bool NEXT = decltype(next)::value;
    constexpr int P = decltype(par)::value;
    const float *cur = s_buf[P];
    float *nbuf = s_buf[P ^ 1];
    floatx4 *stg = stage[P ^ 1];
    const int kb3 = min(s + 3, n_steps - 1) * BK;
    static_for<NQ>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      constexpr bool more = q + 1 < NQ;
      constexpr bool reads = more || NEXT;
      constexpr bool stages = NEXT && more;
      constexpr int lo = stages ? q * CPT / (NQ - 1) : 0;
      constexpr int hi = stages ? (q + 1) * CPT / (NQ - 1) : 0;
      // one scheduling region: this group's MFMAs, the next group's operand
      // reads and this group's share of the staging, interleaved
      __builtin_amdgcn_sched_barrier(0);
      floatx4 an[TM], bn[TN];
      if constexpr (more)
        read_ops(cur, q + 1, an, bn);
      else if constexpr (NEXT)
        read_ops(nbuf, 0, an, bn);
#pragma unroll
      for (int i = lo; i < hi; ++i) {
        *reinterpret_cast<floatx4 *>(nbuf + dst[i]) = stg[i];
        stg[i] = gload(i, kb3);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int ti = 0; ti < TM; ++ti)
#pragma unroll
          for (int tj = 0; tj < TN; ++tj)
            acc[ti][tj] =
                __builtin_amdgcn_mfma_f32_16x16x4f32(av[ti][e], bv[tj][e], acc[ti][tj], 0, 0, 0);
      interleave_group<4 * TM * TN, reads ? TM + TN : 0, hi - lo>();
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (NEXT && q == NQ - 2) __syncthreads();
      if constexpr (reads) {
#pragma unroll
        for (int ti = 0; ti < TM; ++ti) av[ti] = an[ti];
#pragma unroll
        for (int tj = 0; tj < TN; ++tj) bv[tj] = bn[tj];
      }
    });
  };

  auto load = [&](floatx4 *stg, int st) {
    const int kb = min(st, n_steps - 1) * BK;
#pragma unroll
    for (int i = 0; i < CPT; ++i) stg[i] = gload(i, kb);
  };
  load(stage[0], 0);
#pragma unroll
  for (int i = 0; i < CPT; ++i) *reinterpret_cast<floatx4 *>(s_buf[0] + dst[i]) = stage[0][i];
  load(stage[1], 1);
  load(stage[0], 2);
  __syncthreads();
  read_ops(s_buf[0], 0, av, bv);
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  int s = 0;
  for (; s + 2 < n_steps; s += 2) {
    step(s, std::true_type{}, P0{});
    step(s + 1, std::true_type{}, P1{});
  }
  if (s + 1 < n_steps) {
    step(s, std::true_type{}, P0{});
    step(s + 1, std::false_type{}, P1{});
  } else {
    step(s, std::false_type{}, P0{});
  }

  if (n_split > 1) {
    // partial float4 (ti, tj) of thread tid of split q of tile t at float4
    // index ((t * n_split + q) * TM*TN + ti*TN + tj) * NT + tid
    const auto rs = ikv::partial_rsrc(
        part, static_cast<size_t>(n_tiles) * n_split * TM * TN * NT * sizeof(floatx4));
    auto at = [&](int q, int ti, int tj) {
      return static_cast<unsigned>(
          (((static_cast<size_t>(t) * n_split + q) * TM * TN + ti * TN + tj) * NT + tid) *
          sizeof(floatx4));
    };
#pragma unroll
    for (int ti = 0; ti < TM; ++ti)
#pragma unroll
      for (int tj = 0; tj < TN; ++tj) {
        const floatx4 a = acc[ti][tj];
        ikv::store4_agent(rs, at(sp, ti, tj), make_float4(a[0], a[1], a[2], a[3]));
      }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's stores performed
    __syncthreads();                // ... and every other wave's
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(counters + t, 1, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == n_split - 1;
    __syncthreads();
    if (!s_last) return;
#pragma unroll
    for (int ti = 0; ti < TM; ++ti)
#pragma unroll
      for (int tj = 0; tj < TN; ++tj) {
        floatx4 sum{};
        for (int q = 0; q < n_split; ++q) {
          floatx4 v = acc[ti][tj];
          if (q != sp) {
            const float4 l = ikv::load4_agent(rs, at(q, ti, tj));
            v = floatx4{l.x, l.y, l.z, l.w};
          }
          sum = q == 0 ? v : sum + v;
        }
        acc[ti][tj] = sum;
      }
    if (tid == 0) __hip_atomic_store(counters + t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // acc[ti][tj] register r of lane l: token wm*16*TM + 16*ti + 4*(l/16) + r,
  // output wn*16*TN + 16*tj + l%16 of the tile. The tile goes to LDS row by
  // row (stride BN + 4 floats: the 4 row groups of a store land 16 banks
  // apart) and leaves as 16-byte row pieces, 16 B per lane instead of 4.
  constexpr int OS = BN + 4;
  static_assert(BM * OS <= 2 * ROWS * BK, "the output tile fits the staging buffers");
  float *const s_out = &s_buf[0][0];
  __syncthreads();  // every wave's operand reads of the last step are done
#pragma unroll
  for (int ti = 0; ti < TM; ++ti)
#pragma unroll
    for (int tj = 0; tj < TN; ++tj)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        s_out[(wm * 16 * TM + 16 * ti + 4 * h4 + r) * OS + wn * 16 * TN + 16 * tj + r16] =
            acc[ti][tj][r];
  __syncthreads();
  constexpr int P4 = BN / 4;  // 16-byte pieces per tile row
  static_assert(BM * P4 % NT == 0, "whole rounds of pieces");
  const bool vec = ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(residual)) & 15) == 0;
#pragma unroll
  for (int e0 = 0; e0 < BM * P4; e0 += NT) {
    const int e = e0 + tid;
    const int row = e / P4, c = e - (e / P4) * P4;
    const int tok = m0 + row;
    if (tok < m) {
      const float *src = s_out + row * OS + 4 * c;
      const size_t o = static_cast<size_t>(tok) * n_out + n0 + 4 * c;
      if (vec) {
        float4 v = *reinterpret_cast<const float4 *>(src);
        if (residual) {
          const float4 rr = *reinterpret_cast<const float4 *>(residual + o);
          v = make_float4(v.x + rr.x, v.y + rr.y, v.z + rr.z, v.w + rr.w);
        }
        *reinterpret_cast<float4 *>(out + o) = v;
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          float v = src[u];
          if (residual) v += residual[o + u];
          out[o + u] = v;
        }
      }
    }
  }
}

template <int TM, int TN, int WM, int WN>
int launch(const float *w, const float *x, float *out, const float *residual, int n_out, int k,
           int m, int n_split, float *part, int *counters, hipStream_t s) {
  constexpr int BM = 16 * TM * WM, BN = 16 * TN * WN;
  static_assert(BM <= 128 && BN <= 128, "kMaxK covers the panels");
  const int tiles_m = (m + BM - 1) / BM;
  const int tiles_n = n_out / BN;
  const int64_t n_tiles = static_cast<int64_t>(tiles_m) * tiles_n;
  if (n_tiles > INT_MAX / 2) return -EOVERFLOW;
  const int64_t per = (n_tiles + kXcds - 1) / kXcds;
  if (per * n_split * kXcds > INT_MAX / 2) return -EOVERFLOW;
  gemm_nt_kernel<TM, TN, WM, WN><<<static_cast<unsigned>(per * n_split * kXcds), WM * WN * 64, 0,
                                   s>>>(w, x, out, residual, n_out, k, m, tiles_n,
                                        static_cast<int>(n_tiles), n_split, part, counters);
  return ikv::launch_status();
}

struct TileShape {
  int bm, bn;   // tokens x outputs
  float cost;   // time of one tile's K step relative to 32 x 32, one tile per CU
};
// Index = the tile code of gemm_nt_tile. The plan's cost model: a launch of
// T tiles, each split S ways, takes ceil(T * S / 256) rounds over the CUs of
// cost * (steps / S + kFillSteps) each, steps = k / 64 (kFillSteps: the
// pipeline's fill and the merge, in steps). Fitted to a sweep of the
// Qwen3-0.6B and -8B projections at 65-2047 tokens over every tile shape and
// 1-8 splits: each plan within 4.5% of the fastest measured.
constexpr TileShape kTiles[] = {{128, 128, 12.5f}, {64, 64, 3.9f}, {64, 32, 2.0f},
                                {32, 64, 2.1f},    {32, 32, 1.0f}};
constexpr int kNumTiles = 5;
constexpr double kFillSteps = 2.0;
constexpr int kMinSplitSteps = 4;   // steps of BK columns per split, at least
constexpr int kMaxSplit = 8;

// Split-K workspace: tile counters (all 0 between launches), then partials.
constexpr int kSplitCounters = 4096;
constexpr size_t kSplitCounterBytes = kSplitCounters * sizeof(int);
constexpr size_t kSplitPartBytes = size_t(8) << 20;

int64_t tile_count(int tile, int n, int m) {
  return int64_t((m + kTiles[tile].bm - 1) / kTiles[tile].bm) * (n / kTiles[tile].bn);
}

bool split_fits(int tile, int n, int m, int n_split, size_t part_bytes) {
  const int64_t tiles = tile_count(tile, n, m);
  return tiles <= kSplitCounters &&
         static_cast<size_t>(tiles) * n_split * kTiles[tile].bm * kTiles[tile].bn * sizeof(float) <=
             part_bytes;
}

__global__ void zero_ints_kernel(int *p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// The split-K workspace of (current device, stream s): allocated and its
// counters cleared (a kernel on s) on the first call for the pair, kept
// until the process ends. Calls on one stream are ordered, so they never
// share a workspace at the same time.
int split_workspace(hipStream_t s, float **part, int **counters) {
  struct Entry {
    int dev;
    hipStream_t stream;
    char *mem;
  };
  constexpr int kMaxEntries = 64;
  static std::mutex mu;
  static Entry table[kMaxEntries];
  static int n_entries = 0;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < n_entries; ++i)
    if (table[i].dev == dev && table[i].stream == s) {
      *counters = reinterpret_cast<int *>(table[i].mem);
      *part = reinterpret_cast<float *>(table[i].mem + kSplitCounterBytes);
      return 0;
    }
  if (n_entries == kMaxEntries) return -ENOMEM;
  void *mem = nullptr;
  e = hipMalloc(&mem, kSplitCounterBytes + kSplitPartBytes);
  if (e != hipSuccess) return static_cast<int>(e);
  zero_ints_kernel<<<kSplitCounters / 256, 256, 0, s>>>(static_cast<int *>(mem), kSplitCounters);
  e = hipGetLastError();
  if (e != hipSuccess) {
    (void)hipFree(mem);
    return static_cast<int>(e);
  }
  table[n_entries++] = {dev, s, static_cast<char *>(mem)};
  *counters = static_cast<int *>(mem);
  *part = reinterpret_cast<float *>(static_cast<char *>(mem) + kSplitCounterBytes);
  return 0;
}

}  // namespace

namespace ikv {

bool gemm_nt_supported(int64_t n_out, int64_t k, int64_t m) {
  // k bound: a 128-row panel of k floats is one buffer resource's range
  return m >= 1 && n_out % 64 == 0 && k % BK == 0 && k > 0 && n_out <= INT_MAX / 2 &&
         k <= kMaxK && m <= INT_MAX / 2;
}

GemmPlan gemm_plan(int64_t n_out, int64_t k, int64_t m, bool may_split) {
  const int n = static_cast<int>(n_out), mm = static_cast<int>(m);
  const int steps = static_cast<int>(k / BK);
  // the least estimated time; on a tie the larger tile, then fewer splits
  GemmPlan p{4, 1};
  double best = -1;
  for (int i = 0; i < kNumTiles; ++i) {
    if (n % kTiles[i].bn) continue;
    const int64_t tiles = tile_count(i, n, mm);
    for (int sk = 1; sk <= (may_split ? kMaxSplit : 1); ++sk) {
      if (sk > 1 && (steps < sk * kMinSplitSteps || !split_fits(i, n, mm, sk, kSplitPartBytes)))
        break;
      const double rounds = double((tiles * sk + kCUs - 1) / kCUs);
      const double est = rounds * kTiles[i].cost * (double(steps) / sk + kFillSteps);
      if (best < 0 || est < best) {
        best = est;
        p = GemmPlan{i, sk};
      }
    }
  }
  return p;
}

// The tile shapes (tokens x outputs): 0 128 x 128, 1 64 x 64, 2 64 x 32,
// 3 32 x 64, 4 32 x 32; each a 2 x 2 grid of wavefronts.
int gemm_nt_tile(int tile, int n_split, const float *w, const float *x, float *out,
                 const float *residual, int n, int kk, int mm, float *part, int *counters,
                 hipStream_t s) {
  if (n_split < 1 || n_split > kk / BK) return -EINVAL;
  switch (tile) {
    case 0:
      if (n % 128) return -ENOTSUP;
      return launch<4, 4, 2, 2>(w, x, out, residual, n, kk, mm, n_split, part, counters, s);
    case 1: return launch<2, 2, 2, 2>(w, x, out, residual, n, kk, mm, n_split, part, counters, s);
    case 2: return launch<2, 1, 2, 2>(w, x, out, residual, n, kk, mm, n_split, part, counters, s);
    case 3: return launch<1, 2, 2, 2>(w, x, out, residual, n, kk, mm, n_split, part, counters, s);
    case 4: return launch<1, 1, 2, 2>(w, x, out, residual, n, kk, mm, n_split, part, counters, s);
    default: return -EINVAL;
  }
}

int gemm_nt_f32(const float *w, const float *x, float *out, const float *residual, int64_t n_out,
                int64_t k, int64_t m, bool may_split, hipStream_t s) {
  if (!gemm_nt_supported(n_out, k, m)) return -ENOTSUP;
  if (!aligned16(w) || !aligned16(x)) return -EINVAL;
  const GemmPlan p = gemm_plan(n_out, k, m, may_split);
  float *part = nullptr;
  int *counters = nullptr;
  if (p.split > 1) {
    const int rc = split_workspace(s, &part, &counters);
    if (rc) return rc;
  }
  return gemm_nt_tile(p.tile, p.split, w, x, out, residual, static_cast<int>(n_out),
                      static_cast<int>(k), static_cast<int>(m), part, counters, s);
}

}  // namespace ikv

extern "C" int ikv_gemm_nt_f32(const float *w, const float *x, float *out, int64_t n_out, int64_t k,
                               int64_t m, const float *residual, void *stream) {
  if (!w || !x || !out) return -EINVAL;
  if (n_out < 0 || k < 0 || m < 0) return -EINVAL;
  if (n_out == 0 || m == 0) return 0;
  if (n_out > INT_MAX / 2 || k > INT_MAX / 2 || m > INT_MAX / 2) return -EOVERFLOW;
  if (!ikv::gemm_nt_supported(n_out, k, m)) return -ENOTSUP;
  return ikv::gemm_nt_f32(w, x, out, residual, n_out, k, m, false,
                          static_cast<hipStream_t>(stream));
}

#if IKV_GEMM_BENCH
// Bench-only (libikv_bench.so): one product on a chosen tile shape (see
// gemm_nt_tile) and split of K, the split-K workspace from the caller
// (ws_bytes >= 16 KiB of zeroed counters plus the partials).
extern "C" int ikv_bench_gemm_nt_tile_f32(const float *w, const float *x, float *out,
                                          int64_t n_out, int64_t k, int64_t m,
                                          const float *residual, int tile, int n_split, void *ws,
                                          size_t ws_bytes, void *stream) {
  if (!w || !x || !out || n_out <= 0 || k <= 0 || m <= 0) return -EINVAL;
  if (!ikv::gemm_nt_supported(n_out, k, m)) return -ENOTSUP;
  if (tile < 0 || tile >= kNumTiles || n_split < 1) return -EINVAL;
  float *part = nullptr;
  int *counters = nullptr;
  if (n_split > 1) {
    if (!ws || ws_bytes < kSplitCounterBytes ||
        !split_fits(tile, int(n_out), int(m), n_split, ws_bytes - kSplitCounterBytes))
      return -EINVAL;
    counters = static_cast<int *>(ws);
    part = reinterpret_cast<float *>(static_cast<char *>(ws) + kSplitCounterBytes);
  }
  return ikv::gemm_nt_tile(tile, n_split, w, x, out, residual, static_cast<int>(n_out),
                           static_cast<int>(k), static_cast<int>(m), part, counters,
                           static_cast<hipStream_t>(stream));
}

extern "C" int ikv_bench_gemm_plan(int64_t n_out, int64_t k, int64_t m, int *tile, int *n_split) {
  if (!tile || !n_split || n_out <= 0 || k <= 0 || m <= 0) return -EINVAL;
  if (!ikv::gemm_nt_supported(n_out, k, m)) return -ENOTSUP;
  const ikv::GemmPlan p = ikv::gemm_plan(n_out, k, m, true);
  *tile = p.tile;
  *n_split = p.split;
  return 0;
}
#endif
