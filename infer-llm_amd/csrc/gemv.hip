// gemv.hip — the projections of a Qwen3 step: out[m][n] = sum_k x[m][k] w[n][k].
//
// Replaces CPUBackend::compute_mul_mat (src/backends/cpu_backend.cpp:386-424)
// and CUDA_F32 mul_mat (src/kernels/cuda/kernel_f32.cu:142-205), which gave
// every output element its own thread and re-read x per element.
//
// Decode (m == 1) is a matrix-vector product that streams the weight from
// HBM once (F32 weights: 4 bytes per multiply-add, far below the FP32
// ridge), so the kernel is built for bandwidth: each wavefront owns RPW
// weight rows; a lane loads 16-byte pieces k = 4*lane + 256*j of every row
// (1 KiB per wave per load, coalesced) with non-temporal loads, the next
// 1024-column batch of every row in flight while the current one is
// multiplied; x comes through L1/L2 (it is shared by every wave); the row
// sums finish with DPP/swizzle half-wave reductions. Fused variants: a
// residual add (o_proj, ffn_down), three projections of one input in one
// launch (q, k, v), and the SwiGLU pair gate/up (each wave owns matching
// gate and up rows and writes up * silu(gate)). The q/k/v and SwiGLU forms
// can also fold in the RMSNorm of their input (attn_norm, ffn_norm): every
// wave computes the row's scale with the lane-strided double sum of
// ikv::rms_scale_strided (the order ikv_rms_norm_f32 uses for such rows)
// while its first weight batch is in flight, and multiplies x by scale and
// the norm weight as it reads it — the same float operations as the
// standalone norm, so the products see the same inputs bit for bit.
//
// Prefill (m > 1) is a dense F32 GEMM: up to 64 tokens the few-token MFMA
// kernel below, otherwise the tiled MFMA GEMM of gemm.hip; shapes neither
// takes (n_out or k not a multiple of 64, unaligned rows) run the per-output
// wavefront kernel over every token (slow, exact order per output).
#include <climits>

#include "coherent.hpp"
#include "gemm.hpp"
#include "gemv_dev.hpp"
#include "ikv_common.hpp"
#include "../../include/ikv_model.h"

namespace {

#ifndef IKV_GEMV_WAVES
#define IKV_GEMV_WAVES 4
#endif
#ifndef IKV_GEMV_RPW_SMALL
#define IKV_GEMV_RPW_SMALL 1  // rows per wave below 8192 output rows
#endif
#ifndef IKV_GEMV3_RPW
#define IKV_GEMV3_RPW 2  // rows per wave of the q/k/v launch (measured: 5.3 us vs 5.8 at 1 for 0.6B)
#endif
constexpr int kWaves = IKV_GEMV_WAVES;
constexpr int kThreads = kWaves * 64;
using namespace ikv::gemv;

// out[n] = w[n] . x (+ residual[n]); RPW rows per wave, n_out % RPW == 0.
template <int RPW>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const float *__restrict__ w,
                                                        const float *__restrict__ x, float *out,
                                                        const float *residual, int n_out, int K) {
  const int wave = blockIdx.x * kWaves + (threadIdx.x >> 6);
  const int row0 = wave * RPW;
  if (row0 >= n_out) return;
  const float *rows[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) rows[r] = w + static_cast<size_t>(row0 + r) * K;
  float s[RPW];
  wave_dots<RPW>(rows, x, K, s);
  const int lane = threadIdx.x & 63;
  if (lane < RPW) {
    float v = s[0];
#pragma unroll
    for (int r = 1; r < RPW; ++r)
      if (lane == r) v = s[r];
    if (residual) v += residual[row0 + lane];
    out[row0 + lane] = v;
  }
}

// Three weight matrices sharing x; wave rows fall in exactly one of them
// (each n_i % RPW == 0).
template <int RPW>
__global__ __launch_bounds__(kThreads) void gemv3_kernel(const float *__restrict__ w0,
                                                         const float *__restrict__ w1,
                                                         const float *__restrict__ w2,
                                                         const float *__restrict__ x, float *out0,
                                                         float *out1, float *out2, int n0, int n1,
                                                         int n2, int K, const float *nw, float eps) {
  const int wave = blockIdx.x * kWaves + (threadIdx.x >> 6);
  int row0 = wave * RPW;
  const float *w;
  float *out;
  if (row0 < n0) {
    w = w0;
    out = out0;
  } else if (row0 < n0 + n1) {
    row0 -= n0;
    w = w1;
    out = out1;
  } else if (row0 < n0 + n1 + n2) {
    row0 -= n0 + n1;
    w = w2;
    out = out2;
  } else {
    return;
  }
  const float *rows[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) rows[r] = w + static_cast<size_t>(row0 + r) * K;
  float s[RPW];
  wave_dots<RPW>(rows, x, K, s, nw, eps);
  const int lane = threadIdx.x & 63;
  if (lane < RPW) {
    float v = s[0];
#pragma unroll
    for (int r = 1; r < RPW; ++r)
      if (lane == r) v = s[r];
    out[row0 + lane] = v;
  }
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// ---------------------------------------------------------------------------
// The SwiGLU product with its input staged in LDS once per workgroup: xs = x,
// or with norm weights nw its RMSNorm (x * scale) * nw, the scale from
// ikv::rms_scale_strided over the staged row (one wave) and the products
// elementwise by every thread. These are the float operations of the per-wave form
// above, so each output is bitwise the same. The per-wave form recomputes the
// scale and re-reads x and nw from L2 in every wave. At the Qwen3-8B shape
// (12288 x 4096 gate and up) that costs more than the weight stream leaves
// room for: 71 us per wave, 65 us staged, 62 us with no norm at all. Each
// wave first issues its first weight batch, so HBM latency overlaps the
// staging. It then walks rows wave, wave + n_waves, ..., so a workgroup
// stages its input once for several rows. (Staging the q/k/v product, one
// row group per wave at these sizes, measured no faster than its per-wave
// form.)
constexpr int kStageMaxK = 8192;  // LDS bytes = 4 K (+ 4 for the scale)
#ifndef IKV_GEMV_STAGED_WGS
#define IKV_GEMV_STAGED_WGS 768  // 3 resident 4-wave workgroups per CU at this kernel's registers
#endif
constexpr int kStagedMaxWgs = IKV_GEMV_STAGED_WGS;
// Only with the norm folded in, and only for large products: with no norm
// there is nothing to save (8B: 63 us staged, 61 us per wave), and with one
// or two rows per wave the staging's barriers are exposed (Qwen3-0.6B
// gate/up: 7.24 us staged, 7.08 us per wave).
constexpr int64_t kStagedMinFloats = int64_t(16) << 20;

__device__ __forceinline__ void stage_input(const float *x, const float *nw, float eps, int K,
                                            float4 *xs) {
  const int n4 = K / 4;
  for (int i = threadIdx.x; i < n4; i += kThreads) xs[i] = reinterpret_cast<const float4 *>(x)[i];
  __syncthreads();
  if (nw) {
    __shared__ float s_scale;
    if (threadIdx.x < 64) {
      const float sc = ikv::rms_scale_strided(xs, K, eps, threadIdx.x);
      if (threadIdx.x == 0) s_scale = sc;
    }
    __syncthreads();
    const float scale = s_scale;
    for (int i = threadIdx.x; i < n4; i += kThreads)
      xs[i] = normed(xs[i], scale, reinterpret_cast<const float4 *>(nw)[i]);
    __syncthreads();
  }
}

// wave_dots with x read from the staged LDS row and the first batch of every
// row already in cur.
template <int NR>
__device__ __forceinline__ void wave_dots_staged(const float *const (&rows)[NR], const float4 *xs,
                                                 int K, float4 (&cur)[NR][kBatch], float (&out)[NR]) {
  const int lane = threadIdx.x & 63;
  float4 nxt[NR][kBatch];
  float4 acc[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int k0 = 0; k0 < K; k0 += kBatchCols) {
    const bool more = k0 + kBatchCols < K;
    if (more) {
#pragma unroll
      for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int j = 0; j < kBatch; ++j)
          nxt[r][j] = nt_load4(rows[r] + k0 + kBatchCols + 4 * lane + 256 * j);
    }
    float4 xv[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) xv[j] = xs[(k0 >> 2) + lane + 64 * j];
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        acc[r].x = fmaf(cur[r][j].x, xv[j].x, acc[r].x);
        acc[r].y = fmaf(cur[r][j].y, xv[j].y, acc[r].y);
        acc[r].z = fmaf(cur[r][j].z, xv[j].z, acc[r].z);
        acc[r].w = fmaf(cur[r][j].w, xv[j].w, acc[r].w);
      }
    if (more) {
#pragma unroll
      for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int j = 0; j < kBatch; ++j) cur[r][j] = nxt[r][j];
    }
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) out[r] = wave_sum64((acc[r].x + acc[r].y) + (acc[r].z + acc[r].w));
}

template <int NR>
__device__ __forceinline__ void first_batch(const float *const (&rows)[NR], float4 (&cur)[NR][kBatch]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int j = 0; j < kBatch; ++j) cur[r][j] = nt_load4(rows[r] + 4 * lane + 256 * j);
}

__global__ __launch_bounds__(kThreads) void gemv_swiglu_staged_kernel(
    const float *__restrict__ wg, const float *__restrict__ wu, const float *__restrict__ x,
    float *__restrict__ out, int n_out, int K, const float *nw, float eps) {
  extern __shared__ float4 xs[];
  const int n_waves = gridDim.x * kWaves;
  const int first = blockIdx.x * kWaves + (threadIdx.x >> 6);
  int n = first;
  const float *rows[2];
  float4 cur[2][kBatch];
  if (n < n_out) {
    rows[0] = wg + static_cast<size_t>(n) * K;
    rows[1] = wu + static_cast<size_t>(n) * K;
    first_batch<2>(rows, cur);
  }
  stage_input(x, nw, eps, K, xs);
  for (; n < n_out; n += n_waves) {
    if (n != first) {
      rows[0] = wg + static_cast<size_t>(n) * K;
      rows[1] = wu + static_cast<size_t>(n) * K;
      first_batch<2>(rows, cur);
    }
    float sres[2];
    wave_dots_staged<2>(rows, xs, K, cur, sres);
    if ((threadIdx.x & 63) == 0) out[n] = sres[1] * silu(sres[0]);
  }
}

int staged_grid(int64_t waves) {
  const int64_t wgs = (waves + kWaves - 1) / kWaves;
  return static_cast<int>(wgs < kStagedMaxWgs ? wgs : kStagedMaxWgs);
}

// out[n] = (w_up[n] . x) * silu(w_gate[n] . x); one output per wave.
__global__ __launch_bounds__(kThreads) void gemv_swiglu_kernel(const float *__restrict__ wg,
                                                               const float *__restrict__ wu,
                                                               const float *__restrict__ x,
                                                               float *__restrict__ out, int n_out,
                                                               int K, const float *nw, float eps) {
  const int n = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (n >= n_out) return;
  const float *rows[2] = {wg + static_cast<size_t>(n) * K, wu + static_cast<size_t>(n) * K};
  float s[2];
  wave_dots<2>(rows, x, K, s, nw, eps);
  if ((threadIdx.x & 63) == 0) out[n] = s[1] * silu(s[0]);
}

// Any shape: one wave per output row, scalar loads (sizes the fast kernels
// do not take: K % 1024 != 0 or unaligned pointers).
__global__ __launch_bounds__(kThreads) void gemv_generic_kernel(const float *__restrict__ w,
                                                                const float *__restrict__ x,
                                                                float *out, const float *residual,
                                                                int n_out, int K, int mode,
                                                                const float *__restrict__ w_up) {
  const int n = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (n >= n_out) return;
  const int lane = threadIdx.x & 63;
  const float *row = w + static_cast<size_t>(n) * K;
  // token blockIdx.y of a multi-token product (mode 0)
  x += static_cast<size_t>(blockIdx.y) * K;
  out += static_cast<size_t>(blockIdx.y) * n_out;
  if (residual) residual += static_cast<size_t>(blockIdx.y) * n_out;
  float a = 0.f, b = 0.f;
  for (int k = lane; k < K; k += 64) {
    a = fmaf(row[k], x[k], a);
    if (mode == 2) b = fmaf(w_up[static_cast<size_t>(n) * K + k], x[k], b);
  }
  a = wave_sum64(a);
  b = wave_sum64(b);
  if (lane == 0) {
    float v = a;
    if (mode == 2) v = b * silu(a);
    if (residual) v += residual[n];
    out[n] = v;
  }
}

bool fast_ok(int64_t k, std::initializer_list<const void *> ptrs) {
  if (k % kBatchCols != 0) return false;
  for (const void *p : ptrs)
    if (p && !ikv::aligned16(p)) return false;
  return true;
}

int grid_for(int64_t waves) { return static_cast<int>((waves + kWaves - 1) / kWaves); }

// Few-token products (2 <= m <= kSkinnyMaxM, the prefill of a short prompt):
// out[t][n] = sum_k w[n][k] x[t][k] (+ residual[t][n]) on F32 MFMA
// (v_mfma_f32_16x16x4_f32). A workgroup owns a 16-row tile of w and a
// 16-token tile of x; its 8 wavefronts take 8 equal slices of k. A wavefront
// moves its slice in steps of 64 columns: each load instruction reads 4 rows
// x 256 contiguous bytes (w, then x), the step is written to the wavefront's
// own LDS tile with 16-byte slots XOR-swizzled by row, and read back in the
// MFMA operand layout (lane (kk, j) takes row j, columns 16u + 4kk..+3), the
// swizzle keeping both the writes and the reads free of bank conflicts. Two
// steps of loads are in flight in registers; a wavefront's LDS accesses run
// in order, so one LDS tile per wavefront suffices. The 8 partial tiles are
// summed through LDS in wave order, so results do not depend on timing.
// blockIdx = n_tile + n_tiles * m_tile: with n_tiles a multiple of 8, the
// token tiles of one w tile run on the same XCD and share its L2. A library
// GEMM of these shapes picks output tiles so large that a 3072-row
// projection of 32 tokens runs on 48 workgroups.
typedef float floatx4 __attribute__((ext_vector_type(4)));
constexpr int kSkinnyMaxM = 64;
constexpr int kSkinnyWaves = 8;
constexpr int kSkinnyCols = 64;  // k columns per step

// MT token tiles of 16 per workgroup: the 16 weight rows of a step are staged
// once and multiplied into MT accumulators (one weight read per 16 * MT
// tokens; MT = 2 fits 112 KB of LDS with 8 wavefronts).
template <int MT>
__global__ __launch_bounds__(kSkinnyWaves * 64) void skinny_kernel(const float *__restrict__ w,
                                                                   const float *__restrict__ x,
                                                                   float *out, const float *residual,
                                                                   int n_out, int k, int m, int n_tiles) {
  __shared__ __attribute__((aligned(16))) float s_tile[kSkinnyWaves][1 + MT][16][kSkinnyCols];
  __shared__ float s_red[MT][kSkinnyWaves][64][4];
  const int nt = blockIdx.x % n_tiles;
  const int mt = blockIdx.x / n_tiles;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int j = lane & 15;
  const int kk = lane >> 4;
  const int n0 = nt * 16, m0 = mt * 16 * MT;
  const int kw = k / kSkinnyWaves;  // a multiple of 2 * kSkinnyCols
  const int kb0 = wave * kw;
  const int n_steps = kw / kSkinnyCols;
  // staging: instruction i reads rows 4i + lane / 16, 16-byte column lane % 16,
  // through a buffer resource over the 16 w rows and one over the
  // workgroup's x rows (rows past m read zeros; their outputs are not
  // stored): a fixed byte offset per instruction and the step's column
  // offset as the scalar offset, so the loop issues no address arithmetic
  const int sc = lane & 15;
  const __amdgpu_buffer_rsrc_t rsw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(w + static_cast<size_t>(n0) * k), 0, 16 * k * 4, ikv::kBufWord3);
  const __amdgpu_buffer_rsrc_t rsx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(x + static_cast<size_t>(m0) * k), 0, min(16 * MT, m - m0) * k * 4,
      ikv::kBufWord3);
  unsigned voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * i + (lane >> 4);
    voff[i] = static_cast<unsigned>((r * k + kb0 + 4 * sc) * 4);
  }
  const unsigned tile_bytes = static_cast<unsigned>(16 * k * 4);  // one token tile of x
  float(*tw)[kSkinnyCols] = s_tile[wave][0];
  floatx4 rw0[4], rx0[MT][4], rw1[4], rx1[MT][4];  // two steps in flight
  floatx4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  auto load_step = [&](floatx4 (&rw)[4], floatx4 (&rx)[MT][4], int step) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      rw[i] = __builtin_amdgcn_raw_buffer_load_b128(rsw, voff[i], kSkinnyCols * step * 4, 0);
#pragma unroll
      for (int t = 0; t < MT; ++t)
        rx[t][i] = __builtin_amdgcn_raw_buffer_load_b128(rsx, voff[i] + t * tile_bytes,
                                                         kSkinnyCols * step * 4, 0);
    }
  };
  // store a register set as the current step, refill it with step `next`
  // (if any), then multiply the step out of LDS
  auto body = [&](floatx4 (&rw)[4], floatx4 (&rx)[MT][4], int next) __attribute__((always_inline)) {
    // each register set is refilled right after its LDS write, in the
    // order it was loaded
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * i + (lane >> 4);
      *reinterpret_cast<floatx4 *>(&tw[r][4 * (sc ^ r)]) = rw[i];
      if (next >= 0)
        rw[i] = __builtin_amdgcn_raw_buffer_load_b128(rsw, voff[i], kSkinnyCols * next * 4, 0);
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        *reinterpret_cast<floatx4 *>(&s_tile[wave][1 + t][r][4 * (sc ^ r)]) = rx[t][i];
        if (next >= 0)
          rx[t][i] = __builtin_amdgcn_raw_buffer_load_b128(rsx, voff[i] + t * tile_bytes,
                                                           kSkinnyCols * next * 4, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // the refill stays ahead of this step's reads and MFMAs
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int slot = (4 * u + kk) ^ j;
      const floatx4 a = *reinterpret_cast<const floatx4 *>(&tw[j][4 * slot]);
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const floatx4 c = *reinterpret_cast<const floatx4 *>(&s_tile[wave][1 + t][j][4 * slot]);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], c[0], acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], c[1], acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], c[2], acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], c[3], acc[t], 0, 0, 0);
      }
    }
  };
  load_step(rw0, rx0, 0);
  load_step(rw1, rx1, 1);
  for (int s = 0; s + 2 < n_steps; s += 2) {  // n_steps is even: every refill is a real step
    body(rw0, rx0, s + 2);
    body(rw1, rx1, s + 3);
  }
  body(rw0, rx0, -1);
  body(rw1, rx1, -1);
  // lane l, register r of acc[t]: w row n0 + 4 (l / 16) + r, token
  // m0 + 16 t + l % 16
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) s_red[t][wave][lane][r] = acc[t][r];
  __syncthreads();
  if (threadIdx.x < 256) {
    const int l = threadIdx.x >> 2;
    const int r = threadIdx.x & 3;
    const int n = n0 + 4 * (l >> 4) + r;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int tok = m0 + 16 * t + (l & 15);
      float v = s_red[t][0][l][r];
#pragma unroll
      for (int q = 1; q < kSkinnyWaves; ++q) v += s_red[t][q][l][r];
      if (tok < m) {
        const size_t o = static_cast<size_t>(tok) * n_out + n;
        if (residual) v += residual[o];
        out[o] = v;
      }
    }
  }
}

bool skinny_ok(int64_t n_out, int64_t k, int64_t m, std::initializer_list<const void *> ptrs) {
  if (m < 2 || m > kSkinnyMaxM || n_out % 16 != 0 || k % (2 * kSkinnyCols * kSkinnyWaves) != 0)
    return false;
  if (k > INT_MAX / (32 * 4)) return false;  // 32 rows of k floats: one buffer range

  for (const void *p : ptrs)
    if (p && !ikv::aligned16(p)) return false;
  return true;
}

}  // namespace

extern "C" int ikv_mul_mat_f32(const float *w, const float *x, float *out, int64_t n_out,
                               int64_t k, int64_t m, const float *residual, void *stream) {
  if (!w || !x || !out) return -EINVAL;
  if (n_out < 0 || k < 0 || m < 0) return -EINVAL;
  if (n_out == 0 || m == 0) return 0;
  if (k == 0) return -EINVAL;
  if (n_out > INT_MAX / 2 || k > INT_MAX / 2 || m > INT_MAX / 2) return -EOVERFLOW;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (m == 1) {
    if (fast_ok(k, {w, x})) {
      // two rows per wave for many rows or a large product (x is then read
      // once per two rows); one for the small products of Qwen3-0.6B
      const bool big = n_out >= 8192 || n_out * k >= kStagedMinFloats;
      const int rpw = (big && n_out % 2 == 0) ? 2
                      : (n_out % IKV_GEMV_RPW_SMALL == 0 ? IKV_GEMV_RPW_SMALL : 1);
      if (rpw == 2)
        gemv_kernel<2><<<grid_for(n_out / 2), kThreads, 0, s>>>(w, x, out, residual, int(n_out), int(k));
      else if (rpw == 4)
        gemv_kernel<4><<<grid_for(n_out / 4), kThreads, 0, s>>>(w, x, out, residual, int(n_out), int(k));
      else
        gemv_kernel<1><<<grid_for(n_out), kThreads, 0, s>>>(w, x, out, residual, int(n_out), int(k));
    } else {
      gemv_generic_kernel<<<grid_for(n_out), kThreads, 0, s>>>(w, x, out, residual, int(n_out),
                                                                int(k), 0, nullptr);
    }
    return ikv::launch_status();
  }
  if (skinny_ok(n_out, k, m, {w, x})) {
    const int n_tiles = static_cast<int>(n_out / 16);
    // 17-64 tokens over 256+ weight tiles (one workgroup per CU even with
    // two token tiles each): two token tiles per workgroup, each weight step
    // staged once per 32 tokens (Qwen3-8B q and down at 32 tokens 21.2 ->
    // 16.6 and 57.5 -> 37.1 us). Fewer weight tiles keep one token tile per
    // workgroup, for the workgroup count (the 0.6B o projection at 32
    // tokens: 5.7 us with one, 8.5 with two).
    if (m > 16 && n_tiles >= 256) {
      const int m_pairs = static_cast<int>((m + 31) / 32);
      skinny_kernel<2><<<n_tiles * m_pairs, kSkinnyWaves * 64, 0, s>>>(
          w, x, out, residual, int(n_out), int(k), int(m), n_tiles);
    } else {
      const int m_tiles = static_cast<int>((m + 15) / 16);
      skinny_kernel<1><<<n_tiles * m_tiles, kSkinnyWaves * 64, 0, s>>>(
          w, x, out, residual, int(n_out), int(k), int(m), n_tiles);
    }
    return ikv::launch_status();
  }
  if (ikv::gemm_nt_supported(n_out, k, m) && ikv::aligned16(w) && ikv::aligned16(x))
    return ikv::gemm_nt_f32(w, x, out, residual, n_out, k, m, true, s);
  // any other shape: one wavefront per output, blockIdx.y the token
  if (m > 65535) return -ENOTSUP;
  gemv_generic_kernel<<<dim3(grid_for(n_out), static_cast<unsigned>(m)), kThreads, 0, s>>>(
      w, x, out, residual, int(n_out), int(k), 0, nullptr);
  return ikv::launch_status();
}

extern "C" int ikv_gemv3_f32(const float *w0, const float *w1, const float *w2, const float *x,
                             float *out0, float *out1, float *out2, int64_t n0, int64_t n1,
                             int64_t n2, int64_t k, const float *norm_w, float eps, void *stream) {
  if (!w0 || !w1 || !w2 || !x || !out0 || !out1 || !out2) return -EINVAL;
  if (n0 < 0 || n1 < 0 || n2 < 0 || k <= 0) return -EINVAL;
  if (n0 + n1 + n2 > INT_MAX / 2 || k > INT_MAX / 2) return -EOVERFLOW;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (norm_w && !fast_ok(k, {w0, w1, w2, x, norm_w})) return -ENOTSUP;
  if (!fast_ok(k, {w0, w1, w2, x})) {
    int rc = ikv_mul_mat_f32(w0, x, out0, n0, k, 1, nullptr, stream);
    if (rc == 0) rc = ikv_mul_mat_f32(w1, x, out1, n1, k, 1, nullptr, stream);
    if (rc == 0) rc = ikv_mul_mat_f32(w2, x, out2, n2, k, 1, nullptr, stream);
    return rc;
  }
  const int64_t total = n0 + n1 + n2;
  if (total == 0) return 0;
  constexpr int R3 = IKV_GEMV3_RPW;
  if (R3 > 1 && n0 % R3 == 0 && n1 % R3 == 0 && n2 % R3 == 0)
    gemv3_kernel<R3><<<grid_for(total / R3), kThreads, 0, s>>>(w0, w1, w2, x, out0, out1, out2,
                                                               int(n0), int(n1), int(n2), int(k),
                                                               norm_w, eps);
  else
    gemv3_kernel<1><<<grid_for(total), kThreads, 0, s>>>(w0, w1, w2, x, out0, out1, out2, int(n0),
                                                        int(n1), int(n2), int(k), norm_w, eps);
  return ikv::launch_status();
}

extern "C" int ikv_gemv_swiglu_f32(const float *w_gate, const float *w_up, const float *x,
                                   float *out, int64_t n_out, int64_t k, const float *norm_w,
                                   float eps, void *stream) {
  if (!w_gate || !w_up || !x || !out) return -EINVAL;
  if (n_out < 0 || k <= 0) return -EINVAL;
  if (n_out == 0) return 0;
  if (n_out > INT_MAX / 2 || k > INT_MAX / 2) return -EOVERFLOW;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (norm_w && !fast_ok(k, {w_gate, w_up, x, norm_w})) return -ENOTSUP;
  if (norm_w && k <= kStageMaxK && 2 * n_out * k >= kStagedMinFloats)
    gemv_swiglu_staged_kernel<<<staged_grid(n_out), kThreads, sizeof(float) * static_cast<size_t>(k), s>>>(
        w_gate, w_up, x, out, int(n_out), int(k), norm_w, eps);
  else if (fast_ok(k, {w_gate, w_up, x}))
    gemv_swiglu_kernel<<<grid_for(n_out), kThreads, 0, s>>>(w_gate, w_up, x, out, int(n_out), int(k),
                                                            norm_w, eps);
  else
    gemv_generic_kernel<<<grid_for(n_out), kThreads, 0, s>>>(w_gate, x, out, nullptr, int(n_out),
                                                              int(k), 2, w_up);
  return ikv::launch_status();
}
