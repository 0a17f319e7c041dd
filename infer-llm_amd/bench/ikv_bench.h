/*
 * ikv_bench.h — the measurement library libikv_bench.so, which bench.py loads
 * beside libikv.so; nothing of the KV-cache path links it.
 *
 * No counterpart in the reference. It holds
 *  - probes that report, in the same run, what this box sustains next to the
 *    nominal peaks: a streaming read of any size (a long one, and one the
 *    size of a decode layer, 33.6 MB), and the cost of an empty kernel;
 *  - a build of the decode kernels (attn_decode.hip) with phase stamps, whose
 *    entry points are those of include/ikv.h, and the reader of the stamps;
 *  - the prefill GEMM (gemm.hip) on a chosen tile shape.
 * Conventions as in ikv.h (device pointers, stream as void*, 0 / -errno /
 * hipError_t).
 */
#ifndef IKV_BENCH_H
#define IKV_BENCH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reads `bytes` (a multiple of 16) from src with `grid` workgroups of 512
 * threads. Workgroup b reads the b-th of `grid` contiguous slices; each lane
 * issues `loads_per_lane` (1, 4, 8 or 16) independent 16-byte non-temporal
 * loads before using any, so a slice of at most grid * 8 KiB * loads_per_lane
 * bytes is in flight at once. Each workgroup writes one float of its sum to
 * sink[blockIdx] (sink holds >= grid floats). */
int ikv_probe_read(const void *src, size_t bytes, float *sink, int grid, int loads_per_lane,
                   void *stream);

/* Launches an empty kernel of `grid` workgroups. */
int ikv_probe_empty(int grid, void *stream);

/* The phase stamps of the last decode launch of this library's decode build:
 * for workgroup w = split * n_head_kv + kv_head (w < 1024), 16 words at
 * 16 w: the 100 MHz s_memrealtime count at its entry, first tile scored,
 * last tile scored (wave 0), waves merged, partial published, arrival
 * counted, merge done (the merging workgroup), then XCC id | role << 8
 * (role 0 published, 1 merged, 2 one split), then each wave's last tile
 * scored. read copies n_words (<= 16384) words to host memory; clear zeroes
 * them. */
int ikv_bench_timeline_read(unsigned long long *dst, size_t n_words);
int ikv_bench_timeline_clear(void);

/* ikv_gemm_nt_f32 (include/ikv_model.h) on tile shape `tile` (tokens x
 * outputs: 0 128 x 128, 1 64 x 64, 2 64 x 32, 3 32 x 64, 4 32 x 32) with K
 * split over n_split workgroups per tile (1 <= n_split <= k / 64), for the
 * benchmark's sweep of the plans that ikv_mul_mat_f32 chooses among. For
 * n_split > 1, ws holds 16 KiB of tile counters (zero before the first
 * call; each call leaves them zero) followed by the partial tiles
 * (ws_bytes in all); -EINVAL when they do not fit. */
int ikv_bench_gemm_nt_tile_f32(const float *w, const float *x, float *out, int64_t n_out,
                               int64_t k, int64_t m, const float *residual, int tile,
                               int n_split, void *ws, size_t ws_bytes, void *stream);

/* The plan ikv_mul_mat_f32 takes for an n_out x k x m product: tile code
 * (as above) and K splits, written to *tile and *n_split. */
int ikv_bench_gemm_plan(int64_t n_out, int64_t k, int64_t m, int *tile, int *n_split);

#ifdef __cplusplus
}
#endif

#endif /* IKV_BENCH_H */
