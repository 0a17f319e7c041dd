/*
 * ikv_probe.h — measurement probes built into libikv.so.
 *
 * No counterpart in the reference: these kernels exist so that bench.py can
 * report, in the same run, the HBM bandwidth this box actually sustains
 * next to the nominal 8 TB/s peak — a long streaming read, a streaming read
 * of one decode layer's size (33.6 MB), and the cost of an empty kernel.
 * Conventions as in ikv.h (device pointers, stream as void*, 0 / -errno /
 * hipError_t).
 */
#ifndef IKV_PROBE_H
#define IKV_PROBE_H

#include <stddef.h>

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

#ifdef __cplusplus
}
#endif

#endif /* IKV_PROBE_H */
