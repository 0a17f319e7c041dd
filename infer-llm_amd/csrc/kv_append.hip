// kv_append.hip — byte-exact KV append into the contiguous cache.
//
// Replaces the D2D cudaMemcpyAsync of CUDA_F32::compute_cpy
// (reference src/kernels/cuda/kernel_f32.cu:305-319). The writable cache view
// [n_past, n_past+n_new) is contiguous (token stride = row_bytes), so the
// append is one linear copy of n_rows*row_bytes bytes. HBM-bound: every byte
// is read once and written once, with 16-byte accesses when both pointers and
// the size allow it. No arithmetic touches the data, so the copy is bit-exact.
// The paged form scatters token rows into the blocks of a paged pool.
#include "ikv_common.hpp"
#include "../../include/ikv.h"

namespace {

__global__ __launch_bounds__(256) void copy16_kernel(uint4 *__restrict__ dst,
                                                      const uint4 *__restrict__ src, size_t n16) {
  size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (; i < n16; i += stride) dst[i] = src[i];
}

__global__ __launch_bounds__(256) void copy1_kernel(unsigned char *__restrict__ dst,
                                                     const unsigned char *__restrict__ src,
                                                     size_t n) {
  size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (; i < n; i += stride) dst[i] = src[i];
}

// Row i of src goes to pool row table[t / bt] * bt + t % bt, t = first + i;
// 16-byte pieces, per_row of them per row.
__global__ __launch_bounds__(256) void scatter16_kernel(uint4 *__restrict__ pool,
                                                         const uint4 *__restrict__ src,
                                                         ikv::Pages pg, int64_t first,
                                                         size_t n16, size_t per_row) {
  size_t u = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (; u < n16; u += stride) {
    const size_t i = u / per_row;
    const size_t c = u - i * per_row;
    const int64_t t = first + static_cast<int64_t>(i);
    const int64_t b = t / pg.bt;
    const int blk = pg.table[b];
    if (static_cast<unsigned>(blk) >= static_cast<unsigned>(pg.n_blocks)) {
      ikv::raise_status(pg.status, IKV_STATUS_BLOCK);  // dropped: no block to write
      continue;
    }
    const size_t row = static_cast<size_t>(blk) * pg.bt + static_cast<size_t>(t - b * pg.bt);
    pool[row * per_row + c] = src[u];
  }
}

unsigned grid_for(size_t items) {
  // Enough workgroups to cover every CU of all 8 XCDs several times over,
  // capped so large appends loop inside the kernel.
  size_t g = (items + 255) / 256;
  if (g > 4096) g = 4096;
  if (g == 0) g = 1;
  return static_cast<unsigned>(g);
}

}  // namespace

extern "C" int ikv_append_f32(void *dst_rows, const void *src_rows, size_t n_rows,
                              size_t row_bytes, void *stream) {
  if (n_rows == 0 || row_bytes == 0) return 0;
  if (!dst_rows || !src_rows) return -EINVAL;
  if (row_bytes > SIZE_MAX / n_rows) return -EOVERFLOW;
  const size_t bytes = n_rows * row_bytes;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (ikv::aligned16(dst_rows) && ikv::aligned16(src_rows) && (bytes & 15u) == 0) {
    const size_t n16 = bytes / 16;
    copy16_kernel<<<grid_for(n16), 256, 0, s>>>(static_cast<uint4 *>(dst_rows),
                                                static_cast<const uint4 *>(src_rows), n16);
  } else {
    copy1_kernel<<<grid_for(bytes), 256, 0, s>>>(static_cast<unsigned char *>(dst_rows),
                                                 static_cast<const unsigned char *>(src_rows),
                                                 bytes);
  }
  return ikv::launch_status();
}

extern "C" int ikv_append_paged_f32(void *pool, const void *src_rows, const ikv_kv_pages *pages,
                                    int64_t first_token, size_t n_rows, size_t row_bytes,
                                    void *stream) {
  if (n_rows == 0 || row_bytes == 0) return 0;
  if (!pool || !src_rows || first_token < 0) return -EINVAL;
  ikv::Pages pg;
  if (const int rc = ikv::pages_arg(pages, pg)) return rc;
  if ((row_bytes & 15u) != 0 || !ikv::aligned16(pool) || !ikv::aligned16(src_rows)) return -EINVAL;
  if (row_bytes > SIZE_MAX / n_rows) return -EOVERFLOW;
  if (static_cast<uint64_t>(first_token) + n_rows > static_cast<uint64_t>(INT64_MAX / 2))
    return -EOVERFLOW;
  const size_t per_row = row_bytes / 16;
  const size_t n16 = n_rows * per_row;
  scatter16_kernel<<<grid_for(n16), 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<uint4 *>(pool), static_cast<const uint4 *>(src_rows), pg, first_token, n16,
      per_row);
  return ikv::launch_status();
}

extern "C" const char *ikv_version(void) { return "ikv 0.1 gfx950"; }
