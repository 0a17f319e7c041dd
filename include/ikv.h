/*
 * ikv.h — C-ABI of the MI355X (gfx950) KV-cache hot path.
 *
 * This is the layer the HIP backend's dispatch calls, in the place where the
 * reference's CUDA backend calls CUDA_F32::compute_* (reference
 * include/kernels/cuda/kernel_f32.hpp:5-29, dispatched from
 * src/backends/cuda_backend.cpp:208-241). Arguments are plain pointers and
 * sizes; no C++ or torch types cross it.
 *
 * Layouts are the reference Tensor layouts (include/tensor.hpp:12-29,
 * dims[0] innermost), all contiguous F32:
 *   q, out      [n_q][n_head][head_dim]
 *   k, v caches [n_kv][n_head_kv][head_dim]   (token stride n_head_kv*head_dim)
 *   theta/sin/cos tables [n_ctx][head_dim/2]
 *
 * Conventions:
 *   - Device pointers unless a name ends in _host.
 *   - stream is a hipStream_t passed as void*; NULL means the null stream.
 *   - No entry point allocates, frees or synchronises. Work is enqueued on
 *     `stream` and errors inside kernels never fault the device.
 *   - Return value: 0 on success; a negative errno (-EINVAL, -ENOTSUP,
 *     -EOVERFLOW, -ENOSPC) when arguments are rejected before any launch; a positive
 *     hipError_t when a launch fails. The HIP backend maps negative codes to
 *     std::errc and positive ones to std::errc::io_error, as check_cuda does
 *     (reference include/cuda_util.hpp:7-16).
 *   - Bad data inside a launch (a position, block entry or token id out of
 *     range) never faults: the kernel ORs one IKV_STATUS_* bit into the
 *     caller's device status word, when one is given, and carries on.
 */
#ifndef IKV_H
#define IKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Bits of the device status word (see the conventions above). */
#define IKV_STATUS_POSITION 1 /* a RoPE position outside [0, n_ctx) */
#define IKV_STATUS_BLOCK 2    /* a paged block-table entry outside the pool */
#define IKV_STATUS_TOKEN 4    /* a get_rows id outside the table */

/* Version string of the library, e.g. "ikv 0.1 gfx950". */
const char *ikv_version(void);

/* ---------------------------------------------------------------------
 * KV append.
 * Replaces CUDA_F32::compute_cpy (src/kernels/cuda/kernel_f32.cu:305-319) and
 * CPUBackend::compute_cpy (src/backends/cpu_backend.cpp:705-742): copies
 * n_rows * row_bytes contiguous bytes from src_rows to dst_rows (the writable
 * cache view [n_past, n_past+n_new)). Byte-exact; nothing else is written.
 * ------------------------------------------------------------------- */
int ikv_append_f32(void *dst_rows, const void *src_rows, size_t n_rows, size_t row_bytes,
                   void *stream);

/* ---------------------------------------------------------------------
 * Decode attention, one query token, GQA, split-K over the context, with an
 * optional fused KV append. One kernel launch: the last split of each KV head
 * to finish merges that head's split partials.
 * Replaces compute_flash_attn for n_q == 1 (src/kernels/cuda/kernel_f32.cu:
 * 452-511; CPU semantics src/backends/cpu_backend.cpp:525-634).
 *
 *   q        [n_head][head_dim]
 *   k_cache, v_cache  readable cache views, [n_kv][n_head_kv][head_dim]
 *   k_new, v_new      NULL, or the new token's rows [n_head_kv][head_dim].
 *            When given, row n_kv-1 of the caches is read from them and is
 *            also written to the caches (the append of ModelBase::append_kv,
 *            src/model.cpp:602-625, fused into the attention launch).
 *   out      [n_head][head_dim]
 *   scale    softmax scale; <= 0 selects 1/sqrtf(head_dim)
 *   workspace  device memory of ikv_attn_decode_workspace_bytes() bytes
 *            for the split partials and one arrival counter per KV head.
 *            It must be zero-filled before its first use (hipMemset at
 *            allocation); every launch leaves the counters at zero again,
 *            so the same workspace serves every later launch and context
 *            length of every shape with the same n_head_kv that it is large
 *            enough for (zero it again before using it for another n_head_kv;
 *            the split count is not monotone in n_kv, so size it for every
 *            context it will serve). Unused, and may be NULL, when the
 *            context fits one split. Launches that share one workspace must
 *            be ordered (same stream); concurrent ones race.
 * The split kernel takes head_dim 128 with n_head/n_head_kv 1, 2, 4 or 8.
 * Any other head_dim in [1, 512] and any n_head that n_head_kv divides run
 * a generic path instead: the append, then two launches, the context split
 * over workgroups that each serve all query heads of one KV head and a merge
 * of the splits in order (their partials in the workspace), or, when
 * n_head/n_head_kv * ceil(head_dim/64) exceeds 32 (dims per lane rounded to
 * 1, 2, 4, 8) or the workspace is smaller than
 * ikv_attn_decode_workspace_bytes() asks, one workgroup per query head over
 * all keys. With qk-norm + RoPE folded in, those run first as their own
 * kernels into the workspace, which then holds the rotated q and k rows
 * ahead of the partials. Same semantics within the attention bar, slower,
 * no replay form. Larger head_dim: -ENOTSUP.
 * ------------------------------------------------------------------- */
size_t ikv_attn_decode_workspace_bytes(int n_head, int n_head_kv, int head_dim, int64_t n_kv);

int ikv_attn_decode_f32(const float *q, float *k_cache, float *v_cache, const float *k_new,
                        const float *v_new, float *out, int n_head, int n_head_kv, int head_dim,
                        int64_t n_kv, float scale, void *workspace, size_t workspace_bytes,
                        void *stream);

/* ---------------------------------------------------------------------
 * ikv_attn_decode_f32 without a workspace argument, for callers that
 * cannot allocate one: code under HIP graph capture, serving loops and
 * harnesses that forbid allocation. It has no counterpart in the reference.
 * It allocates nothing (no hipMalloc, no allocating library call): the
 * split partials and arrival counters live in a device array of
 * IKV_DECODE_NOALLOC_SCRATCH_BYTES that the library holds on each device it
 * runs on until the process ends. Every call on one device shares that
 * array, so calls that overlap on one device race (order them on one
 * stream). Each call clears the counters it needs with a fill kernel on
 * `stream` before the attention launch (no memset, so the call may be
 * captured in a HIP graph). The first call on a device looks up the array's
 * address there (hipGetSymbolAddress), so make it outside stream capture. Returns -ENOSPC when
 * ikv_attn_decode_workspace_bytes() of the shape exceeds that size (every
 * supported shape of up to 128 KV heads fits). Other arguments, results and
 * return codes as for ikv_attn_decode_f32: the output and cache rows are
 * bit-identical to its.
 * ------------------------------------------------------------------- */
#define IKV_DECODE_NOALLOC_SCRATCH_BYTES (2u << 20)

int ikv_attn_decode_noalloc_f32(const float *q, float *k_cache, float *v_cache,
                                const float *k_new, const float *v_new, float *out, int n_head,
                                int n_head_kv, int head_dim, int64_t n_kv, float scale,
                                void *stream);

/* ---------------------------------------------------------------------
 * Decode with the step's qk-RMSNorm + RoPE folded into the same launch:
 *   q     = rope(rms_norm(q_raw, q_norm_w)),  k = rope(rms_norm(k_raw, k_norm_w))
 * per head row (ikv_qk_norm_rope_f32's arithmetic, at position pos[0]), then
 * k (rotated) and v_new are appended at row n_kv-1 and ikv_attn_decode_f32's
 * attention runs — the RMS_NORM -> ROPE -> CPY -> VIEW -> FLASH_ATTN_EXT
 * chain of one Qwen3 layer for one token (src/models/Qwen3.cpp:66-83). The
 * appended key row is bit-identical to the one the separate ops produce.
 * q_raw [n_head][head_dim], k_raw / v_new [n_head_kv][head_dim]; norm
 * weights [head_dim]; pos: device int32; sin/cos tables [n_ctx][head_dim/2]
 * as for ikv_rope_neox_f32. A position outside [0, n_ctx) does not fault:
 * q and k become zero rows and IKV_STATUS_POSITION is raised in *status.
 * Workspace and other arguments as for ikv_attn_decode_f32.
 * ------------------------------------------------------------------- */
int ikv_attn_decode_rope_f32(const float *q_raw, const float *k_raw, const float *v_new,
                             float *k_cache, float *v_cache, float *out, int n_head, int n_head_kv,
                             int head_dim, int64_t n_kv, float scale, const float *q_norm_w,
                             const float *k_norm_w, float eps, const int32_t *pos,
                             const float *sin_tab, const float *cos_tab, int64_t n_ctx,
                             int *status, void *workspace, size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------
 * The whole attention input side of one Qwen3 layer for one token, in one
 * launch: the q/k/v projections of x (attn_norm folded in when attn_norm_w is
 * not NULL, as for ikv_gemv3_f32, include/ikv_model.h) written to q_out
 * [n_head][head_dim], k_out and v_out [n_head_kv][head_dim], then
 * ikv_attn_decode_rope_f32 on them (qk-RMSNorm + RoPE at pos[0], append at
 * row n_kv-1, attention) — the MUL_MAT x3 -> RMS_NORM -> ROPE -> CPY -> VIEW
 * -> FLASH_ATTN_EXT chain of src/models/Qwen3.cpp:53-88. For short contexts
 * only (one decode split, n_kv <= 128): -ENOTSUP otherwise, and for n_embd
 * not a multiple of 1024, and the caller makes the two launches. Outputs and
 * cache rows are bit-identical to ikv_gemv3_f32 followed by
 * ikv_attn_decode_rope_f32. w_q [n_head*head_dim][n_embd], w_k and w_v
 * [n_head_kv*head_dim][n_embd], x [n_embd]; the workspace is a decode
 * workspace (ikv_attn_decode_workspace_bytes, zero-filled once): its
 * arrival counters, which every launch leaves at zero again.
 * ------------------------------------------------------------------- */
int ikv_qkv_attn_decode_f32(const float *w_q, const float *w_k, const float *w_v, const float *x,
                            const float *attn_norm_w, float attn_eps, float *q_out, float *k_out,
                            float *v_out, int64_t n_embd, float *k_cache, float *v_cache,
                            float *out, int n_head, int n_head_kv, int head_dim, int64_t n_kv,
                            float scale, const float *q_norm_w, const float *k_norm_w, float eps,
                            const int32_t *pos, const float *sin_tab, const float *cos_tab,
                            int64_t n_ctx, int *status, void *workspace, size_t workspace_bytes,
                            void *stream);

/* ---------------------------------------------------------------------
 * Replay forms, for a decode step recorded once (a captured HIP graph) and
 * replayed at successive positions; they have no counterpart in the
 * reference, whose step is rebuilt and relaunched every token
 * (src/model.cpp:164-311). The context is not an argument: every launch
 * reads pos[0] on the device and attends over n_kv = pos[0] + 1 keys,
 * appending at row pos[0]. The launch is planned for n_kv_max keys (its
 * grid and workspace); for every n_kv in [n, ikv_attn_decode_replay_limit(
 * ..., n, width)] a launch planned for that limit gives bit-identical
 * results to ikv_attn_decode_rope_f32 / ikv_qkv_attn_decode_f32 at n_kv
 * (it only adds empty splits). pos[0] outside [0, n_kv_max) raises
 * IKV_STATUS_POSITION in *status and the launch runs as n_kv_max keys
 * (results invalid, accesses in bounds: the caches must hold n_kv_max
 * rows). ikv_attn_decode_rope_paged_replay_f32 (below, with the paged
 * cache) is the paged form: it reads block-table entries only for blocks
 * that hold keys [0, pos[0]], so the table need cover only those.
 * ------------------------------------------------------------------- */
int ikv_attn_decode_rope_replay_f32(const float *q_raw, const float *k_raw, const float *v_new,
                                    float *k_cache, float *v_cache, float *out, int n_head,
                                    int n_head_kv, int head_dim, int64_t n_kv_max, float scale,
                                    const float *q_norm_w, const float *k_norm_w, float eps,
                                    const int32_t *pos, const float *sin_tab,
                                    const float *cos_tab, int64_t n_ctx, int *status,
                                    void *workspace, size_t workspace_bytes, void *stream);
int ikv_qkv_attn_decode_replay_f32(const float *w_q, const float *w_k, const float *w_v,
                                   const float *x, const float *attn_norm_w, float attn_eps,
                                   float *q_out, float *k_out, float *v_out, int64_t n_embd,
                                   float *k_cache, float *v_cache, float *out, int n_head,
                                   int n_head_kv, int head_dim, int64_t n_kv_max, float scale,
                                   const float *q_norm_w, const float *k_norm_w, float eps,
                                   const int32_t *pos, const float *sin_tab, const float *cos_tab,
                                   int64_t n_ctx, int *status, void *workspace,
                                   size_t workspace_bytes, void *stream);
/* The largest m in [n_kv, n_kv + width - 1] such that a replay launch
 * planned for m keys is bit-identical to the per-context launch at every
 * context in [n_kv, m]; 0 for a shape the decode rejects or width < 1. */
int64_t ikv_attn_decode_replay_limit(int n_head, int n_head_kv, int head_dim, int64_t n_kv,
                                     int64_t width);

/* ---------------------------------------------------------------------
 * Prefill / general attention, n_q >= 1 query tokens, causal: key j is
 * visible to query t iff j <= n_past + t (src/backends/cpu_backend.cpp:578,
 * src/kernels/cuda/kernel_f32.cu:346). F32 MFMA tiles; K/V tiles staged in
 * LDS and shared by the n_head/n_head_kv query heads of a KV head.
 * Replaces compute_flash_attn for n_q > 1. Needs no workspace.
 * The MFMA kernel takes head_dim 128 with n_head/n_head_kv 1, 2, 4 or 8;
 * any other head_dim in [1, 512] and any n_head that n_head_kv divides run
 * the generic path (decode above). Larger head_dim: -ENOTSUP. The MFMA
 * kernel's shapes with n_head_kv > 65536: -EOVERFLOW.
 * ------------------------------------------------------------------- */
int ikv_attn_prefill_f32(const float *q, const float *k, const float *v, float *out, int n_head,
                         int n_head_kv, int head_dim, int64_t n_q, int64_t n_kv, int64_t n_past,
                         float scale, void *stream);

/* ---------------------------------------------------------------------
 * Paged KV cache. The reference's KVCacheConfig::block_tokens > 0
 * (include/kvcache/kvutil.hpp:43) asks for a cache cut into blocks, with a
 * sequence's tokens spread over several storage slices
 * (src/kvcache/kvstrategy.cpp:83-158) and an attention kernel that follows
 * them (the TODO at include/op_factory.hpp:38). Here one layer's K (and V)
 * cache is a pool of n_pool_blocks blocks of block_tokens token rows,
 * [n_pool_blocks * block_tokens][n_head_kv][head_dim], and logical token t of
 * a sequence lives in pool row
 *     block_table[t / block_tokens] * block_tokens + t % block_tokens.
 * block_tokens must be a positive multiple of 64 (a tile of the kernels never
 * straddles two blocks). block_table is device memory with an entry for every
 * block the call touches; an entry outside [0, n_pool_blocks) does not fault:
 * reads take block 0's rows instead, writes to that block are dropped (no
 * other sequence's rows are touched), and IKV_STATUS_BLOCK is raised in
 * *status (device int, if non-NULL).
 * ------------------------------------------------------------------- */
typedef struct ikv_kv_pages {
    const int32_t *block_table;
    int64_t block_tokens;
    int64_t n_pool_blocks;
    int32_t *status;
} ikv_kv_pages;

/* Writes n_rows token rows (row_bytes each, one token's K or V for all KV
 * heads) from src_rows to logical tokens [first_token, first_token + n_rows)
 * of the paged pool. Byte-exact; nothing else is written. row_bytes must be a
 * multiple of 16. */
int ikv_append_paged_f32(void *pool, const void *src_rows, const ikv_kv_pages *pages,
                         int64_t first_token, size_t n_rows, size_t row_bytes, void *stream);

/* ikv_attn_decode_f32 / ikv_attn_decode_rope_f32 / ikv_attn_prefill_f32 over
 * a paged cache: k_pool / v_pool are the pools, tokens [0, n_kv) are read
 * through `pages`, and the fused append writes logical row n_kv - 1. Same
 * splits, same arithmetic: the results are bit-identical to the contiguous
 * entry points' on the same logical cache. Workspaces as for those. */
int ikv_attn_decode_paged_f32(const float *q, float *k_pool, float *v_pool,
                              const ikv_kv_pages *pages, const float *k_new, const float *v_new,
                              float *out, int n_head, int n_head_kv, int head_dim, int64_t n_kv,
                              float scale, void *workspace, size_t workspace_bytes, void *stream);
int ikv_attn_decode_rope_paged_f32(const float *q_raw, const float *k_raw, const float *v_new,
                                   float *k_pool, float *v_pool, const ikv_kv_pages *pages,
                                   float *out, int n_head, int n_head_kv, int head_dim,
                                   int64_t n_kv, float scale, const float *q_norm_w,
                                   const float *k_norm_w, float eps, const int32_t *pos,
                                   const float *sin_tab, const float *cos_tab, int64_t n_ctx,
                                   int *status, void *workspace, size_t workspace_bytes,
                                   void *stream);
/* The replay form of ikv_attn_decode_rope_paged_f32 (see the replay forms
 * above: the context is pos[0] + 1, read on the device; planned for
 * n_kv_max keys; bit-identical to ikv_attn_decode_rope_paged_f32 at every
 * context the replay limit allows). */
int ikv_attn_decode_rope_paged_replay_f32(const float *q_raw, const float *k_raw,
                                          const float *v_new, float *k_pool, float *v_pool,
                                          const ikv_kv_pages *pages, float *out, int n_head,
                                          int n_head_kv, int head_dim, int64_t n_kv_max,
                                          float scale, const float *q_norm_w,
                                          const float *k_norm_w, float eps, const int32_t *pos,
                                          const float *sin_tab, const float *cos_tab,
                                          int64_t n_ctx, int *status, void *workspace,
                                          size_t workspace_bytes, void *stream);
int ikv_attn_prefill_paged_f32(const float *q, const float *k_pool, const float *v_pool,
                               const ikv_kv_pages *pages, float *out, int n_head, int n_head_kv,
                               int head_dim, int64_t n_q, int64_t n_kv, int64_t n_past,
                               float scale, void *stream);

/* ---------------------------------------------------------------------
 * RMS norm over rows of `dim` floats: out = (x * s) * w with
 * s = float(1 / sqrt(sum_d double(x_d*x_d) / dim + eps)) — the arithmetic of
 * CPUBackend::compute_rms_norm (src/backends/cpu_backend.cpp:335-382).
 * The double sum is taken in parallel and the float scale is certified
 * against the reference's index-order sum: when the parallel sum's double
 * scale lies farther from a float rounding midpoint than the two sums can
 * differ, both round to the same float; otherwise (about 2^-16 of rows) the
 * row is summed again in index order. Results are bit-identical to the
 * reference for every row, and to the norm folded into ikv_gemv3_f32 /
 * ikv_gemv_swiglu_f32.
 * Replaces CUDA_F32::compute_rms_norm (src/kernels/cuda/kernel_f32.cu:16-90).
 * ------------------------------------------------------------------- */
int ikv_rms_norm_f32(const float *x, const float *w, float *out, int64_t rows, int64_t dim,
                     float eps, void *stream);

/* ---------------------------------------------------------------------
 * Host helper: the RoPE angle table [n_ctx][head_dim/2] of
 * GraphContext::get_rope_theta_table (src/graph.cpp:92-135):
 * freq_i = 1.0f / powf(theta_base, (2.0f*i) / head_dim) in float, widened
 * to double; theta_host[pos][i] = (float)(pos * freq_i). head_dim even.
 * ------------------------------------------------------------------- */
int ikv_rope_theta_table_f32(float theta_base, int head_dim, int64_t n_ctx, float *theta_host);

/* ---------------------------------------------------------------------
 * Host helper: sin/cos tables from a RoPE angle table (host memory).
 * sin_host[i] = sinf(theta_host[i]), cos_host[i] = cosf(theta_host[i]) —
 * the per-step computation of src/backends/cpu_backend.cpp:472-487, done
 * once so that the device tables can stay resident in HBM.
 * ------------------------------------------------------------------- */
int ikv_rope_sincos_table_f32(const float *theta_host, size_t count, float *sin_host,
                              float *cos_host);

/* ---------------------------------------------------------------------
 * RoPE, NeoX half split: for pair (j, j+head_dim/2) of every head of token t
 * at position p = pos[t]:  o_j = x0*c - x1*s,  o_{j+h} = x0*s + x1*c  with
 * c = cos_tab[p][j], s = sin_tab[p][j]  (src/backends/cpu_backend.cpp:
 * 443-523). Replaces CUDA_F32::compute_rope (src/kernels/cuda/kernel_f32.cu:
 * 242-301). A position outside [0, n_ctx) does not fault: its rows are
 * written as zeros and IKV_STATUS_POSITION is raised in *status (device int,
 * if non-NULL).
 * x may equal out.
 * ------------------------------------------------------------------- */
int ikv_rope_neox_f32(const float *x, float *out, const int32_t *pos, int64_t n_tokens,
                      int n_heads, int head_dim, const float *sin_tab, const float *cos_tab,
                      int64_t n_ctx, int *status, void *stream);

/* ---------------------------------------------------------------------
 * Fused qk-RMSNorm + RoPE: ikv_rms_norm_f32 over each head row with weight
 * w[head_dim], then ikv_rope_neox_f32, in one launch. Bit-identical to the
 * two ops in sequence (the RMSNorm -> RoPE order of Qwen3Model::build_graph,
 * src/models/Qwen3.cpp:66-71).
 * ------------------------------------------------------------------- */
int ikv_qk_norm_rope_f32(const float *x, const float *w, float *out, const int32_t *pos,
                         int64_t n_tokens, int n_heads, int head_dim, float eps,
                         const float *sin_tab, const float *cos_tab, int64_t n_ctx, int *status,
                         void *stream);

#ifdef __cplusplus
}
#endif

#endif /* IKV_H */
