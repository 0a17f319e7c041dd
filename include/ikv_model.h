/*
 * ikv_model.h — C-ABI of the ops around the KV-cache path that a whole
 * Qwen3 step needs on the MI355X (gfx950): the projections (mul_mat), the
 * token-embedding gather, the elementwise ops of the FFN and residuals, the
 * greedy sampler, and the synthetic weight initialiser of the benchmarks.
 *
 * These replace the reference's CPU / CUDA ops of the same names
 * (src/backends/cpu_backend.cpp:259-332, 386-424, 636-703;
 * src/kernels/cuda/kernel_f32.cu:94-205, 515-630; src/sampler.cpp:42-65) so
 * that the scheduler keeps a whole Qwen3 graph on the HIP backend instead of
 * copying weights to the CPU every step (src/scheduler.cpp:67-69).
 * Conventions as in ikv.h: device pointers unless a name ends in _host,
 * stream as void*, 0 / negative errno / positive hipError_t, F32 row-major
 * with the reference Tensor layout (dims[0] innermost).
 */
#ifndef IKV_MODEL_H
#define IKV_MODEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------
 * mul_mat: out[m][n] = sum_k x[m][k] * w[n][k]   (w: [n_out][k] rows, the
 * ggml [K, N] weight of CPUBackend::compute_mul_mat,
 * src/backends/cpu_backend.cpp:386-424; x: [m][k]; out: [m][n_out]).
 * m == 1 (decode) runs a hand-written streaming GEMV. 2 <= m <= 64 with
 * n_out % 16 == 0, k % 1024 == 0 and 16-byte aligned w and x runs a
 * hand-written F32 MFMA kernel. Other m > 1 with n_out % 64 == 0,
 * k % 64 == 0, k < 2^22 and 16-byte aligned w and x run the tiled F32 MFMA GEMM of
 * ikv_gemm_nt_f32, with K split over several workgroups when its tiles
 * would leave compute units idle: such a call needs a split-K workspace of
 * its device and stream, which the first one allocates (8 MiB + 16 KiB,
 * kept until exit; so make it outside HIP graph capture; -ENOMEM after 64
 * device-stream pairs). Any other shape runs one wavefront per output
 * (m <= 65535, else -ENOTSUP). Every path is deterministic: a fixed
 * summation order per output for given n_out, k and m.
 * residual: NULL, or [m][n_out] added to the result (out may equal
 * residual).
 * ------------------------------------------------------------------- */
int ikv_mul_mat_f32(const float *w, const float *x, float *out, int64_t n_out, int64_t k,
                    int64_t m, const float *residual, void *stream);

/* The hand-written F32 MFMA GEMM of mul_mat for prompts (the same product,
 * CPUBackend::compute_mul_mat, src/backends/cpu_backend.cpp:386-424), for
 * any m >= 1: n_out % 64 == 0, k % 64 == 0, k < 2^22, 16-byte aligned w and x (else
 * -ENOTSUP / -EINVAL, nothing launched). Deterministic (a fixed summation
 * order per output); never splits K, so it allocates nothing. residual as
 * for mul_mat. */
int ikv_gemm_nt_f32(const float *w, const float *x, float *out, int64_t n_out, int64_t k,
                    int64_t m, const float *residual, void *stream);

/* Three projections of one input in one launch (the q, k, v projections of
 * a Qwen3 layer, src/models/Qwen3.cpp:56-58), m == 1:
 * out_i = w_i · x' for i = 0, 1, 2 with w_i [n_i][k], where x' = x, or, when
 * norm_w is not NULL, x' = ikv_rms_norm_f32(x, norm_w, eps) (the layer's
 * attn_norm folded in; k % 1024 == 0 and 16-byte aligned operands, else
 * -ENOTSUP). */
int ikv_gemv3_f32(const float *w0, const float *w1, const float *w2, const float *x, float *out0,
                  float *out1, float *out2, int64_t n0, int64_t n1, int64_t n2, int64_t k,
                  const float *norm_w, float eps, void *stream);

/* SwiGLU FFN input, m == 1: out[n] = (w_up[n] · x') * silu(w_gate[n] · x') —
 * mul_mat(ffn_gate), mul_mat(ffn_up), silu, mul of Qwen3Model::build_graph
 * (src/models/Qwen3.cpp:103-113) in one launch; silu(g) = g / (1 + exp(-g))
 * (src/backends/cpu_backend.cpp:660-673). x' as for ikv_gemv3_f32 (ffn_norm
 * folded in when norm_w is not NULL). */
int ikv_gemv_swiglu_f32(const float *w_gate, const float *w_up, const float *x, float *out,
                        int64_t n_out, int64_t k, const float *norm_w, float eps, void *stream);

/* ---------------------------------------------------------------------
 * get_rows: out[i][:] = table[ids[i]][:] for i < n_ids, rows of row_len
 * floats (CPUBackend::compute_get_rows, src/backends/cpu_backend.cpp:
 * 259-332; the token embedding). An id outside [0, n_rows) does not fault:
 * its output row is zeros and IKV_STATUS_TOKEN (include/ikv.h) is raised in
 * *status (device int, if non-NULL).
 * ------------------------------------------------------------------- */
int ikv_get_rows_f32(const float *table, const int32_t *ids, float *out, int64_t n_ids,
                     int64_t row_len, int64_t n_rows, int *status, void *stream);

/* Elementwise over n floats (src/backends/cpu_backend.cpp:636-703):
 * add: out = a + b; mul: out = a * b; silu: out = x / (1 + exp(-x)).
 * out may equal an input. */
int ikv_add_f32(const float *a, const float *b, float *out, int64_t n, void *stream);
int ikv_mul_f32(const float *a, const float *b, float *out, int64_t n, void *stream);
int ikv_silu_f32(const float *x, float *out, int64_t n, void *stream);
/* out = up * silu(gate): the SILU node and the MUL that consumes it
 * (src/models/Qwen3.cpp:107-112) in one pass, bitwise equal to the two ops.
 * out may equal gate or up. */
int ikv_silu_mul_f32(const float *gate, const float *up, float *out, int64_t n, void *stream);

/* ---------------------------------------------------------------------
 * Greedy sampling on the device (sample_greedy, src/sampler.cpp:42-65):
 * *token = the index of the largest of logits[0, n); ties go to the lowest
 * index. A NaN or +inf logit, or all logits -inf, writes *token = -1 (the
 * reference returns invalid_argument). n must be in [1, 2^31). token is a
 * device int32; token_mirror, if not NULL, receives the same value and may
 * be pinned host memory (hipHostMalloc), so that the host reads the token
 * once the stream has passed this launch, with no copy of its own.
 * ------------------------------------------------------------------- */
int ikv_argmax_f32(const float *logits, int64_t n, int32_t *token, int32_t *token_mirror,
                   void *stream);

/* The same sampler over up to 64 workgroups (no counterpart in the reference:
 * its sampler runs on the host). workspace: device memory of at least
 * ikv_argmax_workspace_bytes() bytes, 256-byte aligned, zero-filled once
 * before its first use; each call leaves it as it expects to find it, so it
 * is reused call after call. Calls sharing a workspace must not overlap
 * (one stream). Returns -EINVAL for a missing, small or misaligned
 * workspace. The result equals ikv_argmax_f32's. */
size_t ikv_argmax_workspace_bytes(void);
int ikv_argmax_ws_f32(const float *logits, int64_t n, int32_t *token, int32_t *token_mirror,
                      void *workspace, size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------
 * Host helper: the benchmarks' synthetic weights. out_host[i] =
 * std * N(0,1) sample number (offset + i) of the stream `seed`:
 * splitmix64 outputs 2j+1 and 2j+2 of the seed give the uniforms of
 * Box-Muller pair j (u1 = (z1 >> 11 + 1) 2^-53, u2 = (z2 >> 11) 2^-53,
 * r = sqrt(-2 ln u1), normals r cos(2 pi u2), r sin(2 pi u2)), times std,
 * computed in double and rounded once to float. Any split of [0, n) over calls gives the
 * same values. Uses up to `threads` host threads (<= 1: the calling thread).
 * ------------------------------------------------------------------- */
int ikv_synth_normal_f32(uint64_t seed, uint64_t offset, size_t n, double std, float *out_host,
                         int threads);

#ifdef __cplusplus
}
#endif

#endif /* IKV_MODEL_H */
