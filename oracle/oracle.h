/*
 * oracle.h — CPU restatement of Infer-LLM's hot-path CPU ops.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the HIP path is
 * compared against. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it. The product (libikv.so) never links it.
 *
 * Every function restates one reference function; the citation is on each
 * declaration. Layouts follow the reference Tensor convention
 * (include/tensor.hpp:12-29): dims[0] is innermost, so a [D, H, T] tensor is
 * stored token-major, head next, dim innermost.
 *
 * Parity pins (what checks each function; see tests/test_oracle.py):
 *   oracle_rms_norm_f32    float64 brute force; RMS of output == 1 for w == 1
 *   oracle_rope_theta_table float64 closed form pos * theta^(-2i/D)
 *   oracle_rope_neox_f32   pos 0 == identity; per-pair norm preserved;
 *                          float64 rotation by the table's angles
 *   oracle_flash_attn_f32  float64 brute force; L=1 -> v0; identical keys ->
 *                          mean(V); GQA head permutation; causal future
 *                          perturbation; decode == prefill row
 *   oracle_cpy             byte equality + sentinel bytes untouched
 */
#ifndef IKV_ORACLE_H
#define IKV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Worker pool following ThreadPool (src/backends/cpu_backend.cpp:6-95):
 * persistent workers, one index per atomic fetch, the calling thread also
 * takes indices. n_workers <= 1 runs every index on the calling thread
 * (cpu_backend.cpp:66-69). Returns the number of threads that execute work
 * (n_workers + 1 when n_workers > 1, else 1). */
int oracle_set_workers(int n_workers);
/* Default worker count: hardware_concurrency * 0.5, at least 1, or
 * INFERLLM_THREADS when set (cpu_backend.cpp:167-198). */
int oracle_default_workers(void);

/* compute_rms_norm (src/backends/cpu_backend.cpp:335-382).
 * x, out: rows x dim floats; w: dim floats. */
void oracle_rms_norm_f32(const float *x, const float *w, float *out,
                         int64_t rows, int64_t dim, float eps);

/* GraphContext::get_rope_theta_table (src/graph.cpp:92-135).
 * out: [n_ctx][head_dim/2] floats. */
void oracle_rope_theta_table(float theta_base, uint32_t head_dim,
                             uint32_t n_ctx, float *out);

/* compute_rope (src/backends/cpu_backend.cpp:443-523), NeoX half split.
 * x, out: [n_tokens][n_heads][head_dim]; pos: n_tokens int32;
 * theta: [n_ctx][head_dim/2]. Returns 0, or -22 when a position is outside
 * [0, n_ctx) (the reference reads out of bounds there; the oracle refuses). */
int oracle_rope_neox_f32(const float *x, const int32_t *pos,
                         const float *theta, int64_t n_ctx, float *out,
                         int64_t head_dim, int64_t n_heads, int64_t n_tokens);

/* compute_flash_attn (src/backends/cpu_backend.cpp:525-634).
 * q: [n_q][n_head][D]; k, v: [n_kv][n_head_kv][D]; out: [n_q][n_head][D].
 * Key k is visible to query t iff k <= n_past + t (cpu_backend.cpp:578).
 * The scale is 1/sqrtf(D) (cpu_backend.cpp:575; AttnParams.scale ignored). */
void oracle_flash_attn_f32(const float *q, const float *k, const float *v,
                           float *out, int64_t head_dim, int64_t n_head,
                           int64_t n_q, int64_t n_head_kv, int64_t n_kv,
                           int64_t n_past);

/* compute_cpy (src/backends/cpu_backend.cpp:705-742): contiguous byte copy.
 * Returns 0, or -22 for null pointers. */
int oracle_cpy(void *dst, const void *src, size_t bytes);

/* Decode step of the path (one layer): append one token's K,V rows at
 * position n_past into the caches, then attend over [0, n_past+1) —
 * compute_cpy x2 then compute_flash_attn, as ordered by ModelBase::append_kv
 * (src/model.cpp:602-625). k_cache/v_cache: [capacity][n_head_kv][D]. */
void oracle_decode_append_attn_f32(const float *q, const float *k_new,
                                   const float *v_new, float *k_cache,
                                   float *v_cache, float *out,
                                   int64_t head_dim, int64_t n_head,
                                   int64_t n_head_kv, int64_t n_past);

#ifdef __cplusplus
}
#endif

#endif
