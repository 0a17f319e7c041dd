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
 *   oracle_mul_mat_f32     float64 brute force; identity matrix; rows of w
 *                          selected by one-hot x are returned exactly
 *   oracle_get_rows_f32    rows equal the table's rows bytewise
 *   oracle_silu_f32        closed forms silu(0) = 0, silu(x) - silu(-x) = x
 *   oracle_sample_greedy   ties -> lowest id; NaN / +inf / all -inf -> -1
 *   oracle_qwen3_step      op-by-op recomposition from the functions above
 *                          (float64 brute force of a one-layer model);
 *                          cached decode == recompute of the whole prefix
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

/* ---- ops around the path and the whole Qwen3 step (oracle_model.c) ---- */

/* compute_get_rows (src/backends/cpu_backend.cpp:259-332): out[i] =
 * table[ids[i]], rows of row_len floats. Returns -22 for an id outside
 * [0, n_rows) (the reference reads outside the table there). */
int oracle_get_rows_f32(const float *table, const int32_t *ids, float *out, int64_t n_ids,
                        int64_t row_len, int64_t n_rows);

/* compute_mul_mat (src/backends/cpu_backend.cpp:386-424): out[t][o] =
 * sum_k x[t][k] * w[o][k], one float accumulator from 0.0f in index order,
 * one pool task per output element. w: [n_out][k]; x: [m][k]. */
void oracle_mul_mat_f32(const float *w, const float *x, float *out, int64_t n_out, int64_t k,
                        int64_t m);

/* compute_add / compute_mul / compute_silu (src/backends/cpu_backend.cpp:
 * 636-703) over n floats; out may equal an input. */
void oracle_add_f32(const float *a, const float *b, float *out, int64_t n);
void oracle_mul_f32(const float *a, const float *b, float *out, int64_t n);
void oracle_silu_f32(const float *x, float *out, int64_t n);

/* sample_greedy (src/sampler.cpp:42-65): argmax, ties -> lowest id; -1 for
 * NaN, +inf, all -inf or n <= 0 (the reference's invalid_argument). */
int32_t oracle_sample_greedy(const float *logits, int64_t n);

typedef struct {
    int64_t n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, n_ctx_train;
    float rms_eps, rope_theta;
} oracle_qwen3_hparams;

/* One layer's weights, rows as in the reference's ggml tensors
 * (src/model.cpp:192-306): wq [n_head*head_dim][n_embd], wk/wv
 * [n_head_kv*head_dim][n_embd], wo [n_embd][n_head*head_dim], ffn_gate/up
 * [n_ff][n_embd], ffn_down [n_embd][n_ff]; norms [n_embd] / [head_dim]. */
typedef struct {
    const float *attn_norm, *wq, *wk, *wv, *q_norm, *k_norm, *wo, *ffn_norm, *ffn_gate, *ffn_up,
        *ffn_down;
} oracle_qwen3_layer;

/* One step of Qwen3Model::build_graph (src/models/Qwen3.cpp:4-136) with the
 * ops above, in graph order: tokens at positions n_past .. n_past+n_tokens-1;
 * appends this step's K (after RoPE) and V to k_cache[l] / v_cache[l]
 * ([capacity][n_head_kv][head_dim]) at n_past; theta: the angle table
 * [n_ctx_train][head_dim/2]; logits: [n_tokens][n_vocab] (only the last row
 * is computed when last_row_only). output is the tied token_embd when the
 * model has no separate output weight. Returns 0, -22 or -12. */
int oracle_qwen3_step(const oracle_qwen3_hparams *hp, const oracle_qwen3_layer *layers,
                      const float *token_embd, const float *output_norm, const float *output,
                      const float *theta, const int32_t *tokens, int64_t n_tokens, int64_t n_past,
                      float *const *k_cache, float *const *v_cache, float *logits,
                      int last_row_only);

#ifdef __cplusplus
}
#endif

#endif
