/*
 * oracle_model.c — CPU restatement of the reference's ops around the
 * KV-cache path and of a whole Qwen3 step.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for the HIP model
 * path and the CPU baseline of bench.py. The product never links it.
 *
 * Rounding follows the reference's C++ exactly where it matters for token
 * identity: mul_mat sums x[k]*w[k] in one float accumulator from 0.0f in
 * index order (no FMA: baseline x86-64, -ffp-contract=off); silu is
 * x / (1.0f + expf(-x)).
 */
#include <emmintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "oracle_pool.h"

/* ------------------------------------------------------------------ */
/* get_rows (src/backends/cpu_backend.cpp:259-332)                     */
/* ------------------------------------------------------------------ */

int oracle_get_rows_f32(const float *table, const int32_t *ids, float *out, int64_t n_ids,
                        int64_t row_len, int64_t n_rows) {
    for (int64_t i = 0; i < n_ids; ++i)
        if (ids[i] < 0 || ids[i] >= n_rows) return -22;
    for (int64_t i = 0; i < n_ids; ++i)
        memcpy(out + i * row_len, table + (int64_t)ids[i] * row_len, (size_t)row_len * sizeof(float));
    return 0;
}

/* ------------------------------------------------------------------ */
/* mul_mat (src/backends/cpu_backend.cpp:386-424)                      */
/* ------------------------------------------------------------------ */

struct mm_ctx {
    const float *w, *x;
    float *out;
    int64_t n_out, k;
};

/* One task per output element, i = token * n_out + output (cpu_backend.cpp:
 * 405-423): a sequential float dot product. */
static void mm_elem(int64_t i, void *p) {
    const struct mm_ctx *c = p;
    const int64_t token = i / c->n_out;
    const int64_t output = i % c->n_out;
    const float *x = c->x + token * c->k;
    const float *w = c->w + output * c->k;
    float sum = 0.0f;
    for (int64_t k = 0; k < c->k; ++k) sum += x[k] * w[k];
    c->out[i] = sum;
}

/* Several tokens at once (prompt steps): the same per-element arithmetic on
 * tiles of MM_TO outputs x MM_TT tokens, so that long prompts finish in
 * minutes. Each output element is still one float accumulator from 0.0f,
 * updated for k = 0..K-1 in index order with a rounded product and then a
 * rounded add: _mm_mul_ps / _mm_add_ps are four independent IEEE single
 * multiplies / adds (SSE2, baseline x86-64, no FMA), one lane per output.
 * Only the loop nest differs from mm_elem (16 independent chains in flight
 * instead of one), so every element has mm_elem's bits. */
#define MM_TO 32
#define MM_TT 32

struct mm_tile_ctx {
    const float *w, *x;
    float *out;
    int64_t n_out, k, m, n_otiles;
};

static void mm_tile(int64_t i, void *p) {
    const struct mm_tile_ctx *c = p;
    const int64_t K = c->k;
    const int64_t o0 = (i % c->n_otiles) * MM_TO;
    const int64_t t0 = (i / c->n_otiles) * MM_TT;
    const int64_t no = c->n_out - o0 < MM_TO ? c->n_out - o0 : MM_TO;
    const int64_t nt = c->m - t0 < MM_TT ? c->m - t0 : MM_TT;
    /* rows o0..o0+no-1 interleaved by 4: wi[(g*K + k)*4 + r] = w[o0+4g+r][k] */
    float *wi = (float *)aligned_alloc(16, sizeof(float) * (size_t)(MM_TO * K));
    for (int64_t g = 0; g < MM_TO / 4; ++g)
        for (int64_t r = 0; r < 4; ++r) {
            const int64_t o = 4 * g + r;
            float *dst = wi + g * K * 4 + r;
            if (o < no) {
                const float *src = c->w + (o0 + o) * K;
                for (int64_t kk = 0; kk < K; ++kk) dst[kk * 4] = src[kk];
            } else {
                for (int64_t kk = 0; kk < K; ++kk) dst[kk * 4] = 0.0f;
            }
        }
    for (int64_t g = 0; 4 * g < no; ++g) {
        const float *wg = wi + g * K * 4;
        for (int64_t tq = 0; tq < nt; tq += 4) {
            const float *xr[4];
            for (int j = 0; j < 4; ++j)
                xr[j] = c->x + (t0 + (tq + j < nt ? tq + j : tq)) * K;
            __m128 a0 = _mm_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
            for (int64_t kk = 0; kk < K; ++kk) {
                const __m128 wv = _mm_load_ps(wg + kk * 4);
                a0 = _mm_add_ps(a0, _mm_mul_ps(_mm_set1_ps(xr[0][kk]), wv));
                a1 = _mm_add_ps(a1, _mm_mul_ps(_mm_set1_ps(xr[1][kk]), wv));
                a2 = _mm_add_ps(a2, _mm_mul_ps(_mm_set1_ps(xr[2][kk]), wv));
                a3 = _mm_add_ps(a3, _mm_mul_ps(_mm_set1_ps(xr[3][kk]), wv));
            }
            float acc[4][4];
            _mm_storeu_ps(acc[0], a0);
            _mm_storeu_ps(acc[1], a1);
            _mm_storeu_ps(acc[2], a2);
            _mm_storeu_ps(acc[3], a3);
            for (int j = 0; j < 4 && tq + j < nt; ++j)
                for (int r = 0; r < 4 && 4 * g + r < no; ++r)
                    c->out[(t0 + tq + j) * c->n_out + o0 + 4 * g + r] = acc[j][r];
        }
    }
    free(wi);
}

void oracle_mul_mat_f32(const float *w, const float *x, float *out, int64_t n_out, int64_t k,
                        int64_t m) {
    if (m >= 4 && k > 0) {
        struct mm_tile_ctx c = {w, x, out, n_out, k, m, (n_out + MM_TO - 1) / MM_TO};
        oracle_pool_for(c.n_otiles * ((m + MM_TT - 1) / MM_TT), mm_tile, &c);
        return;
    }
    struct mm_ctx c = {w, x, out, n_out, k};
    oracle_pool_for(n_out * m, mm_elem, &c);
}

/* ------------------------------------------------------------------ */
/* add / mul / silu (src/backends/cpu_backend.cpp:636-703)             */
/* ------------------------------------------------------------------ */

void oracle_add_f32(const float *a, const float *b, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

void oracle_mul_f32(const float *a, const float *b, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = a[i] * b[i];
}

void oracle_silu_f32(const float *x, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = x[i] / (1.0f + expf(-x[i]));
}

/* ------------------------------------------------------------------ */
/* sample_greedy (src/sampler.cpp:42-65)                               */
/* ------------------------------------------------------------------ */

int32_t oracle_sample_greedy(const float *logits, int64_t n) {
    if (n <= 0) return -1;
    float best = -INFINITY;
    int32_t id = -1;
    for (int64_t i = 0; i < n; ++i) {
        const float s = logits[i];
        if (isnan(s) || s == INFINITY) return -1;
        if (s > best) {
            best = s;
            id = (int32_t)i;
        }
    }
    return id;
}

/* ------------------------------------------------------------------ */
/* One Qwen3 step (src/models/Qwen3.cpp:4-136)                         */
/* ------------------------------------------------------------------ */

int oracle_qwen3_step(const oracle_qwen3_hparams *hp, const oracle_qwen3_layer *layers,
                      const float *token_embd, const float *output_norm, const float *output,
                      const float *theta, const int32_t *tokens, int64_t n_tokens, int64_t n_past,
                      float *const *k_cache, float *const *v_cache, float *logits,
                      int last_row_only) {
    if (!hp || !layers || !token_embd || !output_norm || !output || !theta || !tokens || !logits ||
        n_tokens <= 0 || n_past < 0)
        return -22;
    const int64_t E = hp->n_embd, D = hp->head_dim, Hq = hp->n_head, Hkv = hp->n_head_kv;
    const int64_t Q = Hq * D, KV = Hkv * D, F = hp->n_ff, n = n_tokens;
    if (n_past + n > hp->n_ctx_train) return -22;

    float *x = malloc(sizeof(float) * n * E);        /* inpL */
    float *cur = malloc(sizeof(float) * n * E);
    float *q = malloc(sizeof(float) * n * Q), *q2 = malloc(sizeof(float) * n * Q);
    float *k = malloc(sizeof(float) * n * KV), *k2 = malloc(sizeof(float) * n * KV);
    float *v = malloc(sizeof(float) * n * KV);
    float *att = malloc(sizeof(float) * n * Q);
    float *ffn_inp = malloc(sizeof(float) * n * E);
    float *g = malloc(sizeof(float) * n * F), *u = malloc(sizeof(float) * n * F);
    int32_t *pos = malloc(sizeof(int32_t) * n);
    int rc = 0;
    if (!x || !cur || !q || !q2 || !k || !k2 || !v || !att || !ffn_inp || !g || !u || !pos) {
        rc = -12;
        goto done;
    }
    for (int64_t t = 0; t < n; ++t) pos[t] = (int32_t)(n_past + t);

    rc = oracle_get_rows_f32(token_embd, tokens, x, n, E, hp->n_vocab);
    if (rc) goto done;
    for (int64_t l = 0; l < hp->n_layer; ++l) {
        const oracle_qwen3_layer *L = &layers[l];
        oracle_rms_norm_f32(x, L->attn_norm, cur, n, E, hp->rms_eps);
        oracle_mul_mat_f32(L->wq, cur, q, Q, E, n);
        oracle_mul_mat_f32(L->wk, cur, k, KV, E, n);
        oracle_mul_mat_f32(L->wv, cur, v, KV, E, n);
        oracle_rms_norm_f32(q, L->q_norm, q2, n * Hq, D, hp->rms_eps);
        oracle_rms_norm_f32(k, L->k_norm, k2, n * Hkv, D, hp->rms_eps);
        rc = oracle_rope_neox_f32(q2, pos, theta, hp->n_ctx_train, q, D, Hq, n);
        if (rc) goto done;
        rc = oracle_rope_neox_f32(k2, pos, theta, hp->n_ctx_train, k, D, Hkv, n);
        if (rc) goto done;
        /* append_kv: k after RoPE, v as projected (src/model.cpp:602-625) */
        oracle_cpy(k_cache[l] + n_past * KV, k, sizeof(float) * n * KV);
        oracle_cpy(v_cache[l] + n_past * KV, v, sizeof(float) * n * KV);
        oracle_flash_attn_f32(q, k_cache[l], v_cache[l], att, D, Hq, n, Hkv, n_past + n, n_past);
        oracle_mul_mat_f32(L->wo, att, cur, E, Q, n);
        oracle_add_f32(cur, x, ffn_inp, n * E);
        oracle_rms_norm_f32(ffn_inp, L->ffn_norm, cur, n, E, hp->rms_eps);
        oracle_mul_mat_f32(L->ffn_gate, cur, g, F, E, n);
        oracle_mul_mat_f32(L->ffn_up, cur, u, F, E, n);
        oracle_silu_f32(g, g, n * F);
        oracle_mul_f32(u, g, u, n * F);
        oracle_mul_mat_f32(L->ffn_down, u, cur, E, F, n);
        oracle_add_f32(cur, ffn_inp, x, n * E);
    }
    oracle_rms_norm_f32(x, output_norm, cur, n, E, hp->rms_eps);
    if (last_row_only)
        oracle_mul_mat_f32(output, cur + (n - 1) * E, logits + (n - 1) * hp->n_vocab, hp->n_vocab, E, 1);
    else
        oracle_mul_mat_f32(output, cur, logits, hp->n_vocab, E, n);
done:
    free(x); free(cur); free(q); free(q2); free(k); free(k2); free(v); free(att);
    free(ffn_inp); free(g); free(u); free(pos);
    return rc;
}
