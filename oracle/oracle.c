/*
 * oracle.c — CPU restatement of Infer-LLM's hot-path CPU ops.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the CPU
 * baseline timed by bench.py. Nothing in the product links or loads it.
 *
 * Built with the reference's Release flags (-O3 -DNDEBUG, no -march, no
 * fast-math; benchmarks/cpu/CMakeLists.txt:6-8) plus -ffp-contract=off, which
 * changes nothing on baseline x86-64 (no FMA unit is targeted) and keeps the
 * per-operation float rounding of the reference explicit.
 *
 * Arithmetic is written to round exactly where the reference's C++ rounds:
 * float*float products stay float, `double += float` widens, std::exp /
 * std::sin / std::cos / std::pow on floats are expf / sinf / cosf / powf.
 */
#include "oracle.h"
#include "oracle_pool.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------ */
/* Worker pool (src/backends/cpu_backend.cpp:6-95)                     */
/* ------------------------------------------------------------------ */

typedef void (*task_fn)(int64_t i, void *ctx);

static struct {
    pthread_mutex_t mtx;
    pthread_cond_t cv_start, cv_done;
    pthread_t *threads;
    int n_threads;
    int stop;
    long epoch;
    int n_done;
    task_fn fn;
    void *ctx;
    int64_t n;
    _Atomic int64_t next;
} g_pool = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER,
            PTHREAD_COND_INITIALIZER, NULL, 0, 0, 0, 0, NULL, NULL, 0, 0};

static void *worker_loop(void *arg) {
    (void)arg;
    long last_epoch = 0;
    for (;;) {
        pthread_mutex_lock(&g_pool.mtx);
        while (!g_pool.stop && g_pool.epoch == last_epoch)
            pthread_cond_wait(&g_pool.cv_start, &g_pool.mtx);
        if (g_pool.stop) {
            pthread_mutex_unlock(&g_pool.mtx);
            return NULL;
        }
        last_epoch = g_pool.epoch;
        task_fn fn = g_pool.fn;
        void *ctx = g_pool.ctx;
        int64_t n = g_pool.n;
        pthread_mutex_unlock(&g_pool.mtx);

        for (;;) {
            int64_t i = atomic_fetch_add_explicit(&g_pool.next, 1, memory_order_relaxed);
            if (i >= n) break;
            fn(i, ctx);
        }

        pthread_mutex_lock(&g_pool.mtx);
        if (++g_pool.n_done == g_pool.n_threads) pthread_cond_signal(&g_pool.cv_done);
        pthread_mutex_unlock(&g_pool.mtx);
    }
}

static void pool_shutdown(void) {
    pthread_mutex_lock(&g_pool.mtx);
    g_pool.stop = 1;
    pthread_cond_broadcast(&g_pool.cv_start);
    pthread_mutex_unlock(&g_pool.mtx);
    for (int i = 0; i < g_pool.n_threads; ++i) pthread_join(g_pool.threads[i], NULL);
    free(g_pool.threads);
    g_pool.threads = NULL;
    g_pool.n_threads = 0;
    g_pool.stop = 0;
    g_pool.epoch = 0;
}

int oracle_set_workers(int n_workers) {
    if (n_workers < 1) n_workers = 1;
    if (g_pool.threads) pool_shutdown();
    g_pool.n_threads = n_workers;
    g_pool.threads = (pthread_t *)calloc((size_t)n_workers, sizeof(pthread_t));
    for (int i = 0; i < n_workers; ++i)
        pthread_create(&g_pool.threads[i], NULL, worker_loop, NULL);
    return n_workers > 1 ? n_workers + 1 : 1;
}

int oracle_default_workers(void) {
    const char *env = getenv("INFERLLM_THREADS");
    int n = env ? atoi(env) : 0;
    if (n <= 0) {
        long hw = sysconf(_SC_NPROCESSORS_ONLN);
        if (hw < 1) hw = 1;
        n = (int)((double)hw * 0.5);
    }
    return n < 1 ? 1 : n;
}

static void parallel_for(int64_t n, task_fn fn, void *ctx) {
    if (n <= 0) return;
    if (g_pool.n_threads <= 1) {
        for (int64_t i = 0; i < n; ++i) fn(i, ctx);
        return;
    }
    pthread_mutex_lock(&g_pool.mtx);
    g_pool.fn = fn;
    g_pool.ctx = ctx;
    g_pool.n = n;
    atomic_store_explicit(&g_pool.next, 0, memory_order_relaxed);
    g_pool.n_done = 0;
    g_pool.epoch++;
    pthread_cond_broadcast(&g_pool.cv_start);
    pthread_mutex_unlock(&g_pool.mtx);

    for (;;) {
        int64_t i = atomic_fetch_add_explicit(&g_pool.next, 1, memory_order_relaxed);
        if (i >= n) break;
        fn(i, ctx);
    }

    pthread_mutex_lock(&g_pool.mtx);
    while (g_pool.n_done != g_pool.n_threads) pthread_cond_wait(&g_pool.cv_done, &g_pool.mtx);
    pthread_mutex_unlock(&g_pool.mtx);
}

void oracle_pool_for(int64_t n, void (*fn)(int64_t i, void *ctx), void *ctx) {
    parallel_for(n, fn, ctx);
}

/* ------------------------------------------------------------------ */
/* RMS norm (src/backends/cpu_backend.cpp:335-382)                     */
/* ------------------------------------------------------------------ */

struct rms_ctx {
    const float *x, *w;
    float *out;
    int64_t dim;
    float eps;
};

static void rms_row(int64_t i, void *p) {
    const struct rms_ctx *c = (const struct rms_ctx *)p;
    const float *x = c->x + i * c->dim;
    float *o = c->out + i * c->dim;
    double sum = 0; /* cpu_backend.cpp:369 — float squares summed in double */
    for (int64_t d = 0; d < c->dim; ++d) {
        float sq = x[d] * x[d];
        sum += sq;
    }
    /* cpu_backend.cpp:376: 1.0f / std::sqrt(double) in double, then float */
    float scale = (float)(1.0 / sqrt(sum / (double)c->dim + (double)c->eps));
    for (int64_t d = 0; d < c->dim; ++d) {
        float t = x[d] * scale;
        o[d] = t * c->w[d];
    }
}

void oracle_rms_norm_f32(const float *x, const float *w, float *out, int64_t rows,
                         int64_t dim, float eps) {
    struct rms_ctx c = {x, w, out, dim, eps};
    parallel_for(rows, rms_row, &c);
}

/* ------------------------------------------------------------------ */
/* RoPE angle table (src/graph.cpp:92-135)                             */
/* ------------------------------------------------------------------ */

void oracle_rope_theta_table(float theta_base, uint32_t head_dim, uint32_t n_ctx, float *out) {
    const uint32_t half = head_dim / 2;
    double *freq = (double *)malloc(sizeof(double) * (half ? half : 1));
    for (uint32_t i = 0; i < half; ++i) {
        /* graph.cpp:121: 2.0f*i/head_dim is float; std::pow(float,float) is
         * powf; 1.0f/powf is float; stored widened to double. */
        float e = 2.0f * (float)i;
        e = e / (float)head_dim;
        float f = 1.0f / powf(theta_base, e);
        freq[i] = (double)f;
    }
    for (uint32_t pos = 0; pos < n_ctx; ++pos) {
        float *row = out + (size_t)pos * half;
        for (uint32_t i = 0; i < half; ++i) row[i] = (float)((double)pos * freq[i]);
    }
    free(freq);
}

/* ------------------------------------------------------------------ */
/* RoPE, NeoX half split (src/backends/cpu_backend.cpp:443-523)        */
/* ------------------------------------------------------------------ */

struct rope_ctx {
    const float *x;
    float *out;
    const float *sin_c, *cos_c;
    int64_t head_dim, n_heads;
};

static void rope_row(int64_t i, void *p) {
    const struct rope_ctx *c = (const struct rope_ctx *)p;
    const int64_t n_pairs = c->head_dim / 2;
    const int64_t token = i / c->n_heads;
    const float *x = c->x + i * c->head_dim;
    float *o = c->out + i * c->head_dim;
    const float *sn = c->sin_c + token * n_pairs;
    const float *cs = c->cos_c + token * n_pairs;
    for (int64_t j = 0; j < n_pairs; ++j) {
        const float x0 = x[j];
        const float x1 = x[n_pairs + j];
        const float cj = cs[j], sj = sn[j];
        /* cpu_backend.cpp:518-519 */
        const float a = x0 * cj, b = x1 * sj;
        const float e = x0 * sj, f = x1 * cj;
        o[j] = a - b;
        o[n_pairs + j] = e + f;
    }
}

int oracle_rope_neox_f32(const float *x, const int32_t *pos, const float *theta, int64_t n_ctx,
                         float *out, int64_t head_dim, int64_t n_heads, int64_t n_tokens) {
    const int64_t n_pairs = head_dim / 2;
    for (int64_t t = 0; t < n_tokens; ++t)
        if (pos[t] < 0 || pos[t] >= n_ctx) return -22;
    float *sin_c = (float *)malloc(sizeof(float) * (size_t)(n_tokens * n_pairs + 1));
    float *cos_c = (float *)malloc(sizeof(float) * (size_t)(n_tokens * n_pairs + 1));
    /* cpu_backend.cpp:472-487: sin/cos per token on the calling thread */
    for (int64_t t = 0; t < n_tokens; ++t) {
        const float *ang = theta + (int64_t)pos[t] * n_pairs;
        for (int64_t j = 0; j < n_pairs; ++j) {
            sin_c[t * n_pairs + j] = sinf(ang[j]);
            cos_c[t * n_pairs + j] = cosf(ang[j]);
        }
    }
    struct rope_ctx c = {x, out, sin_c, cos_c, head_dim, n_heads};
    parallel_for(n_heads * n_tokens, rope_row, &c);
    free(sin_c);
    free(cos_c);
    return 0;
}

/* ------------------------------------------------------------------ */
/* GQA attention (src/backends/cpu_backend.cpp:525-634)                */
/* ------------------------------------------------------------------ */

struct attn_ctx {
    const float *q, *k, *v;
    float *out;
    int64_t D, Hq, Hkv, n_kv, n_past, group;
};

static void attn_row(int64_t i, void *p) {
    const struct attn_ctx *c = (const struct attn_ctx *)p;
    const int64_t D = c->D;
    const int64_t q_token = i / c->Hq;
    const int64_t q_head = i % c->Hq;
    const int64_t kv_head = q_head / c->group; /* cpu_backend.cpp:563 */
    const float *qs = c->q + i * D;
    float *o = c->out + i * D;
    float *scores = (float *)malloc(sizeof(float) * (size_t)(c->n_kv > 0 ? c->n_kv : 1));
    const float scale = 1.0f / sqrtf((float)D); /* cpu_backend.cpp:575 */
    for (int64_t kt = 0; kt < c->n_kv; ++kt) {
        if (kt > c->n_past + q_token) { /* cpu_backend.cpp:578 */
            scores[kt] = -INFINITY;
            continue;
        }
        const float *ks = c->k + (kt * c->Hkv + kv_head) * D;
        float dot = 0.0f;
        for (int64_t d = 0; d < D; ++d) {
            float pr = qs[d] * ks[d];
            dot += pr;
        }
        scores[kt] = dot * scale;
    }
    /* std::max_element: first maximum (only its value is used) */
    float mx = c->n_kv > 0 ? scores[0] : 0.0f;
    for (int64_t kt = 1; kt < c->n_kv; ++kt)
        if (mx < scores[kt]) mx = scores[kt];
    float sum = 0.0f;
    for (int64_t kt = 0; kt < c->n_kv; ++kt) {
        scores[kt] = expf(scores[kt] - mx);
        sum += scores[kt];
    }
    for (int64_t kt = 0; kt < c->n_kv; ++kt) scores[kt] /= sum;
    for (int64_t d = 0; d < D; ++d) o[d] = 0.0f;
    for (int64_t kt = 0; kt < c->n_kv; ++kt) { /* cpu_backend.cpp:619-631 */
        const float *vs = c->v + (kt * c->Hkv + kv_head) * D;
        const float wgt = scores[kt];
        for (int64_t d = 0; d < D; ++d) {
            float pr = wgt * vs[d];
            o[d] += pr;
        }
    }
    free(scores);
}

void oracle_flash_attn_f32(const float *q, const float *k, const float *v, float *out,
                           int64_t head_dim, int64_t n_head, int64_t n_q, int64_t n_head_kv,
                           int64_t n_kv, int64_t n_past) {
    struct attn_ctx c = {q, k, v, out, head_dim, n_head, n_head_kv, n_kv, n_past,
                         n_head / n_head_kv};
    parallel_for(n_head * n_q, attn_row, &c);
}

/* ------------------------------------------------------------------ */
/* KV append (src/backends/cpu_backend.cpp:705-742)                    */
/* ------------------------------------------------------------------ */

int oracle_cpy(void *dst, const void *src, size_t bytes) {
    if (!dst || !src) return -22;
    memcpy(dst, src, bytes);
    return 0;
}

void oracle_decode_append_attn_f32(const float *q, const float *k_new, const float *v_new,
                                   float *k_cache, float *v_cache, float *out, int64_t head_dim,
                                   int64_t n_head, int64_t n_head_kv, int64_t n_past) {
    const size_t row = (size_t)(n_head_kv * head_dim);
    oracle_cpy(k_cache + (size_t)n_past * row, k_new, row * sizeof(float));
    oracle_cpy(v_cache + (size_t)n_past * row, v_new, row * sizeof(float));
    oracle_flash_attn_f32(q, k_cache, v_cache, out, head_dim, n_head, 1, n_head_kv, n_past + 1,
                          n_past);
}
