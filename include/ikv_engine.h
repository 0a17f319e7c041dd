/*
 * ikv_engine.h — C-ABI of the engine level: a Qwen3 model on the HIP backend
 * and the benchmark runner's greedy generation loop.
 *
 * This is the caller of the KV-cache path at model level. It stands in for
 * what the reference's benchmark drives through C++ (ModelBase::load_model /
 * load_weight, src/model.cpp:60-311; Runner::evaluate and run,
 * benchmarks/cpu/bench.cpp:130-281), so that tests and bench.py can run a
 * whole model from Python: the graph is Qwen3Model::build_graph
 * (src/models/Qwen3.cpp:4-136), executed by the engine's Scheduler on
 * HIPBackend, KV cache in HBM through KVCacheManager / ContiguousKVStrategy /
 * NaiveKVStorage.
 *
 * Unlike include/ikv.h, these entry points allocate: the model's weights,
 * KV caches and activation arena live in device memory until
 * ikv_qwen3_destroy. Return values: 0, or a negative errno.
 */
#ifndef IKV_ENGINE_H
#define IKV_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Hyperparameters (the GGUF keys of src/model.cpp:60-163). */
typedef struct ikv_qwen3_config {
    uint32_t n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, n_ctx_train;
    float rope_theta, rms_norm_eps;
    /* 0: the logits use the token embedding (tied, as when a GGUF file has
     * no "output.weight"); 1: a separate "output.weight" [n_vocab][n_embd]
     * projects them (src/model.cpp:203-210). */
    uint32_t untied_output;
} ikv_qwen3_config;

/* TTFT and TPOT as benchmarks/cpu/bench.cpp:239-281 defines them:
 * ttft = first sampled token - start, tpot = (last - first) / (n_gen - 1);
 * build / execute / sample: graph construction, scheduling + enqueue, and
 * device argmax + token read-back (which waits for the step's kernels),
 * summed over steps. */
typedef struct ikv_qwen3_timing {
    double ttft_s, tpot_s, wall_s, build_s, execute_s, sample_s;
} ikv_qwen3_timing;

typedef struct ikv_qwen3 ikv_qwen3;

/* Creates the model on HIP device `device` with weights allocated (not yet
 * initialised) and a KV cache of max_ctx tokens per layer. */
int ikv_qwen3_create(const ikv_qwen3_config *cfg, int device, int64_t max_ctx, ikv_qwen3 **out);
/* The same with a paged KV cache (KVCacheConfig::block_tokens > 0,
 * include/kvcache/kvutil.hpp:43 of the reference): per layer a pool of
 * pool_blocks blocks of block_tokens tokens (a positive multiple of 64;
 * pool_blocks 0 = enough for one max_ctx sequence), blocks taken as a
 * sequence grows and returned when the next generate() starts a new one. */
int ikv_qwen3_create_paged(const ikv_qwen3_config *cfg, int device, int64_t max_ctx,
                           int64_t block_tokens, int64_t pool_blocks, ikv_qwen3 **out);
/* The same with the KV cache in the HBM <-> host offload tier (the
 * reference's OffloadKVStorage, include/kvcache/KVStorages/
 * offloadKVStorage.hpp): every layer's cache has a pinned host copy, and at
 * most hbm_bytes of them are resident in HBM; a layer is uploaded when a step
 * acquires it, and the least recently used layer is written back and
 * dropped to make room. Only token rows that hold data move: an upload copies
 * the rows the host copy holds (none for a new sequence), a write-back the
 * rows written since the upload. Tokens are those of the all-HBM cache. */
int ikv_qwen3_create_offload(const ikv_qwen3_config *cfg, int device, int64_t max_ctx,
                             uint64_t hbm_bytes, ikv_qwen3 **out);

/* Page-ins (host -> HBM), page-outs (write-backs), evictions and bytes moved
 * by an offloaded cache since creation (zeros for the other caches). */
typedef struct ikv_qwen3_kv_counters {
    uint64_t page_ins, page_outs, evictions, bytes_in, bytes_out;
} ikv_qwen3_kv_counters;
int ikv_qwen3_kv_stats(const ikv_qwen3 *m, ikv_qwen3_kv_counters *out);

/* Weight tensors by GGUF name (ModelBase::load_weight, src/model.cpp:
 * 164-311): "token_embd.weight", "blk.<i>.attn_q.weight", ...,
 * "output_norm.weight", then "output.weight" when the config is untied
 * (otherwise the output projection is the tied token embedding).
 * Index order is the synthetic initialiser's draw order. */
int ikv_qwen3_tensor_count(const ikv_qwen3 *m);
const char *ikv_qwen3_tensor_name(const ikv_qwen3 *m, int index);
/* Element count of a named tensor, or 0 when the name is unknown. */
size_t ikv_qwen3_tensor_size(const ikv_qwen3 *m, const char *name);
int ikv_qwen3_set_tensor(ikv_qwen3 *m, const char *name, const float *host, size_t count);
/* Random-init weights of the benchmark configurations: every matrix
 * N(0, std^2) drawn from one ikv_synth_normal_f32 stream in tensor order,
 * every norm weight 1.0. */
int ikv_qwen3_init_synthetic(ikv_qwen3 *m, uint64_t seed, double std, int threads);

/* Greedy generation: prompt, then n_gen tokens (the first from the prompt's
 * last logits row, each next one from feeding back the previous token).
 * tokens_out holds n_gen ids. Each call starts a new sequence. */
int ikv_qwen3_generate(ikv_qwen3 *m, const int32_t *prompt, int64_t n_prompt, int64_t n_gen,
                       int32_t *tokens_out, ikv_qwen3_timing *timing);

/* n_seq (1..4) sequences of one cache decoded in turn: every prompt's
 * prefill, then n_gen - 1 rounds of one token per sequence. prompts is
 * [n_seq][n_prompt], tokens_out [n_seq][n_gen]; each sequence's tokens are
 * those ikv_qwen3_generate gives its prompt alone. On an offloaded cache
 * whose HBM budget holds fewer layers than the sequences together, each
 * turn pages the next sequence's layers in (and the last one's written
 * rows out): the reference's multi-sequence offload tier
 * (include/kvcache/KVStorages/offloadKVStorage.hpp:57-179) under load.
 * timing->tpot_s is per round of all sequences; ttft_s ends with the first
 * round. */
int ikv_qwen3_generate_interleaved(ikv_qwen3 *m, const int32_t *prompts, int64_t n_seq,
                                   int64_t n_prompt, int64_t n_gen, int32_t *tokens_out,
                                   ikv_qwen3_timing *timing);

/* Fusions taken and kernel launches in the last step. */
typedef struct ikv_qwen3_stats {
    int launches, fused_norm_rope, fused_append_decode, fused_swiglu, fused_residual, fused_qkv,
        fused_norm_mm, fused_rope_decode;
    int fused_qkv_decode; /* decodes run inside their q/k/v launch (short contexts) */
    int fused_append;     /* cache appends written by their producer (prefill K and V) */
    /* over the last ikv_qwen3_generate: decode steps captured as a HIP graph,
     * and decode steps launched from one (captured ones included) */
    int step_captures, step_replays;
} ikv_qwen3_stats;
int ikv_qwen3_last_stats(const ikv_qwen3 *m, ikv_qwen3_stats *out);
/* 0 disables the HIP backend's graph fusions (every node its own launch). */
int ikv_qwen3_set_fusion(ikv_qwen3 *m, int on);
/* 1 (the default): the decode steps of ikv_qwen3_generate are captured as a
 * HIP graph once per range of contexts the decode's split plan allows (up to
 * 256 tokens) and replayed, the position advancing on the device, so that a
 * step costs the host one graph launch and one sampler launch; the tokens are
 * those of the eager steps. Taken with a contiguous or paged cache (not the
 * offload tier) and fusions on.
 * 0: every step is built and launched from the host (the reference's way,
 * src/model.cpp:164-311). No counterpart in the reference. */
int ikv_qwen3_set_step_replay(ikv_qwen3 *m, int on);

/* Keep, during each later ikv_qwen3_generate, the logits the greedy sampler
 * reads at each of the n_steps steps (step 0 samples from the prompt's last
 * logits row, step i > 0 from decode step i), for checks at logit level; the
 * reference's sampler reads the same row (src/sampler.cpp:5-35). The rows
 * are copied on the device stream after their step, outside any captured
 * graph, into a device buffer of n_steps x n_vocab floats that this call
 * allocates (n_steps = 0 frees it and keeps none). ikv_qwen3_captured_logits
 * copies them to host memory in the order of `steps`; count must be n_steps
 * x n_vocab. No counterpart in the reference. */
int ikv_qwen3_capture_logits(ikv_qwen3 *m, const int64_t *steps, int64_t n_steps);
int ikv_qwen3_captured_logits(const ikv_qwen3 *m, float *host, size_t count);

void ikv_qwen3_destroy(ikv_qwen3 *m);

#ifdef __cplusplus
}
#endif

#endif /* IKV_ENGINE_H */
