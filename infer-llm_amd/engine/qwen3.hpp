// qwen3.hpp — the Qwen3 model graph and a generation runner on the HIP
// backend: the caller side of the KV-cache path at model level.
//
// Qwen3Model restates Qwen3Model::build_graph (reference
// src/models/Qwen3.cpp:4-136): embedding -> per layer [RMSNorm -> q/k/v
// projections -> attention slice (reshape, qk-RMSNorm, RoPE, KV append,
// flash attention) -> o_proj -> residual -> RMSNorm -> gate/up -> SiLU ->
// mul -> down -> residual] -> RMSNorm -> logits. Weights carry the GGUF names
// of ModelBase::load_weight (src/model.cpp:164-311) and live in one HBM
// arena of the backend's WEIGHTS pool; the output projection is the tied
// token embedding.
//
// Qwen3Runner restates the benchmark Runner (benchmarks/cpu/bench.cpp:
// 130-219): per step reserve -> build graph -> execute -> sample -> commit,
// with the reference's TTFT / TPOT definitions (benchmarks/cpu/bench.cpp:
// 239-281). Sampling is greedy on the device (ikv_argmax_f32) into a device
// token slot that the next step's embedding reads directly, and positions
// come from a resident device table, so no step waits for the previous one
// on the host: the host builds and enqueues step i+1 while the GPU runs step
// i, then reads back token i, which the sampler also writes to pinned host
// memory (one event per slot). A token is "ready" when the host has it, as
// in the reference's loop.
#pragma once

#include <chrono>
#include <cstdint>
#include <memory>
#include <string>
#include <system_error>
#include <unordered_map>
#include <vector>

#include "expected.hpp"
#include "graph.hpp"
#include "hip_backend.hpp"
#include "kvcache/kvcache_manager.hpp"
#include "kvcache/offload_storage.hpp"
#include "scheduler.hpp"

struct Qwen3Hparams {
  uint32_t n_layer = 28;
  uint32_t n_embd = 1024;
  uint32_t n_head = 16;
  uint32_t n_head_kv = 8;
  uint32_t head_dim = 128;
  uint32_t n_ff = 3072;
  uint32_t n_vocab = 151936;
  uint32_t n_ctx_train = 40960;
  float rope_theta = 1e6f;
  float rms_norm_eps = 1e-6f;
  // A separate output projection "output.weight"; false ties the logits to
  // the token embedding (src/model.cpp:203-210).
  bool untied_output = false;
};

struct Qwen3LayerWeights {
  Tensor *attn_norm = nullptr, *wq = nullptr, *wk = nullptr, *wv = nullptr;
  Tensor *attn_q_norm = nullptr, *attn_k_norm = nullptr, *wo = nullptr, *ffn_norm = nullptr;
  Tensor *ffn_gate = nullptr, *ffn_up = nullptr, *ffn_down = nullptr;
};

class Qwen3Model {
 public:
  explicit Qwen3Model(const Qwen3Hparams &hp);
  ~Qwen3Model();
  Qwen3Model(const Qwen3Model &) = delete;
  Qwen3Model &operator=(const Qwen3Model &) = delete;

  // One WEIGHTS allocation for every tensor (256-byte aligned each).
  infer::expected<void, std::error_code> alloc_weights(Backend *backend);
  // Names in the order the synthetic initialiser draws them.
  std::vector<std::string> tensor_names() const;
  Tensor *find(const std::string &name) const;
  // Host -> device copy of one weight (count floats).
  infer::expected<void, std::error_code> set_tensor(const std::string &name, const float *host,
                                                    size_t count);
  // Random-init weights of the benchmark configurations: every matrix
  // N(0, std^2) from one counter-based stream (ikv_synth_normal_f32) in
  // tensor_names() order, norm weights 1.0.
  infer::expected<void, std::error_code> init_synthetic(uint64_t seed, double std, int threads);

  infer::expected<Graph, std::error_code> build_graph(GraphContext &ctx) const;
  const Qwen3Hparams &hparams() const { return _hp; }
  size_t weight_bytes() const { return _arena_bytes; }

 private:
  Tensor *make(const std::string &name, std::initializer_list<int64_t> shape);

  Qwen3Hparams _hp;
  Backend *_backend = nullptr;
  void *_arena = nullptr;
  size_t _arena_bytes = 0;
  std::vector<std::unique_ptr<Tensor>> _tensors;
  std::unordered_map<std::string, Tensor *> _map;
  Tensor *_token_embd = nullptr, *_output_norm = nullptr;
  Tensor *_output = nullptr;  // the token embedding when tied
  std::vector<Qwen3LayerWeights> _layers;
};

// How the runner keeps its KV cache.
//   default            one contiguous HBM cache per layer (ContiguousKVStrategy
//                      over NaiveKVStorage)
//   block_tokens > 0   paged: PagedKVStrategy over a BlockPoolKVStorage of
//                      pool_blocks blocks per layer (0 = one sequence's worth)
//   offload_bytes > 0  contiguous caches in an OffloadKVStorage: pinned host
//                      copies, at most offload_bytes of them resident in HBM
//                      (LRU eviction with write-back)
struct KVOptions {
  size_t block_tokens = 0;
  size_t pool_blocks = 0;
  size_t offload_bytes = 0;
};

struct GenerationTiming {
  double ttft_s = 0;      // first sampled token - start
  double tpot_s = 0;      // (last - first) / (n_gen - 1)
  double wall_s = 0;
  double build_s = 0;     // graph construction, summed over steps
  double execute_s = 0;   // scheduling + enqueue, summed
  double sample_s = 0;    // device argmax + token read-back (waits for the step), summed
};

class Qwen3Runner {
 public:
  Qwen3Runner(Qwen3Model &model, HIPBackend &backend, size_t capacity, KVOptions kv = {});
  ~Qwen3Runner();
  infer::expected<void, std::error_code> init();
  // prompt, then n_gen greedy tokens (the first from the prompt's last
  // logits row); tokens_out receives the n_gen sampled ids.
  infer::expected<void, std::error_code> generate(const std::vector<int32_t> &prompt, size_t n_gen,
                                                  std::vector<int32_t> &tokens_out,
                                                  GenerationTiming &timing);
  // Up to kMaxInterleaved sequences decoded in turn, one step each per
  // round: prefill of every prompt, then n_gen - 1 rounds of one token per
  // sequence. Each sequence's tokens are those generate() gives it alone; on
  // an offloaded cache whose HBM budget holds fewer layers than the
  // sequences have, every turn pages the next sequence's layers in.
  // Timing: ttft = first round done - start, tpot = (last round - first
  // round) / (n_gen - 1), per round of all sequences.
  static constexpr int kMaxInterleaved = 4;
  infer::expected<void, std::error_code> generate_interleaved(
      const std::vector<std::vector<int32_t>> &prompts, size_t n_gen,
      std::vector<std::vector<int32_t>> &tokens_out, GenerationTiming &timing);
  // Page-in / write-back counts of an offloaded cache (zeros otherwise).
  OffloadStats offload_stats() const;
  // Decode steps of generate() replayed from a captured HIP graph (default
  // on). Taken with a contiguous or paged cache and the backend's fusions
  // on; the offload tier, and any step whose capture fails, launch eagerly.
  void set_step_replay(bool on) { _replay = on; }
  struct ReplayStats {
    int captures = 0;  // decode steps captured (each then replayed)
    int replays = 0;   // decode steps launched as a graph (captured ones included)
  };
  // Over the last generate() call.
  ReplayStats replay_stats() const { return _replay_stats; }
  // Keep, during each later generate(), the logits row the sampler reads at
  // each of `steps` (step 0 samples from the prompt's last row; step i > 0
  // from decode step i), copied on the stream after the step (outside any
  // captured graph); empty: keep none. captured_logits copies them, in the
  // order of `steps`, n_vocab floats each.
  infer::expected<void, std::error_code> set_logit_capture(const std::vector<int64_t> &steps);
  infer::expected<void, std::error_code> captured_logits(float *host, size_t count) const;

 private:
  // Enqueues one step of sequence _seq: its input is the host prompt, or
  // (host_tokens NULL) the token in device slot in_slot; its greedy token
  // lands in device slot out_slot and, once event host_slot (default:
  // out_slot) has fired, in _token_host[host_slot].
  infer::expected<void, std::error_code> enqueue_step(const int32_t *host_tokens, int64_t n,
                                                      int in_slot, int out_slot,
                                                      GenerationTiming &timing, int host_slot = -1);
  // One decode step of _seq from the captured graph, captured first when
  // the context is outside the contexts it serves: the input token is in
  // device slot kReplaySlot and the sampled token goes there and to host
  // slot host_slot. not_supported: no graph could be made for this step
  // (nothing was enqueued; launch it eagerly).
  infer::expected<void, std::error_code> replay_step(int host_slot, GenerationTiming &timing);
  infer::expected<void, std::error_code> capture_step(int64_t n_past);
  void drop_step_graph();
  infer::expected<int32_t, std::error_code> collect(int slot);
  // Enqueues the copy of `row` if the step being enqueued is one to keep.
  bool keep_logits(const float *row, int64_t vocab, hipStream_t s);

  Qwen3Model &_model;
  HIPBackend &_backend;
  size_t _capacity;
  KVOptions _kv_opt;
  std::unique_ptr<Backend> _host;  // the host tier of an offloaded cache
  std::unique_ptr<KVCacheManager> _kv;
  std::unique_ptr<Scheduler> _sched;
  std::unique_ptr<GraphContext> _ctx;
  SequenceId _seq = kInvalidSequenceId;
  Tensor *_tokens = nullptr, *_pos = nullptr;
  std::vector<int32_t> _input;
  static constexpr int kSlots = 2 * kMaxInterleaved;
  static constexpr int kReplaySlot = kSlots;  // the device token slot of replayed steps
  int32_t *_token_dev = nullptr;    // [kSlots + 1] sampled-token slots, two per sequence
  int32_t *_token_host = nullptr;   // [kSlots] pinned read-back slots
  int32_t *_token_host_dev = nullptr;  // the same slots as the device addresses them
  int32_t *_positions_dev = nullptr;  // [capacity]: 0, 1, 2, ...
  void *_argmax_ws = nullptr;         // the multi-workgroup sampler's workspace (zeroed once)
  hipEvent_t _ready[kSlots] = {};
  // the captured decode step
  bool _replay = true;
  hipGraphExec_t _step_exec = nullptr;
  int64_t _step_lo = 0, _step_hi = 0;   // the contexts (n_past + 1) it serves
  const float *_step_logits = nullptr;  // its logits row (in the scheduler's arena)
  int64_t _step_vocab = 0;
  int32_t *_pos_state = nullptr;        // device: the position the captured step reads
  ReplayStats _replay_stats;
  // logit capture: the steps, their rows on the device, the step enqueued
  std::vector<int64_t> _logit_steps;
  float *_logit_dev = nullptr;
  size_t _cur_step = 0;
};
