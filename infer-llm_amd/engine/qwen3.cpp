#include "qwen3.hpp"

#include <algorithm>
#include <cstring>

#include "../../include/ikv.h"
#include "../../include/ikv_model.h"
#include "kvcache/kvstorage.hpp"
#include "kvcache/kvstrategy.hpp"
#include "op_factory.hpp"

namespace {

size_t align256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

bool is_norm(const std::string &name) { return name.find("norm") != std::string::npos; }

}  // namespace

// ---------------------------------------------------------------------------
// model

Qwen3Model::Qwen3Model(const Qwen3Hparams &hp) : _hp(hp) {
  const int64_t E = hp.n_embd, D = hp.head_dim, Q = int64_t(hp.n_head) * D,
                KV = int64_t(hp.n_head_kv) * D, F = hp.n_ff;
  _token_embd = make("token_embd.weight", {E, hp.n_vocab});
  _layers.resize(hp.n_layer);
  for (uint32_t l = 0; l < hp.n_layer; ++l) {
    const std::string p = "blk." + std::to_string(l) + ".";
    Qwen3LayerWeights &L = _layers[l];
    L.attn_norm = make(p + "attn_norm.weight", {E});
    L.wq = make(p + "attn_q.weight", {E, Q});
    L.wk = make(p + "attn_k.weight", {E, KV});
    L.wv = make(p + "attn_v.weight", {E, KV});
    L.attn_q_norm = make(p + "attn_q_norm.weight", {D});
    L.attn_k_norm = make(p + "attn_k_norm.weight", {D});
    L.wo = make(p + "attn_output.weight", {Q, E});
    L.ffn_norm = make(p + "ffn_norm.weight", {E});
    L.ffn_gate = make(p + "ffn_gate.weight", {E, F});
    L.ffn_up = make(p + "ffn_up.weight", {E, F});
    L.ffn_down = make(p + "ffn_down.weight", {F, E});
  }
  _output_norm = make("output_norm.weight", {E});
  // last, so that a tied model's synthetic draw order does not depend on it
  _output = hp.untied_output ? make("output.weight", {E, hp.n_vocab}) : _token_embd;
}

Qwen3Model::~Qwen3Model() {
  if (_arena && _backend) _backend->free(BufferKind::WEIGHTS, _arena);
}

Tensor *Qwen3Model::make(const std::string &name, std::initializer_list<int64_t> shape) {
  auto t = std::make_unique<Tensor>(name, GGML_TYPE_F32, shape);
  t->tensorRole = TensorRole::TENSOR_ROLE_WEIGHT;
  Tensor *raw = t.get();
  _map.emplace(name, raw);
  _tensors.push_back(std::move(t));
  return raw;
}

std::vector<std::string> Qwen3Model::tensor_names() const {
  std::vector<std::string> names;
  for (const auto &t : _tensors) names.push_back(t->name);
  return names;
}

Tensor *Qwen3Model::find(const std::string &name) const {
  auto it = _map.find(name);
  return it == _map.end() ? nullptr : it->second;
}

infer::expected<void, std::error_code> Qwen3Model::alloc_weights(Backend *backend) {
  if (!backend || _arena) return infer::fail(std::errc::invalid_argument);
  size_t total = 0;
  for (const auto &t : _tensors) total += align256(t->byte_size());
  auto mem = backend->alloc(BufferKind::WEIGHTS, total);
  if (!mem) return infer::unexpected(mem.error());
  _backend = backend;
  _arena = *mem;
  _arena_bytes = total;
  char *cursor = static_cast<char *>(_arena);
  for (const auto &t : _tensors) {
    t->data = cursor;
    t->backend = backend;
    t->device = backend->device_type();
    cursor += align256(t->byte_size());
  }
  return {};
}

infer::expected<void, std::error_code> Qwen3Model::set_tensor(const std::string &name,
                                                              const float *host, size_t count) {
  Tensor *t = find(name);
  if (!t || !t->data || !host) return infer::fail(std::errc::invalid_argument);
  if (count != t->element_count()) return infer::fail(std::errc::invalid_argument);
  return _backend->copy_tensor_set(t, host, 0, count * sizeof(float));
}

infer::expected<void, std::error_code> Qwen3Model::init_synthetic(uint64_t seed, double std,
                                                                  int threads) {
  if (!_arena) return infer::fail(std::errc::invalid_argument);
  size_t largest = 0;
  for (const auto &t : _tensors) largest = std::max(largest, t->element_count());
  std::vector<float> host(largest);
  uint64_t offset = 0;
  for (const auto &t : _tensors) {
    const size_t n = t->element_count();
    if (is_norm(t->name)) {
      std::fill(host.begin(), host.begin() + n, 1.0f);
    } else {
      if (ikv_synth_normal_f32(seed, offset, n, std, host.data(), threads) != 0)
        return infer::fail(std::errc::invalid_argument);
      offset += n;
    }
    if (auto r = _backend->copy_tensor_set(t.get(), host.data(), 0, n * sizeof(float)); !r) return r;
  }
  return {};
}

infer::expected<Graph, std::error_code> Qwen3Model::build_graph(GraphContext &ctx) const {
  Graph g;
  Tensor *input_token = ctx.get_input_tokens();
  Tensor *inp_pos = ctx.get_input_pos();
  if (!input_token || !inp_pos) return infer::fail(std::errc::invalid_argument);
  g.mark_input(input_token);
  g.mark_input(inp_pos);
  const int64_t n_tokens = inp_pos->dims[0];

  AttentionSliceParams sp;
  sp.n_head = _hp.n_head;
  sp.n_head_kv = _hp.n_head_kv;
  sp.head_dim = _hp.head_dim;
  sp.rms_norm_eps = _hp.rms_norm_eps;
  sp.rope_theta = _hp.rope_theta;
  sp.n_ctx_train = _hp.n_ctx_train;
  const float eps = _hp.rms_norm_eps;

  Tensor *inpL = OpFactory::embedding(g, _token_embd, input_token);
  for (uint32_t i = 0; i < _hp.n_layer; ++i) {
    const Qwen3LayerWeights &L = _layers[i];
    const std::string s = std::to_string(i);
    Tensor *inpSA = inpL;
    Tensor *cur = OpFactory::rms_norm(g, inpL, L.attn_norm, eps, "attn_norm_" + s);
    Tensor *q = OpFactory::mul_mat(g, L.wq, cur, "q_proj" + s);
    Tensor *k = OpFactory::mul_mat(g, L.wk, cur, "k_proj" + s);
    Tensor *v = OpFactory::mul_mat(g, L.wv, cur, "v_proj" + s);
    auto attn = build_attention_slice(g, ctx, q, k, v, L.attn_q_norm, L.attn_k_norm, i, sp);
    if (!attn) return infer::unexpected(attn.error());
    cur = OpFactory::reshape(g, *attn, {int64_t(_hp.head_dim) * _hp.n_head, n_tokens, 1, 1},
                             "attn_reshape_" + s);
    cur = OpFactory::mul_mat(g, L.wo, cur, "o_proj" + s);
    Tensor *ffn_inp = OpFactory::add(g, cur, inpSA, "ffn_inp_" + s);
    cur = OpFactory::rms_norm(g, ffn_inp, L.ffn_norm, eps, "ffn_norm_" + s);
    Tensor *gate = OpFactory::mul_mat(g, L.ffn_gate, cur, "ffn_gate_" + s);
    Tensor *up = OpFactory::mul_mat(g, L.ffn_up, cur, "ffn_up_" + s);
    Tensor *gate_silu = OpFactory::silu(g, gate, "ffn_gate_silu_" + s);
    Tensor *inter = OpFactory::mul(g, up, gate_silu, "ffn_inter_" + s);
    Tensor *ffn_out = OpFactory::mul_mat(g, L.ffn_down, inter, "ffn_out_" + s);
    inpL = OpFactory::add(g, ffn_out, ffn_inp, "result_out_" + s);
  }
  // The sampler reads only the last token's logits (reference
  // src/sampler.cpp:5-35 reads row n_tokens - 1 of the full [vocab, n_tokens]
  // result). The output norm and the projection act on each row alone, so
  // computing them for the last row gives that row's values without the
  // other n_tokens - 1 rows (a [vocab x n_embd] x [n_embd x n_tokens] GEMM at
  // prefill).
  Tensor *last = n_tokens > 1 ? OpFactory::view_rows(g, inpL, n_tokens - 1, 1, "result_last") : inpL;
  Tensor *final_norm = OpFactory::rms_norm(g, last, _output_norm, eps, "result_norm");
  Tensor *logits = OpFactory::mul_mat(g, _output, final_norm, "logits");
  g.mark_output(logits);
  return g;
}

// ---------------------------------------------------------------------------
// runner

Qwen3Runner::Qwen3Runner(Qwen3Model &model, HIPBackend &backend, size_t capacity, KVOptions kv)
    : _model(model), _backend(backend), _capacity(capacity), _kv_opt(kv) {}

Qwen3Runner::~Qwen3Runner() {
  (void)_backend.synchronize();
  drop_step_graph();
  if (_pos_state) (void)hipFree(_pos_state);
  if (_ctx) (void)_ctx->release_kv_access();
  if (_kv && _seq != kInvalidSequenceId) (void)_kv->release_sequence(_seq);
  for (hipEvent_t &e : _ready)
    if (e) (void)hipEventDestroy(e);
  if (_token_dev) (void)hipFree(_token_dev);
  if (_positions_dev) (void)hipFree(_positions_dev);
  if (_argmax_ws) (void)hipFree(_argmax_ws);
  if (_logit_dev) (void)hipFree(_logit_dev);
  if (_token_host) (void)hipHostFree(_token_host);
}

infer::expected<void, std::error_code> Qwen3Runner::init() {
  const Qwen3Hparams &hp = _model.hparams();
  std::vector<KVLayerSpec> specs(hp.n_layer, KVLayerSpec{hp.n_head_kv, hp.head_dim, hp.head_dim});
  std::vector<Backend *> place(hp.n_layer, &_backend);
  KVCacheConfig cfg{.layers = hp.n_layer, .max_tokens_per_sequence = _capacity};
  if (_kv_opt.block_tokens > 0 && _kv_opt.offload_bytes > 0) return infer::fail(std::errc::invalid_argument);
  if (_kv_opt.block_tokens > 0) {
    const size_t bt = _kv_opt.block_tokens;
    const size_t blocks = _kv_opt.pool_blocks ? _kv_opt.pool_blocks : (_capacity + bt - 1) / bt;
    cfg.block_tokens = bt;
    _kv = std::make_unique<KVCacheManager>(std::make_unique<PagedKVStrategy>(
        std::make_unique<BlockPoolKVStorage>(blocks, bt)));
  } else if (_kv_opt.offload_bytes > 0) {
    _host = std::make_unique<PinnedHostBackend>(0);
    OffloadKVStorageConfig oc;
    oc.host_backend = _host.get();
    oc.device_budgets.push_back({.backend = &_backend, .resident_bytes = _kv_opt.offload_bytes,
                                 .prefetch_bytes = _kv_opt.offload_bytes});
    _kv = std::make_unique<KVCacheManager>(std::make_unique<ContiguousKVStrategy>(
        std::make_unique<OffloadKVStorage>(std::move(oc), std::make_unique<LRUKVEvictionPolicy>(),
                                           std::make_unique<NextAccessKVPrefetchPolicy>(2))));
  } else {
    _kv = std::make_unique<KVCacheManager>(
        std::make_unique<ContiguousKVStrategy>(std::make_unique<NaiveKVStorage>()));
  }
  if (auto r = _kv->init(specs, place, cfg); !r) return r;
  if (auto r = _backend.reserve_decode_workspace(int(hp.n_head), int(hp.n_head_kv), int(hp.head_dim),
                                                 int64_t(_capacity));
      !r)
    return r;
  _sched = std::make_unique<Scheduler>(&_backend);
  _ctx = std::make_unique<GraphContext>(nullptr);
  _tokens = _ctx->make_tensor("inp_tokens", GGML_TYPE_I32, {1});
  _pos = _ctx->make_tensor("inp_pos", GGML_TYPE_I32, {1});
  for (Tensor *t : {_tokens, _pos}) t->tensorRole = TensorRole::TNESOR_ROLE_INPUT;
  _ctx->set_input_tokens(_tokens);
  _ctx->set_input_pos(_pos);
  auto fail_alloc = [] {
    (void)hipGetLastError();
    return infer::fail(std::errc::not_enough_memory);
  };
  if (hipMalloc(&_token_dev, (kSlots + 1) * sizeof(int32_t)) != hipSuccess) return fail_alloc();
  if (hipMalloc(&_pos_state, sizeof(int32_t)) != hipSuccess) return fail_alloc();
  if (hipMalloc(&_positions_dev, _capacity * sizeof(int32_t)) != hipSuccess) return fail_alloc();
  if (hipMalloc(&_argmax_ws, ikv_argmax_workspace_bytes()) != hipSuccess ||
      hipMemset(_argmax_ws, 0, ikv_argmax_workspace_bytes()) != hipSuccess)
    return fail_alloc();
  // Mapped and coherent: the sampler's store reaches host memory directly.
  if (hipHostMalloc(&_token_host, kSlots * sizeof(int32_t), hipHostMallocMapped | hipHostMallocCoherent) !=
          hipSuccess ||
      hipHostGetDevicePointer(reinterpret_cast<void **>(&_token_host_dev), _token_host, 0) !=
          hipSuccess)
    return fail_alloc();
  for (hipEvent_t &e : _ready)
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) return fail_alloc();
  std::vector<int32_t> iota(_capacity);
  for (size_t i = 0; i < _capacity; ++i) iota[i] = int32_t(i);
  if (hipMemcpy(_positions_dev, iota.data(), _capacity * sizeof(int32_t), hipMemcpyHostToDevice) !=
      hipSuccess)
    return infer::fail(std::errc::io_error);
  return {};
}

infer::expected<void, std::error_code> Qwen3Runner::enqueue_step(const int32_t *host_tokens,
                                                                 int64_t n, int in_slot,
                                                                 int out_slot,
                                                                 GenerationTiming &timing,
                                                                 int host_slot) {
  using Clock = std::chrono::steady_clock;
  if (host_slot < 0) host_slot = out_slot;
  const auto t0 = Clock::now();
  auto n_past = _kv->length(_seq);
  if (!n_past) return infer::unexpected(n_past.error());
  if (auto r = _kv->reserve_append(_seq, size_t(n)); !r) return r;
  for (Tensor *t : {_tokens, _pos}) {
    t->dims = {n, 1, 1, 1};
    t->set_contiguous_strides();
  }
  if (host_tokens) {  // the prompt: a host input the scheduler stages
    _input.assign(host_tokens, host_tokens + n);
    _tokens->data = _input.data();
    _tokens->device = DeviceType::CPU;
    _tokens->backend = nullptr;
  } else {  // the previous step's greedy token, already on the device
    _tokens->data = _token_dev + in_slot;
    _tokens->device = DeviceType::HIP;
    _tokens->backend = &_backend;
  }
  _pos->data = _positions_dev + *n_past;
  _pos->device = DeviceType::HIP;
  _pos->backend = &_backend;

  auto abort = [&](std::error_code e) -> infer::expected<void, std::error_code> {
    (void)_backend.synchronize();
    (void)_ctx->release_kv_access();
    (void)_kv->abort_append(_seq);
    return infer::unexpected(e);
  };
  auto graph = _model.build_graph(*_ctx);
  if (!graph) return abort(graph.error());
  const auto t1 = Clock::now();
  if (auto r = _sched->execute(*graph); !r) return abort(r.error());
  const Tensor *logits = graph->outputs().front();
  const int64_t vocab = logits->dims[0];
  const float *row = static_cast<const float *>(logits->data) + (logits->dims[1] - 1) * vocab;
  hipStream_t s = _backend.stream();
  // The sampler writes the token to the device slot the next step embeds
  // and to the pinned host slot the host reads once the event has fired.
  if (ikv_argmax_ws_f32(row, vocab, _token_dev + out_slot, _token_host_dev + host_slot, _argmax_ws,
                        ikv_argmax_workspace_bytes(), s) != 0 ||
      !keep_logits(row, vocab, s) || hipEventRecord(_ready[host_slot], s) != hipSuccess)
    return abort(std::make_error_code(std::errc::io_error));
  // The kernels of this step hold no host-side state: hand the layer
  // accesses back and commit the appended range now.
  if (auto r = _ctx->release_kv_access(); !r) return r;
  if (auto r = _kv->commit_append(_seq); !r) return r;
  const auto t2 = Clock::now();
  timing.build_s += std::chrono::duration<double>(t1 - t0).count();
  timing.execute_s += std::chrono::duration<double>(t2 - t1).count();
  return {};
}

// ---------------------------------------------------------------------------
// replayed decode steps

namespace {

// The position slot of the captured step: set before a capture's first
// launch, advanced by the step itself (kernels, so that nothing but launches
// sits in the captured stream).
__global__ void set_position_kernel(int32_t *p, int32_t v) { *p = v; }
__global__ void advance_position_kernel(int32_t *p) { *p += 1; }

// Contexts one capture may serve; the decode's replay limit may cut it short
// where its split plan changes.
constexpr int64_t kReplayWidth = 256;

}  // namespace

void Qwen3Runner::drop_step_graph() {
  if (_step_exec) (void)hipGraphExecDestroy(_step_exec);
  _step_exec = nullptr;
  _step_lo = _step_hi = 0;
  _step_logits = nullptr;
}

// Captures one decode step of _seq at n_past (its host bookkeeping included):
// the token comes from device slot kReplaySlot, the position from
// _pos_state, the decode reads its context from that position and is planned
// for the largest context the capture serves; the step ends by advancing
// _pos_state. The sampler stays outside: its host slot alternates.
infer::expected<void, std::error_code> Qwen3Runner::capture_step(int64_t n_past) {
  const Qwen3Hparams &hp = _model.hparams();
  const int64_t n_kv = n_past + 1;
  int64_t hi = ikv_attn_decode_replay_limit(int(hp.n_head), int(hp.n_head_kv), int(hp.head_dim),
                                            n_kv, kReplayWidth);
  hi = std::min<int64_t>(hi, int64_t(_capacity));
  if (hi < n_kv) return infer::fail(std::errc::not_supported);
  drop_step_graph();
  hipStream_t s = _backend.stream();
  set_position_kernel<<<1, 1, 0, s>>>(_pos_state, int32_t(n_past));
  if (hipGetLastError() != hipSuccess) return infer::fail(std::errc::io_error);
  if (auto r = _kv->reserve_append(_seq, 1); !r) return r;
  for (Tensor *t : {_tokens, _pos}) {
    t->dims = {1, 1, 1, 1};
    t->set_contiguous_strides();
  }
  _tokens->data = _token_dev + kReplaySlot;
  _tokens->device = DeviceType::HIP;
  _tokens->backend = &_backend;
  _pos->data = _pos_state;
  _pos->device = DeviceType::HIP;
  _pos->backend = &_backend;
  if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) {
    (void)hipGetLastError();
    (void)_kv->abort_append(_seq);
    return infer::fail(std::errc::not_supported);
  }
  _backend.set_decode_replay(hi);
  auto graph = _model.build_graph(*_ctx);
  infer::expected<void, std::error_code> r =
      graph ? _sched->execute(*graph) : infer::expected<void, std::error_code>(infer::unexpected(graph.error()));
  if (r) {
    advance_position_kernel<<<1, 1, 0, s>>>(_pos_state);
    if (hipGetLastError() != hipSuccess) r = infer::fail(std::errc::io_error);
  }
  _backend.set_decode_replay(0);
  hipGraph_t g = nullptr;
  const bool ended = hipStreamEndCapture(s, &g) == hipSuccess && g;
  if (r && !ended) r = infer::fail(std::errc::not_supported);
  if (r && hipGraphInstantiate(&_step_exec, g, nullptr, nullptr, 0) != hipSuccess) {
    _step_exec = nullptr;
    r = infer::fail(std::errc::not_supported);
  }
  if (g) (void)hipGraphDestroy(g);
  (void)hipGetLastError();
  if (!r) {
    (void)_ctx->release_kv_access();
    (void)_kv->abort_append(_seq);
    return r;
  }
  const Tensor *logits = graph->outputs().front();
  _step_vocab = logits->dims[0];
  _step_logits = static_cast<const float *>(logits->data) + (logits->dims[1] - 1) * _step_vocab;
  _step_lo = n_kv;
  _step_hi = hi;
  if (auto rr = _ctx->release_kv_access(); !rr) return rr;
  if (auto rr = _kv->commit_append(_seq); !rr) return rr;
  ++_replay_stats.captures;
  return {};
}

infer::expected<void, std::error_code> Qwen3Runner::replay_step(int host_slot,
                                                                GenerationTiming &timing) {
  using Clock = std::chrono::steady_clock;
  const auto t0 = Clock::now();
  auto n_past = _kv->length(_seq);
  if (!n_past) return infer::unexpected(n_past.error());
  const int64_t n_kv = int64_t(*n_past) + 1;
  if (!_step_exec || n_kv < _step_lo || n_kv > _step_hi) {
    if (auto r = capture_step(int64_t(*n_past)); !r) return r;
  } else {
    if (auto r = _kv->reserve_append(_seq, 1); !r) return r;
    if (auto r = _kv->commit_append(_seq); !r) return r;
  }
  const auto t1 = Clock::now();
  hipStream_t s = _backend.stream();
  if (hipGraphLaunch(_step_exec, s) != hipSuccess ||
      ikv_argmax_ws_f32(_step_logits, _step_vocab, _token_dev + kReplaySlot,
                        _token_host_dev + host_slot, _argmax_ws, ikv_argmax_workspace_bytes(),
                        s) != 0 ||
      !keep_logits(_step_logits, _step_vocab, s) || hipEventRecord(_ready[host_slot], s) != hipSuccess)
    return infer::fail(std::errc::io_error);
  ++_replay_stats.replays;
  const auto t2 = Clock::now();
  timing.build_s += std::chrono::duration<double>(t1 - t0).count();
  timing.execute_s += std::chrono::duration<double>(t2 - t1).count();
  return {};
}

infer::expected<void, std::error_code> Qwen3Runner::set_logit_capture(
    const std::vector<int64_t> &steps) {
  if (_logit_dev) {
    (void)_backend.synchronize();
    (void)hipFree(_logit_dev);
    _logit_dev = nullptr;
  }
  _logit_steps.clear();
  if (steps.empty()) return {};
  for (const int64_t st : steps)
    if (st < 0) return infer::fail(std::errc::invalid_argument);
  const size_t vocab = _model.hparams().n_vocab;
  if (hipMalloc(&_logit_dev, steps.size() * vocab * sizeof(float)) != hipSuccess) {
    (void)hipGetLastError();
    _logit_dev = nullptr;
    return infer::fail(std::errc::not_enough_memory);
  }
  _logit_steps = steps;
  return {};
}

infer::expected<void, std::error_code> Qwen3Runner::captured_logits(float *host,
                                                                    size_t count) const {
  const size_t vocab = _model.hparams().n_vocab;
  if (!host || !_logit_dev || count != _logit_steps.size() * vocab)
    return infer::fail(std::errc::invalid_argument);
  if (hipMemcpy(host, _logit_dev, count * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess)
    return infer::fail(std::errc::io_error);
  return {};
}

bool Qwen3Runner::keep_logits(const float *row, int64_t vocab, hipStream_t s) {
  for (size_t k = 0; k < _logit_steps.size(); ++k) {
    if (size_t(_logit_steps[k]) != _cur_step) continue;
    if (size_t(vocab) != _model.hparams().n_vocab) return false;
    if (hipMemcpyAsync(_logit_dev + k * size_t(vocab), row, size_t(vocab) * sizeof(float),
                       hipMemcpyDeviceToDevice, s) != hipSuccess)
      return false;
  }
  return true;
}

infer::expected<int32_t, std::error_code> Qwen3Runner::collect(int slot) {
  if (hipEventSynchronize(_ready[slot]) != hipSuccess) return infer::fail(std::errc::io_error);
  const int32_t tok = _token_host[slot];
  if (tok < 0) return infer::fail(std::errc::invalid_argument);  // NaN / +inf logits
  return tok;
}

infer::expected<void, std::error_code> Qwen3Runner::generate(const std::vector<int32_t> &prompt,
                                                             size_t n_gen,
                                                             std::vector<int32_t> &tokens_out,
                                                             GenerationTiming &timing) {
  using Clock = std::chrono::steady_clock;
  if (prompt.empty() || n_gen == 0) return infer::fail(std::errc::invalid_argument);
  if (prompt.size() + n_gen - 1 > _capacity) return infer::fail(std::errc::value_too_large);
  if (!_kv) return infer::fail(std::errc::invalid_argument);
  auto sid = _kv->create_sequence();
  if (!sid) return infer::unexpected(sid.error());
  _seq = *sid;
  if (auto r = _ctx->set_kv_cache(_kv.get(), _seq); !r) return r;
  timing = GenerationTiming{};
  tokens_out.clear();
  auto finish = [&](infer::expected<void, std::error_code> r) {
    const auto sync = _backend.synchronize();
    drop_step_graph();  // its addresses are this sequence's cache rows
    (void)_ctx->release_kv_access();
    (void)_ctx->set_kv_cache(nullptr, kInvalidSequenceId);
    (void)_kv->release_sequence(_seq);
    _seq = kInvalidSequenceId;
    if (r && !sync) return sync;
    return r;
  };
  const auto start = Clock::now();
  Clock::time_point first{}, last{};
  auto take = [&](int slot, size_t i) -> infer::expected<void, std::error_code> {
    const auto t0 = Clock::now();
    auto tok = collect(slot);
    if (!tok) return infer::unexpected(tok.error());
    const auto ready = Clock::now();
    timing.sample_s += std::chrono::duration<double>(ready - t0).count();
    if (i == 0) first = ready;
    last = ready;
    tokens_out.push_back(*tok);
    return {};
  };
  // Step i hands its token to the host in slot i % 2. Eager steps read
  // device slot (i - 1) % 2 and write slot i % 2; replayed steps, whose
  // graph holds one address, read and write device slot kReplaySlot.
  _replay_stats = {};
  drop_step_graph();
  // (a paged cache replays too: its block tables sit at fixed device
  // addresses, and a step that opens a block writes the new entries before
  // the graph is launched)
  bool replay = _replay && _kv_opt.offload_bytes == 0 && _backend.fusion();
  const bool one_slot = replay;  // the device token stays in kReplaySlot throughout
  _cur_step = 0;
  if (auto r = enqueue_step(prompt.data(), int64_t(prompt.size()), 1, one_slot ? kReplaySlot : 0,
                            timing, 0);
      !r)
    return finish(r);
  for (size_t i = 1; i < n_gen; ++i) {
    const int host_slot = int(i & 1);
    _cur_step = i;
    infer::expected<void, std::error_code> r;
    if (replay) {
      r = replay_step(host_slot, timing);
      if (!r && r.error() == std::make_error_code(std::errc::not_supported)) {
        replay = false;  // this step and the rest launch eagerly
        drop_step_graph();
      }
    }
    if (!replay) {
      r = one_slot ? enqueue_step(nullptr, 1, kReplaySlot, kReplaySlot, timing, host_slot)
                   : enqueue_step(nullptr, 1, int((i - 1) & 1), host_slot, timing);
    }
    if (!r) return finish(r);
    if (auto rr = take(int((i - 1) & 1), i - 1); !rr) return finish(rr);
  }
  if (auto r = take(int((n_gen - 1) & 1), n_gen - 1); !r) return finish(r);
  timing.wall_s = std::chrono::duration<double>(Clock::now() - start).count();
  timing.ttft_s = std::chrono::duration<double>(first - start).count();
  timing.tpot_s =
      n_gen > 1 ? std::chrono::duration<double>(last - first).count() / double(n_gen - 1) : 0.0;
  return finish({});
}

infer::expected<void, std::error_code> Qwen3Runner::generate_interleaved(
    const std::vector<std::vector<int32_t>> &prompts, size_t n_gen,
    std::vector<std::vector<int32_t>> &tokens_out, GenerationTiming &timing) {
  using Clock = std::chrono::steady_clock;
  const size_t n_seq = prompts.size();
  if (n_seq == 0 || n_seq > size_t(kMaxInterleaved) || n_gen == 0)
    return infer::fail(std::errc::invalid_argument);
  for (const auto &p : prompts) {
    if (p.empty()) return infer::fail(std::errc::invalid_argument);
    if (p.size() + n_gen - 1 > _capacity) return infer::fail(std::errc::value_too_large);
  }
  if (!_kv) return infer::fail(std::errc::invalid_argument);
  // interleaved steps are eager: nothing of an earlier generate() is replayed
  // or counted here
  _replay_stats = {};
  drop_step_graph();
  std::vector<SequenceId> seqs;
  auto finish = [&](infer::expected<void, std::error_code> r) {
    const auto sync = _backend.synchronize();
    (void)_ctx->release_kv_access();
    (void)_ctx->set_kv_cache(nullptr, kInvalidSequenceId);
    for (SequenceId id : seqs) (void)_kv->release_sequence(id);
    _seq = kInvalidSequenceId;
    if (r && !sync) return sync;
    return r;
  };
  for (size_t s = 0; s < n_seq; ++s) {
    auto sid = _kv->create_sequence();
    if (!sid) return finish(infer::unexpected(sid.error()));
    seqs.push_back(*sid);
  }
  timing = GenerationTiming{};
  tokens_out.assign(n_seq, {});
  // sequence s, step i: writes slot 2s + i % 2, reads slot 2s + (i - 1) % 2
  auto turn = [&](size_t s, size_t i) -> infer::expected<void, std::error_code> {
    _seq = seqs[s];
    if (auto r = _ctx->set_kv_cache(_kv.get(), _seq); !r) return r;
    const int base = int(2 * s);
    if (i == 0)
      return enqueue_step(prompts[s].data(), int64_t(prompts[s].size()), base + 1, base, timing);
    return enqueue_step(nullptr, 1, base + int((i - 1) & 1), base + int(i & 1), timing);
  };
  const auto start = Clock::now();
  Clock::time_point first{}, last{};
  auto take_round = [&](size_t i) -> infer::expected<void, std::error_code> {
    const auto t0 = Clock::now();
    for (size_t s = 0; s < n_seq; ++s) {
      auto tok = collect(int(2 * s) + int(i & 1));
      if (!tok) return infer::unexpected(tok.error());
      tokens_out[s].push_back(*tok);
    }
    const auto ready = Clock::now();
    timing.sample_s += std::chrono::duration<double>(ready - t0).count();
    if (i == 0) first = ready;
    last = ready;
    return {};
  };
  for (size_t i = 0; i < n_gen; ++i) {
    for (size_t s = 0; s < n_seq; ++s)
      if (auto r = turn(s, i); !r) return finish(r);
    if (i > 0)
      if (auto r = take_round(i - 1); !r) return finish(r);
  }
  if (auto r = take_round(n_gen - 1); !r) return finish(r);
  timing.wall_s = std::chrono::duration<double>(Clock::now() - start).count();
  timing.ttft_s = std::chrono::duration<double>(first - start).count();
  timing.tpot_s =
      n_gen > 1 ? std::chrono::duration<double>(last - first).count() / double(n_gen - 1) : 0.0;
  return finish({});
}

OffloadStats Qwen3Runner::offload_stats() const {
  if (!_kv) return {};
  if (const auto *o = dynamic_cast<const OffloadKVStorage *>(_kv->strategy()->storage())) return o->stats();
  return {};
}

