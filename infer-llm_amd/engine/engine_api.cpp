// engine_api.cpp — the C-ABI of include/ikv_engine.h over Qwen3Model /
// Qwen3Runner on a HIPBackend.
#include <cerrno>
#include <memory>
#include <mutex>
#include <new>
#include <string>

#include "../../include/ikv_engine.h"
#include "backend.hpp"
#include "hip_backend.hpp"
#include "qwen3.hpp"

struct ikv_qwen3 {
  std::unique_ptr<Backend> backend;
  std::unique_ptr<Qwen3Model> model;
  std::unique_ptr<Qwen3Runner> runner;
  std::vector<std::string> names;
};

namespace {

int to_errno(const std::error_code &e) { return e.value() > 0 ? -e.value() : -EIO; }

HIPBackend *hip(ikv_qwen3 *m) { return static_cast<HIPBackend *>(m->backend.get()); }

}  // namespace

namespace {

int create(const ikv_qwen3_config *cfg, int device, int64_t max_ctx, const KVOptions &kv,
           ikv_qwen3 **out) {
  if (!cfg || !out || max_ctx <= 0 || device < 0) return -EINVAL;
  if (kv.block_tokens % 64 != 0) return -EINVAL;
  *out = nullptr;
  if (cfg->n_layer == 0 || cfg->n_embd == 0 || cfg->n_head == 0 || cfg->n_head_kv == 0 ||
      cfg->head_dim == 0 || cfg->n_ff == 0 || cfg->n_vocab == 0 ||
      cfg->n_head % cfg->n_head_kv != 0 || uint64_t(max_ctx) > cfg->n_ctx_train)
    return -EINVAL;
  static std::once_flag registered;
  std::call_once(registered, [] { register_hip_backend(); });
  auto &reg = BackendRegistry::instance();
  reg.probe_all();
  auto created = reg.create("hip:" + std::to_string(device), {});
  if (!created) return to_errno(created.error());
  auto m = std::unique_ptr<ikv_qwen3>(new (std::nothrow) ikv_qwen3);
  if (!m) return -ENOMEM;
  m->backend = std::move(*created);
  Qwen3Hparams hp;
  hp.n_layer = cfg->n_layer;
  hp.n_embd = cfg->n_embd;
  hp.n_head = cfg->n_head;
  hp.n_head_kv = cfg->n_head_kv;
  hp.head_dim = cfg->head_dim;
  hp.n_ff = cfg->n_ff;
  hp.n_vocab = cfg->n_vocab;
  hp.n_ctx_train = cfg->n_ctx_train;
  hp.rope_theta = cfg->rope_theta;
  hp.rms_norm_eps = cfg->rms_norm_eps;
  if (cfg->untied_output > 1) return -EINVAL;
  hp.untied_output = cfg->untied_output != 0;
  m->model = std::make_unique<Qwen3Model>(hp);
  if (auto r = m->model->alloc_weights(m->backend.get()); !r) return to_errno(r.error());
  m->runner = std::make_unique<Qwen3Runner>(*m->model, *hip(m.get()), size_t(max_ctx), kv);
  if (auto r = m->runner->init(); !r) return to_errno(r.error());
  m->names = m->model->tensor_names();
  *out = m.release();
  return 0;
}

}  // namespace

extern "C" int ikv_qwen3_create(const ikv_qwen3_config *cfg, int device, int64_t max_ctx,
                                ikv_qwen3 **out) {
  return create(cfg, device, max_ctx, KVOptions{}, out);
}

extern "C" int ikv_qwen3_create_paged(const ikv_qwen3_config *cfg, int device, int64_t max_ctx,
                                      int64_t block_tokens, int64_t pool_blocks, ikv_qwen3 **out) {
  if (block_tokens <= 0 || pool_blocks < 0) return -EINVAL;
  return create(cfg, device, max_ctx,
                KVOptions{.block_tokens = size_t(block_tokens), .pool_blocks = size_t(pool_blocks)}, out);
}

extern "C" int ikv_qwen3_create_offload(const ikv_qwen3_config *cfg, int device, int64_t max_ctx,
                                        uint64_t hbm_bytes, ikv_qwen3 **out) {
  if (hbm_bytes == 0) return -EINVAL;
  return create(cfg, device, max_ctx, KVOptions{.offload_bytes = size_t(hbm_bytes)}, out);
}

extern "C" int ikv_qwen3_kv_stats(const ikv_qwen3 *m, ikv_qwen3_kv_counters *out) {
  if (!m || !out) return -EINVAL;
  const OffloadStats s = m->runner->offload_stats();
  *out = {s.page_ins, s.page_outs, s.evictions, s.bytes_in, s.bytes_out};
  return 0;
}

extern "C" int ikv_qwen3_tensor_count(const ikv_qwen3 *m) {
  return m ? static_cast<int>(m->names.size()) : 0;
}

extern "C" const char *ikv_qwen3_tensor_name(const ikv_qwen3 *m, int index) {
  if (!m || index < 0 || size_t(index) >= m->names.size()) return nullptr;
  return m->names[size_t(index)].c_str();
}

extern "C" size_t ikv_qwen3_tensor_size(const ikv_qwen3 *m, const char *name) {
  if (!m || !name) return 0;
  const Tensor *t = m->model->find(name);
  return t ? t->element_count() : 0;
}

extern "C" int ikv_qwen3_set_tensor(ikv_qwen3 *m, const char *name, const float *host,
                                    size_t count) {
  if (!m || !name || !host) return -EINVAL;
  auto r = m->model->set_tensor(name, host, count);
  return r ? 0 : to_errno(r.error());
}

extern "C" int ikv_qwen3_init_synthetic(ikv_qwen3 *m, uint64_t seed, double std, int threads) {
  if (!m) return -EINVAL;
  auto r = m->model->init_synthetic(seed, std, threads);
  return r ? 0 : to_errno(r.error());
}

extern "C" int ikv_qwen3_generate(ikv_qwen3 *m, const int32_t *prompt, int64_t n_prompt,
                                  int64_t n_gen, int32_t *tokens_out, ikv_qwen3_timing *timing) {
  if (!m || !prompt || n_prompt <= 0 || n_gen <= 0 || !tokens_out) return -EINVAL;
  std::vector<int32_t> p(prompt, prompt + n_prompt), toks;
  GenerationTiming t;
  auto r = m->runner->generate(p, size_t(n_gen), toks, t);
  if (!r) return to_errno(r.error());
  for (size_t i = 0; i < toks.size(); ++i) tokens_out[i] = toks[i];
  if (timing) *timing = {t.ttft_s, t.tpot_s, t.wall_s, t.build_s, t.execute_s, t.sample_s};
  return 0;
}

extern "C" int ikv_qwen3_generate_interleaved(ikv_qwen3 *m, const int32_t *prompts, int64_t n_seq,
                                              int64_t n_prompt, int64_t n_gen,
                                              int32_t *tokens_out, ikv_qwen3_timing *timing) {
  if (!m || !prompts || n_seq <= 0 || n_seq > Qwen3Runner::kMaxInterleaved || n_prompt <= 0 ||
      n_gen <= 0 || !tokens_out)
    return -EINVAL;
  std::vector<std::vector<int32_t>> p(static_cast<size_t>(n_seq)), toks;
  for (int64_t s = 0; s < n_seq; ++s) p[s].assign(prompts + s * n_prompt, prompts + (s + 1) * n_prompt);
  GenerationTiming t;
  auto r = m->runner->generate_interleaved(p, size_t(n_gen), toks, t);
  if (!r) return to_errno(r.error());
  for (int64_t s = 0; s < n_seq; ++s)
    for (int64_t i = 0; i < n_gen; ++i) tokens_out[s * n_gen + i] = toks[s][i];
  if (timing) *timing = {t.ttft_s, t.tpot_s, t.wall_s, t.build_s, t.execute_s, t.sample_s};
  return 0;
}

extern "C" int ikv_qwen3_last_stats(const ikv_qwen3 *m, ikv_qwen3_stats *out) {
  if (!m || !out) return -EINVAL;
  const auto &s = static_cast<const HIPBackend *>(m->backend.get())->last_stats();
  const Qwen3Runner::ReplayStats rs = m->runner->replay_stats();
  *out = {s.launches,       s.fused_norm_rope, s.fused_append_decode, s.fused_swiglu,
          s.fused_residual, s.fused_qkv,       s.fused_norm_mm,       s.fused_rope_decode,
          s.fused_qkv_decode, s.fused_append,  rs.captures,           rs.replays};
  return 0;
}

extern "C" int ikv_qwen3_capture_logits(ikv_qwen3 *m, const int64_t *steps, int64_t n_steps) {
  if (!m || n_steps < 0 || (n_steps > 0 && !steps)) return -EINVAL;
  std::vector<int64_t> v(steps, steps + n_steps);
  if (auto r = m->runner->set_logit_capture(v); !r) return -r.error().value();
  return 0;
}

extern "C" int ikv_qwen3_captured_logits(const ikv_qwen3 *m, float *host, size_t count) {
  if (!m) return -EINVAL;
  if (auto r = m->runner->captured_logits(host, count); !r) return -r.error().value();
  return 0;
}

extern "C" int ikv_qwen3_set_step_replay(ikv_qwen3 *m, int on) {
  if (!m) return -EINVAL;
  m->runner->set_step_replay(on != 0);
  return 0;
}

extern "C" int ikv_qwen3_set_fusion(ikv_qwen3 *m, int on) {
  if (!m) return -EINVAL;
  hip(m)->set_fusion(on != 0);
  return 0;
}

extern "C" void ikv_qwen3_destroy(ikv_qwen3 *m) {
  if (!m) return;
  m->runner.reset();
  m->model.reset();
  m->backend.reset();
  delete m;
}
