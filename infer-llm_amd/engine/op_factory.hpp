// op_factory.hpp — graph-node constructors for the ops on the KV-cache path
// (reference include/op_factory.hpp:11-54, src/op_factory.cpp:78-182), the
// KV append nodes of ModelBase::append_kv (src/model.cpp:602-625) and the
// Qwen3 layer-attention slice that calls them (src/models/Qwen3.cpp:53-88).
#pragma once

#include <cstdint>
#include <initializer_list>
#include <string_view>
#include <system_error>

#include "expected.hpp"
#include "graph.hpp"
#include "op_params.hpp"
#include "tensor.hpp"

struct OpFactory {
  // Elementwise a + b, a * b of equal shapes (src/op_factory.cpp:16-59).
  static Tensor *add(Graph &g, Tensor *a, Tensor *b, std::string_view name);
  static Tensor *mul(Graph &g, Tensor *a, Tensor *b, std::string_view name);
  // x / (1 + exp(-x)): UNARY with GGML_UNARY_OP_SILU in op_params[0]
  // (src/op_factory.cpp:126-136).
  static Tensor *silu(Graph &g, Tensor *x, std::string_view name);
  // w [n_embd, n_out] (rows of n_embd), x [n_embd, n_tokens] ->
  // out [n_out, n_tokens] (src/op_factory.cpp:98-108).
  static Tensor *mul_mat(Graph &g, Tensor *w, Tensor *x, std::string_view name);
  // GET_ROWS of token_embd [n_embd, n_vocab] by input_token [n_tokens] ->
  // [n_embd, n_tokens] (src/op_factory.cpp:78-94).
  static Tensor *embedding(Graph &g, Tensor *token_embd, Tensor *input_token);
  // out = rms_norm(x) * weight along dims[0]; eps in op_params[0].
  static Tensor *rms_norm(Graph &g, Tensor *x, Tensor *weight, float eps, std::string_view name);
  // NeoX RoPE of x [head_dim, n_heads, n_tokens] at positions pos [n_tokens]
  // with the angle table [head_dim/2, n_ctx].
  static Tensor *rope(Graph &g, Tensor *x, Tensor *pos, Tensor *theta_table, std::string_view name);
  // out [v.dims[0], q.dims[1], q.dims[2], q.dims[3]]; AttnParams in op_params.
  static Tensor *flash_attn(Graph &g, Tensor *q, Tensor *k, Tensor *v, const AttnParams &p,
                            std::string_view name);
  static Tensor *reshape(Graph &g, Tensor *x, std::initializer_list<int64_t> shape,
                         std::string_view name);
  // Rows [row0, row0 + n_rows) of a contiguous [dims0, rows] activation, as a
  // VIEW node aliasing its bytes (data = x's data + offset, set when the
  // scheduler places x; no kernel runs).
  static Tensor *view_rows(Graph &g, Tensor *x, int64_t row0, int64_t n_rows, std::string_view name);
};

// KV append: a CPY node writing `current` into the writable cache view,
// then a VIEW node of the readable view [0, n_past + n_new) whose src[0] is
// the CPY, so consumers of the view run after the append.
Tensor *append_kv(Graph &g, Tensor *current, const Tensor &writable, const Tensor &readable);
// The same pair for a paged layer: a CPY of `current` into its pool blocks
// and a VIEW of logical rows [0, readable.dims[2]) of the pool, each with the
// block table as src[1] and (block_tokens, pool blocks, first token) in
// op_params[0..2].
Tensor *append_kv_paged(Graph &g, Tensor *current, const KVPages &pages, void *pool,
                        const Tensor &readable, std::size_t n_past);

struct AttentionSliceParams {
  uint32_t n_head = 16;
  uint32_t n_head_kv = 8;
  uint32_t head_dim = 128;
  float rms_norm_eps = 1e-6f;
  float rope_theta = 1e6f;
  uint32_t n_ctx_train = 40960;
};

// One layer's attention between the q/k/v projections and the output
// projection: reshape -> qk-RMSNorm -> RoPE -> KV append (k after RoPE, v
// as projected) -> flash attention over the cache, in the order of
// src/models/Qwen3.cpp:61-88. q_proj [n_head*head_dim, n_tokens],
// k_proj/v_proj [n_head_kv*head_dim, n_tokens]. Acquires the layer's KV
// access from `ctx` (released by the caller through release_kv_access()).
// Returns the attention output [head_dim, n_head, n_tokens].
infer::expected<Tensor *, std::error_code> build_attention_slice(
    Graph &g, GraphContext &ctx, Tensor *q_proj, Tensor *k_proj, Tensor *v_proj, Tensor *q_norm_w,
    Tensor *k_norm_w, std::size_t layer, const AttentionSliceParams &p);
