#include "op_factory.hpp"

#include <cassert>
#include <cmath>
#include <cstring>
#include <string>

namespace {

Tensor *new_node(Graph &g, std::string_view name, DataType type, std::initializer_list<int64_t> shape,
                 OperationType op) {
  auto t = std::make_unique<Tensor>(name, type, shape);
  t->op = op;
  t->tensorRole = TensorRole::TENSOR_ROLE_ACTIVATION;
  return g.add_node(std::move(t));
}

}  // namespace

Tensor *OpFactory::add(Graph &g, Tensor *a, Tensor *b, std::string_view name) {
  assert(a->dims == b->dims && a->dataType == b->dataType);
  Tensor *r = new_node(g, name, a->dataType, {a->dims[0], a->dims[1], a->dims[2], a->dims[3]},
                       OperationType::GGML_OP_ADD);
  r->src[0] = a;
  r->src[1] = b;
  return r;
}

Tensor *OpFactory::mul(Graph &g, Tensor *a, Tensor *b, std::string_view name) {
  assert(a->dims == b->dims && a->dataType == b->dataType);
  Tensor *r = new_node(g, name, a->dataType, {a->dims[0], a->dims[1], a->dims[2], a->dims[3]},
                       OperationType::GGML_OP_MUL);
  r->src[0] = a;
  r->src[1] = b;
  return r;
}

Tensor *OpFactory::silu(Graph &g, Tensor *x, std::string_view name) {
  Tensor *r = new_node(g, name, x->dataType, {x->dims[0], x->dims[1], x->dims[2], x->dims[3]},
                       OperationType::GGML_OP_UNARY);
  r->src[0] = x;
  const uint32_t sub = static_cast<uint32_t>(UnaryOp::GGML_UNARY_OP_SILU);
  std::memcpy(&r->op_params[0], &sub, sizeof(sub));
  return r;
}

Tensor *OpFactory::mul_mat(Graph &g, Tensor *w, Tensor *x, std::string_view name) {
  Tensor *r = new_node(g, name, x->dataType, {w->dims[1], x->dims[1]}, OperationType::GGML_OP_MUL_MAT);
  r->src[0] = w;
  r->src[1] = x;
  return r;
}

Tensor *OpFactory::embedding(Graph &g, Tensor *token_embd, Tensor *input_token) {
  Tensor *r = new_node(g, "embedding", token_embd->dataType, {token_embd->dims[0], input_token->dims[0]},
                       OperationType::GGML_OP_GET_ROWS);
  r->src[0] = token_embd;
  r->src[1] = input_token;
  return r;
}

Tensor *OpFactory::rms_norm(Graph &g, Tensor *x, Tensor *weight, float eps, std::string_view name) {
  Tensor *r = new_node(g, name, x->dataType, {x->dims[0], x->dims[1], x->dims[2], x->dims[3]},
                       OperationType::GGML_OP_RMS_NORM);
  r->src[0] = x;
  r->src[1] = weight;
  std::memcpy(&r->op_params[0], &eps, sizeof(eps));
  return r;
}

Tensor *OpFactory::rope(Graph &g, Tensor *x, Tensor *pos, Tensor *theta_table, std::string_view name) {
  Tensor *r = new_node(g, name, x->dataType, {x->dims[0], x->dims[1], x->dims[2], x->dims[3]},
                       OperationType::GGML_OP_ROPE);
  r->src[0] = x;
  r->src[1] = pos;
  r->src[2] = theta_table;
  return r;
}

Tensor *OpFactory::flash_attn(Graph &g, Tensor *q, Tensor *k, Tensor *v, const AttnParams &p,
                              std::string_view name) {
  Tensor *r = new_node(g, name, q->dataType, {v->dims[0], q->dims[1], q->dims[2], q->dims[3]},
                       OperationType::GGML_OP_FLASH_ATTN_EXT);
  r->src[0] = q;
  r->src[1] = k;
  r->src[2] = v;
  std::memcpy(&r->op_params[0], &p, sizeof(p));
  return r;
}

Tensor *OpFactory::reshape(Graph &g, Tensor *x, std::initializer_list<int64_t> shape,
                           std::string_view name) {
  int64_t total = 1;
  for (int64_t d : shape) total *= d;
  assert(static_cast<size_t>(total) == x->element_count());
  (void)total;
  Tensor *r = new_node(g, name, x->dataType, shape, OperationType::GGML_OP_RESHAPE);
  r->src[0] = x;
  return r;
}

Tensor *OpFactory::view_rows(Graph &g, Tensor *x, int64_t row0, int64_t n_rows, std::string_view name) {
  assert(x->is_contiguous() && x->dims[2] == 1 && x->dims[3] == 1);
  assert(row0 >= 0 && n_rows > 0 && row0 + n_rows <= x->dims[1]);
  Tensor *r = new_node(g, name, x->dataType, {x->dims[0], n_rows, 1, 1}, OperationType::GGML_OP_VIEW);
  r->src[0] = x;
  r->offset = row0 * x->strides[1];
  return r;
}

Tensor *append_kv(Graph &g, Tensor *current, const Tensor &writable, const Tensor &readable) {
  // The copies keep data pointing at the storage's cache memory.
  auto write = std::make_unique<Tensor>(writable);
  write->name = current->name + "_cache_write";
  write->op = OperationType::GGML_OP_CPY;
  write->src.fill(nullptr);
  write->src[0] = current;
  write->pinned = true;  // the cache lives on the storage's backend
  Tensor *write_node = g.add_node(std::move(write));

  auto full = std::make_unique<Tensor>(readable);
  full->name = current->name + "_cache_full";
  full->op = OperationType::GGML_OP_VIEW;
  full->src.fill(nullptr);
  full->src[0] = write_node;  // attention reads the view after the append
  full->pinned = true;
  return g.add_node(std::move(full));
}

Tensor *append_kv_paged(Graph &g, Tensor *current, const KVPages &pages, void *pool,
                        const Tensor &readable, std::size_t n_past) {
  // CPY: the step's rows into their pool blocks (first logical token n_past);
  // VIEW: logical rows [0, n_kv) of the pool. Both carry the block table as
  // src[1] and (block_tokens, pool blocks, first token) in op_params.
  auto tag = [&](Tensor &t) {
    t.data = pool;
    t.offset = 0;
    t.layer = readable.layer;
    t.backend = readable.backend;
    t.device = readable.device;
    t.tensorRole = TensorRole::TENSOR_ROLE_KVCACHE;
    t.pinned = true;
    t.op_params[0] = static_cast<int32_t>(pages.block_tokens);
    t.op_params[1] = static_cast<int32_t>(pages.pool_blocks);
    t.op_params[2] = static_cast<int32_t>(n_past);
  };
  auto write = std::make_unique<Tensor>(current->name + "_cache_write", current->dataType,
                                        std::initializer_list<int64_t>{current->dims[0], current->dims[1],
                                                                       current->dims[2], 1});
  write->op = OperationType::GGML_OP_CPY;
  tag(*write);
  write->src[0] = current;
  write->src[1] = pages.block_table;
  Tensor *write_node = g.add_node(std::move(write));

  auto full = std::make_unique<Tensor>(current->name + "_cache_full", readable.dataType,
                                       std::initializer_list<int64_t>{readable.dims[0], readable.dims[1],
                                                                      readable.dims[2], 1});
  full->op = OperationType::GGML_OP_VIEW;
  tag(*full);
  full->src[0] = write_node;
  full->src[1] = pages.block_table;
  return g.add_node(std::move(full));
}

infer::expected<Tensor *, std::error_code> build_attention_slice(
    Graph &g, GraphContext &ctx, Tensor *q_proj, Tensor *k_proj, Tensor *v_proj, Tensor *q_norm_w,
    Tensor *k_norm_w, std::size_t layer, const AttentionSliceParams &p) {
  Tensor *inp_pos = ctx.get_input_pos();
  if (!inp_pos || !q_proj || !k_proj || !v_proj) return infer::fail(std::errc::invalid_argument);
  auto theta = ctx.get_rope_theta_table(p.rope_theta, p.head_dim, p.n_ctx_train);
  if (!theta) return infer::unexpected(theta.error());
  const int64_t n_tokens = inp_pos->dims[0];
  const std::string l = std::to_string(layer);
  const int64_t hd = p.head_dim;

  Tensor *q = OpFactory::reshape(g, q_proj, {hd, p.n_head, n_tokens, 1}, "q_reshape_" + l);
  Tensor *k = OpFactory::reshape(g, k_proj, {hd, p.n_head_kv, n_tokens, 1}, "k_reshape_" + l);
  Tensor *v = OpFactory::reshape(g, v_proj, {hd, p.n_head_kv, n_tokens, 1}, "v_reshape_" + l);
  Tensor *qn = OpFactory::rms_norm(g, q, q_norm_w, p.rms_norm_eps, "attn_q_norm_" + l);
  Tensor *kn = OpFactory::rms_norm(g, k, k_norm_w, p.rms_norm_eps, "attn_k_norm_" + l);
  Tensor *qr = OpFactory::rope(g, qn, inp_pos, *theta, "rope_q_" + l);
  Tensor *kr = OpFactory::rope(g, kn, inp_pos, *theta, "rope_k_" + l);

  auto acc = ctx.acquire_kv_layer(layer);
  if (!acc) return infer::unexpected(acc.error());
  KVLayerAccess &a = **acc;
  if (a.writable.k.empty() || a.readable.k.empty()) return infer::fail(std::errc::invalid_argument);

  AttnParams ap;
  ap.n_head = p.n_head;
  ap.n_head_kv = p.n_head_kv;
  ap.head_dim = p.head_dim;
  ap.scale = 1.0f / std::sqrt(static_cast<float>(p.head_dim));
  ap.causal = true;
  ap.n_ctx = static_cast<uint32_t>(a.n_past);
  ap.sliding_window = 0;

  Tensor *k_cached, *v_cached;
  if (a.pages) {
    // Paged cache: the views span several blocks, so the append and the
    // attention read the pools through the sequence's block table. The
    // logical view keeps the dims [head_dim, n_kv_heads, n_kv, 1].
    Tensor rk = a.readable.k.front().view, rv = a.readable.v.front().view;
    rk.dims[2] = rv.dims[2] = static_cast<int64_t>(a.n_past + a.n_new);
    k_cached = append_kv_paged(g, kr, a.pages, a.pages.k_pool, rk, a.n_past);
    v_cached = append_kv_paged(g, v, a.pages, a.pages.v_pool, rv, a.n_past);
  } else {
    k_cached = append_kv(g, kr, a.writable.k.front().view, a.readable.k.front().view);
    v_cached = append_kv(g, v, a.writable.v.front().view, a.readable.v.front().view);
  }
  return OpFactory::flash_attn(g, qr, k_cached, v_cached, ap, "flash_attn_" + l);
}
