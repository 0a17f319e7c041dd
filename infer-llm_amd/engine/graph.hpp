// graph.hpp — compute graph and per-step context (reference
// include/graph.hpp:16-152, src/graph.cpp:1-197).
//
// Graph owns its node tensors; compute() orders the internal nodes by a DFS
// post-order from the outputs (leaves: weights, inputs, KV views). The
// context owns the step's input tensors, the RoPE angle tables and the KV
// accesses of the step.
#pragma once

#include <cstdint>
#include <deque>
#include <initializer_list>
#include <memory>
#include <string>
#include <system_error>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "expected.hpp"
#include "kvcache/kvutil.hpp"
#include "tensor.hpp"

class KVCacheManager;

class Graph {
 public:
  Graph() = default;
  Graph(Graph &&) = default;
  Graph &operator=(Graph &&) = default;

  Tensor *add_node(std::unique_ptr<Tensor> t);
  // Ownership only (boundary copies): not a node, not ordered, not executed.
  Tensor *adopt(std::unique_ptr<Tensor> t);
  void mark_input(Tensor *t) { _inputs.push_back(t); }
  void mark_output(Tensor *t) { _outputs.push_back(t); }

  // Builds the topological order (when the graph changed) and checks that
  // every leaf has data.
  infer::expected<void, std::error_code> compute();

  const std::vector<Tensor *> &inputs() const { return _inputs; }
  const std::vector<Tensor *> &outputs() const { return _outputs; }
  const std::vector<Tensor *> &nodes() const { return _nodes; }
  const std::vector<Tensor *> &leafs() const { return _leafs; }

 private:
  void build_topo_order(Tensor *t);

  bool _dirty = false;
  std::vector<std::unique_ptr<Tensor>> _owned;
  std::vector<Tensor *> _inputs, _outputs, _nodes, _leafs;
  std::unordered_set<Tensor *> _visited;
};

class GraphContext {
 public:
  GraphContext() = default;
  // host_backend, when given, is recorded as the owner of host tensors.
  explicit GraphContext(Backend *host_backend) : _host_backend(host_backend) {}
  GraphContext(const GraphContext &) = delete;
  GraphContext &operator=(const GraphContext &) = delete;

  void set_input_tokens(Tensor *t) { _inp_tokens = t; }
  void set_input_pos(Tensor *t) { _inp_pos = t; }
  Tensor *get_input_tokens() const { return _inp_tokens; }
  Tensor *get_input_pos() const { return _inp_pos; }

  // Host table [head_dim/2, n_ctx] of angles pos * theta^(-2i/head_dim),
  // cached per (theta_base, head_dim, n_ctx) (reference src/graph.cpp:92-135).
  infer::expected<Tensor *, std::error_code> get_rope_theta_table(float theta_base, uint32_t head_dim,
                                                                  uint32_t n_ctx);
  Tensor *make_tensor(std::string name, DataType type, std::initializer_list<int64_t> shape);

  // No switching manager or sequence while accesses are outstanding.
  infer::expected<void, std::error_code> set_kv_cache(KVCacheManager *kv, SequenceId id) noexcept;
  infer::expected<void, std::error_code> release_kv_access();
  // The returned pointer stays valid until release_kv_access().
  infer::expected<KVLayerAccess *, std::error_code> acquire_kv_layer(std::size_t layer);
  std::size_t outstanding_kv_accesses() const { return _kv_accesses.size(); }

 private:
  Backend *_host_backend = nullptr;
  Tensor *_inp_tokens = nullptr;
  Tensor *_inp_pos = nullptr;
  struct RopeKey {
    float theta_base;
    uint32_t head_dim, n_ctx;
    bool operator==(const RopeKey &o) const noexcept {
      return theta_base == o.theta_base && head_dim == o.head_dim && n_ctx == o.n_ctx;
    }
  };
  struct RopeKeyHash {
    size_t operator()(const RopeKey &k) const noexcept {
      size_t h = std::hash<float>{}(k.theta_base);
      h = h * 1000003u ^ k.head_dim;
      return h * 1000003u ^ k.n_ctx;
    }
  };
  std::unordered_map<RopeKey, Tensor *, RopeKeyHash> _rope_theta_cache;
  std::vector<std::unique_ptr<Tensor>> _owned;
  std::vector<std::unique_ptr<float[]>> _rope_buffers;
  KVCacheManager *_kv_manager = nullptr;
  std::deque<KVLayerAccess> _kv_accesses;  // deque: pointers stay valid on growth
  SequenceId _sequence_id = kInvalidSequenceId;
};
