#include "graph.hpp"

#include <cmath>
#include <new>

#include "../../include/ikv.h"

#include "kvcache/kvcache_manager.hpp"

Tensor *Graph::add_node(std::unique_ptr<Tensor> t) {
  Tensor *raw = t.get();
  _owned.push_back(std::move(t));
  _dirty = true;
  return raw;
}

Tensor *Graph::adopt(std::unique_ptr<Tensor> t) {
  Tensor *raw = t.get();
  _owned.push_back(std::move(t));
  return raw;
}

infer::expected<void, std::error_code> Graph::compute() {
  if (_outputs.empty()) return infer::fail(std::errc::invalid_argument);
  if (_dirty || _nodes.empty()) {
    _visited.clear();
    _nodes.clear();
    _leafs.clear();
    for (Tensor *out : _outputs) build_topo_order(out);
    _dirty = false;
  }
  for (Tensor *leaf : _leafs)
    if (!leaf->data) return infer::fail(std::errc::invalid_argument);
  return {};
}

void Graph::build_topo_order(Tensor *t) {
  if (!t || !_visited.insert(t).second) return;
  for (Tensor *s : t->src) {
    if (!s) break;
    build_topo_order(s);
  }
  (t->op == OperationType::GGML_OP_NONE ? _leafs : _nodes).push_back(t);
}

// ---------------------------------------------------------------------------

infer::expected<Tensor *, std::error_code> GraphContext::get_rope_theta_table(float theta_base,
                                                                              uint32_t head_dim,
                                                                              uint32_t n_ctx) {
  const RopeKey key{theta_base, head_dim, n_ctx};
  if (auto it = _rope_theta_cache.find(key); it != _rope_theta_cache.end()) return it->second;
  const uint32_t half = head_dim / 2;
  Tensor *t = make_tensor("rope_theta", GGML_TYPE_F32, {half, n_ctx, 1, 1});
  t->backend = _host_backend;
  t->device = DeviceType::CPU;
  std::unique_ptr<float[]> buf(new (std::nothrow) float[static_cast<size_t>(half) * n_ctx]);
  if (!buf) return infer::fail(std::errc::not_enough_memory);
  // freq_i = 1 / theta^(2i/d) evaluated in float (the exponent 2i/d too),
  // widened to double; angle = float(double(pos) * freq_i)
  if (ikv_rope_theta_table_f32(theta_base, int(head_dim), n_ctx, buf.get()) != 0)
    return infer::fail(std::errc::invalid_argument);
  t->data = buf.get();
  _rope_buffers.push_back(std::move(buf));
  _rope_theta_cache[key] = t;
  return t;
}

Tensor *GraphContext::make_tensor(std::string name, DataType type,
                                  std::initializer_list<int64_t> shape) {
  _owned.push_back(std::make_unique<Tensor>(name, type, shape));
  return _owned.back().get();
}

infer::expected<void, std::error_code> GraphContext::set_kv_cache(KVCacheManager *kv,
                                                                  SequenceId id) noexcept {
  if (!_kv_accesses.empty() && (kv != _kv_manager || id != _sequence_id))
    return infer::fail(std::errc::device_or_resource_busy);
  _kv_manager = kv;
  _sequence_id = id;
  return {};
}

infer::expected<void, std::error_code> GraphContext::release_kv_access() {
  if (_kv_accesses.empty()) return {};
  if (!_kv_manager) return infer::fail(std::errc::invalid_argument);
  for (KVLayerAccess &a : _kv_accesses) {
    auto r = _kv_manager->release_layer(a);
    if (!r) return r;
  }
  _kv_accesses.clear();
  return {};
}

infer::expected<KVLayerAccess *, std::error_code> GraphContext::acquire_kv_layer(std::size_t layer) {
  if (!_kv_manager) return infer::fail(std::errc::invalid_argument);
  auto r = _kv_manager->acquire_layer(_sequence_id, layer);
  if (!r) return infer::unexpected(r.error());
  _kv_accesses.push_back(std::move(*r));
  return &_kv_accesses.back();
}
