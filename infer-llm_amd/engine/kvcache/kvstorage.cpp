#include "kvstorage.hpp"

#include <cstddef>
#include <limits>

void KVStorage::free(StorageId id) noexcept {
  auto it = _states.find(id);
  if (it == _states.end()) return;
  if (it->second.active_users != 0) {
    it->second.pending_free = true;  // destroyed by the last release_access
    return;
  }
  destroy_object(id);
  _states.erase(id);
}

infer::expected<KVStorageObject, std::error_code> KVStorage::acquire(StorageId id, std::size_t layer) {
  auto it = _states.find(id);
  if (it == _states.end() || it->second.pending_free || it->second.layer != layer ||
      layer >= _backend_layer.size() || !_backend_layer[layer])
    return infer::fail(std::errc::invalid_argument);
  if (it->second.active_users == std::numeric_limits<std::size_t>::max())
    return infer::fail(std::errc::value_too_large);
  if (it->second.active_users == 0) {
    KVObjectAccessRequest req{.id = id, .layer = layer};
    auto prepared = prepare_object(req);
    if (!prepared) return infer::unexpected(prepared.error());
    it = _states.find(id);  // prepare may have touched the table
    if (it == _states.end()) return infer::fail(std::errc::invalid_argument);
  }
  StorageState &st = it->second;
  const KVStorageObject &obj = st.object;
  if (st.pending_free || st.layer != layer || obj.id != id || obj.backend != _backend_layer[layer] ||
      !obj.k_base || !obj.v_base)
    return infer::fail(std::errc::invalid_argument);
  ++st.active_users;
  return obj;
}

void KVStorage::release_access(StorageId id) noexcept {
  auto it = _states.find(id);
  if (it == _states.end() || it->second.active_users == 0) return;
  StorageState &st = it->second;
  --st.active_users;
  if (st.active_users == 0 && st.pending_free) {
    destroy_object(id);
    _states.erase(id);
  }
}

// ---------------------------------------------------------------------------

NaiveKVStorage::~NaiveKVStorage() {
  for (auto &[id, st] : _states)
    if (st.object.backend) st.object.backend->free(BufferKind::KVCACHE, st.object.k_base);
}

infer::expected<void, std::error_code> NaiveKVStorage::init(std::span<const KVLayerSpec> layers,
                                                            std::span<Backend *const> backend_layer) {
  if (layers.size() != backend_layer.size()) return infer::fail(std::errc::invalid_argument);
  _layers.assign(layers.begin(), layers.end());
  _backend_layer.assign(backend_layer.begin(), backend_layer.end());
  return {};
}

infer::expected<StorageId, std::error_code> NaiveKVStorage::alloc(std::size_t layer,
                                                                 std::size_t capacity_tokens) {
  if (layer >= _layers.size()) return infer::fail(std::errc::invalid_argument);
  Backend *backend = _backend_layer[layer];
  if (!backend) return infer::fail(std::errc::invalid_argument);
  const KVLayerSpec &l = _layers[layer];
  const std::size_t k_row = l.n_kv_heads * l.k_head_dim * dataType_size(l.k_type);
  const std::size_t v_row = l.n_kv_heads * l.v_head_dim * dataType_size(l.v_type);
  if (capacity_tokens && (k_row > SIZE_MAX / capacity_tokens || v_row > SIZE_MAX / capacity_tokens))
    return infer::fail(std::errc::value_too_large);
  const std::size_t k_bytes = k_row * capacity_tokens;
  const std::size_t v_bytes = v_row * capacity_tokens;
  auto mem = backend->alloc(BufferKind::KVCACHE, k_bytes + v_bytes);
  if (!mem) return infer::unexpected(mem.error());
  const StorageId id = _next_storage_id++;
  KVStorageObject obj{.id = id,
                      .backend = backend,
                      .capacity_tokens = capacity_tokens,
                      .k_base = *mem,
                      .v_base = static_cast<std::byte *>(*mem) + k_bytes};
  if (!_states.try_emplace(id, StorageState{.object = obj, .layer = layer}).second) {
    backend->free(BufferKind::KVCACHE, *mem);
    return infer::fail(std::errc::file_exists);
  }
  return id;
}

infer::expected<void, std::error_code> NaiveKVStorage::prepare_object(const KVObjectAccessRequest &req) {
  // Objects are allocated on their layer's backend; nothing moves.
  if (req.layer >= _layers.size() || !_states.contains(req.id))
    return infer::fail(std::errc::invalid_argument);
  return {};
}

void NaiveKVStorage::destroy_object(StorageId id) noexcept {
  auto it = _states.find(id);
  if (it == _states.end()) return;
  Backend *backend = _backend_layer[it->second.layer];
  if (backend) backend->free(BufferKind::KVCACHE, it->second.object.k_base);
}
