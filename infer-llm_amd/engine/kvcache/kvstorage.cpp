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

infer::expected<KVStorageObject, std::error_code> KVStorage::acquire(StorageId id, std::size_t layer,
                                                                   const KVObjectAccessRequest *request) {
  auto it = _states.find(id);
  if (it == _states.end() || it->second.pending_free || it->second.layer != layer ||
      layer >= _backend_layer.size() || !_backend_layer[layer])
    return infer::fail(std::errc::invalid_argument);
  if (request && (request->id != id || request->layer != layer)) return infer::fail(std::errc::invalid_argument);
  const KVObjectAccessRequest req = request ? *request : KVObjectAccessRequest{.id = id, .layer = layer};
  if (it->second.active_users == std::numeric_limits<std::size_t>::max())
    return infer::fail(std::errc::value_too_large);
  if (it->second.active_users == 0) {
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
  record_access(req);
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

// ---------------------------------------------------------------------------

BlockPoolKVStorage::~BlockPoolKVStorage() {
  for (std::size_t l = 0; l < _pools.size(); ++l)
    if (_pools[l].base && _backend_layer[l]) _backend_layer[l]->free(BufferKind::KVCACHE, _pools[l].base);
}

infer::expected<void, std::error_code> BlockPoolKVStorage::init(
    std::span<const KVLayerSpec> layers, std::span<Backend *const> backend_layer) {
  if (layers.size() != backend_layer.size() || !_pools.empty() || _blocks == 0 ||
      _block_tokens == 0)
    return infer::fail(std::errc::invalid_argument);
  _layers.assign(layers.begin(), layers.end());
  _backend_layer.assign(backend_layer.begin(), backend_layer.end());
  _pools.resize(layers.size());
  for (std::size_t l = 0; l < layers.size(); ++l) {
    Backend *backend = _backend_layer[l];
    if (!backend) return infer::fail(std::errc::invalid_argument);
    const KVLayerSpec &sp = _layers[l];
    const std::size_t k_row = sp.n_kv_heads * sp.k_head_dim * dataType_size(sp.k_type);
    const std::size_t v_row = sp.n_kv_heads * sp.v_head_dim * dataType_size(sp.v_type);
    const std::size_t rows = _blocks * _block_tokens;
    if (rows / _blocks != _block_tokens || (k_row && rows > SIZE_MAX / 2 / k_row) ||
        (v_row && rows > SIZE_MAX / 2 / v_row))
      return infer::fail(std::errc::value_too_large);
    Pool &p = _pools[l];
    p.k_block_bytes = k_row * _block_tokens;
    p.v_block_bytes = v_row * _block_tokens;
    auto mem = backend->alloc(BufferKind::KVCACHE, (p.k_block_bytes + p.v_block_bytes) * _blocks);
    if (!mem) return infer::unexpected(mem.error());
    p.base = *mem;
    p.k = p.base;
    p.v = static_cast<std::byte *>(p.base) + p.k_block_bytes * _blocks;
    p.free.resize(_blocks);
    // handed out from the back: block 0 first
    for (std::size_t b = 0; b < _blocks; ++b) p.free[b] = _blocks - 1 - b;
  }
  return {};
}

infer::expected<StorageId, std::error_code> BlockPoolKVStorage::alloc(std::size_t layer,
                                                                     std::size_t capacity_tokens) {
  if (layer >= _pools.size() || capacity_tokens != _block_tokens)
    return infer::fail(std::errc::invalid_argument);
  Pool &p = _pools[layer];
  if (p.free.empty()) return infer::fail(std::errc::not_enough_memory);
  const std::size_t b = p.free.back();
  const StorageId id = _next_storage_id++;
  KVStorageObject obj{.id = id,
                      .backend = _backend_layer[layer],
                      .capacity_tokens = _block_tokens,
                      .k_base = static_cast<std::byte *>(p.k) + b * p.k_block_bytes,
                      .v_base = static_cast<std::byte *>(p.v) + b * p.v_block_bytes};
  if (!_states.try_emplace(id, StorageState{.object = obj, .layer = layer}).second)
    return infer::fail(std::errc::file_exists);
  p.free.pop_back();
  _block.emplace(id, b);
  return id;
}

int64_t BlockPoolKVStorage::block_of(StorageId id) const {
  auto it = _block.find(id);
  return it == _block.end() ? -1 : static_cast<int64_t>(it->second);
}

infer::expected<void, std::error_code> BlockPoolKVStorage::prepare_object(
    const KVObjectAccessRequest &req) {
  if (req.layer >= _pools.size() || !_states.contains(req.id))
    return infer::fail(std::errc::invalid_argument);
  return {};
}

void BlockPoolKVStorage::destroy_object(StorageId id) noexcept {
  auto st = _states.find(id);
  auto it = _block.find(id);
  if (st == _states.end() || it == _block.end()) return;
  _pools[st->second.layer].free.push_back(it->second);
  _block.erase(it);
}
