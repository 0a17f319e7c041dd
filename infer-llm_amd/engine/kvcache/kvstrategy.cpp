#include "kvstrategy.hpp"

#include <cstddef>
#include <limits>

infer::expected<KVLayerAccess, std::error_code> KVStrategy::acquire_layer(SequenceId id,
                                                                          std::size_t layer,
                                                                          TokenRange pending) {
  if (!_storage || layer >= _layers.size()) return infer::fail(std::errc::invalid_argument);
  const std::size_t n_past = pending.begin;
  const std::size_t n_new = pending.count;
  if (n_new > std::numeric_limits<std::size_t>::max() - n_past)
    return infer::fail(std::errc::value_too_large);
  const TokenRange read_range{.begin = 0, .count = n_past + n_new};
  auto read_map = lookup(id, layer, read_range);
  if (!read_map) return infer::unexpected(read_map.error());
  auto write_map = lookup(id, layer, pending);
  if (!write_map) return infer::unexpected(write_map.error());

  KVLayerAccess access;
  access._owner = this;
  access.n_past = n_past;
  access.n_new = n_new;
  std::unordered_map<StorageId, KVStorageObject> objects;
  auto readable = make_KVRangeAccess(*read_map, read_range, layer, objects, access);
  if (!readable) {
    (void)release_layer(access);
    return infer::unexpected(readable.error());
  }
  auto writable = make_KVRangeAccess(*write_map, pending, layer, objects, access);
  if (!writable) {
    (void)release_layer(access);
    return infer::unexpected(writable.error());
  }
  access.readable = std::move(*readable);
  access.writable = std::move(*writable);
  if (!objects.empty()) access.backend = objects.begin()->second.backend;
  return access;
}

infer::expected<void, std::error_code> KVStrategy::release_layer(KVLayerAccess &access) noexcept {
  if (!access._owner) return {};  // already released, or moved from
  if (access._owner != this) return infer::fail(std::errc::invalid_argument);
  for (StorageId sid : access._storage_ids) _storage->release_access(sid);
  access._storage_ids.clear();
  access._owner = nullptr;
  access.readable.k.clear();
  access.readable.v.clear();
  access.writable.k.clear();
  access.writable.v.clear();
  access.backend = nullptr;
  access.n_past = access.n_new = 0;
  return {};
}

// Slices -> Tensor views [head_dim, n_kv_heads, count, 1] whose data starts at
// base + token_offset * token_bytes (reference src/kvcache/kvstrategy.cpp:
// 73-168). Each storage object is acquired once per access.
infer::expected<KVRangeAccess, std::error_code> KVStrategy::make_KVRangeAccess(
    const KVMapping &mapping, TokenRange range, std::size_t layer,
    std::unordered_map<StorageId, KVStorageObject> &objects, KVLayerAccess &access) {
  if (!_storage || layer >= _layers.size()) return infer::fail(std::errc::invalid_argument);
  const KVLayerSpec &spec = _layers[layer];
  Backend *backend = objects.empty() ? nullptr : objects.begin()->second.backend;

  auto build = [&](const std::vector<KVSlice> &slices,
                   bool is_k) -> infer::expected<std::vector<KVSegmentView>, std::error_code> {
    const DataType type = is_k ? spec.k_type : spec.v_type;
    const std::size_t head_dim = is_k ? spec.k_head_dim : spec.v_head_dim;
    if (type != GGML_TYPE_F32 && type != GGML_TYPE_F16 && type != GGML_TYPE_BF16 &&
        type != GGML_TYPE_F64)
      return infer::fail(std::errc::not_supported);
    const std::size_t es = dataType_size(type);
    const std::size_t limit = static_cast<std::size_t>(std::numeric_limits<int64_t>::max());
    if (head_dim == 0 || spec.n_kv_heads == 0 || es == 0) return infer::fail(std::errc::invalid_argument);
    if (head_dim > limit / es || spec.n_kv_heads > limit / (head_dim * es))
      return infer::fail(std::errc::value_too_large);
    const std::size_t token_bytes = head_dim * spec.n_kv_heads * es;

    std::vector<KVSegmentView> segments;
    segments.reserve(slices.size());
    std::size_t covered = 0;
    for (const KVSlice &slice : slices) {
      if (slice.storage_id == kInvalidStorageId || slice.token_count == 0 ||
          slice.token_count > range.count - covered)
        return infer::fail(std::errc::invalid_argument);
      auto it = objects.find(slice.storage_id);
      if (it == objects.end()) {
        auto acquired = _storage->acquire(slice.storage_id, layer);
        if (!acquired) return infer::unexpected(acquired.error());
        access._storage_ids.push_back(slice.storage_id);
        it = objects.emplace(slice.storage_id, *acquired).first;
      }
      const KVStorageObject &obj = it->second;
      void *base = is_k ? obj.k_base : obj.v_base;
      if (obj.id != slice.storage_id || !base || !obj.backend ||
          slice.token_offset > obj.capacity_tokens ||
          slice.token_count > obj.capacity_tokens - slice.token_offset)
        return infer::fail(std::errc::invalid_argument);
      if (backend && backend != obj.backend) return infer::fail(std::errc::invalid_argument);
      backend = obj.backend;

      Tensor view(is_k ? "kv_k_view" : "kv_v_view", type,
                  {static_cast<int64_t>(head_dim), static_cast<int64_t>(spec.n_kv_heads),
                   static_cast<int64_t>(slice.token_count), 1});
      view.data = static_cast<std::byte *>(base) + slice.token_offset * token_bytes;
      view.offset = 0;
      view.layer = static_cast<int>(layer);
      view.backend = obj.backend;
      view.device = obj.backend->device_type();
      view.tensorRole = TensorRole::TENSOR_ROLE_KVCACHE;
      segments.push_back(KVSegmentView{.view = std::move(view),
                                       .token_begin = range.begin + covered,
                                       .token_count = slice.token_count});
      covered += slice.token_count;
    }
    if (covered != range.count) return infer::fail(std::errc::invalid_argument);
    return segments;
  };

  auto k = build(mapping.k, true);
  if (!k) return infer::unexpected(k.error());
  auto v = build(mapping.v, false);
  if (!v) return infer::unexpected(v.error());
  return KVRangeAccess{.k = std::move(*k), .v = std::move(*v)};
}

// ---------------------------------------------------------------------------
// ContiguousKVStrategy (reference src/kvcache/KVStrategys/contiguousKVStrategy.cpp)

infer::expected<void, std::error_code> ContiguousKVStrategy::init(
    std::span<const KVLayerSpec> layers, std::span<Backend *const> backend_layer,
    const KVCacheConfig &config) {
  if (!_storage || layers.size() != backend_layer.size() || config.layers != layers.size())
    return infer::fail(std::errc::invalid_argument);
  auto r = _storage->init(layers, backend_layer);
  if (!r) return infer::unexpected(r.error());
  _layers.assign(layers.begin(), layers.end());
  _cfg = config;
  return {};
}

infer::expected<void, std::error_code> ContiguousKVStrategy::create_sequence(SequenceId id) {
  if (id == kInvalidSequenceId) return infer::fail(std::errc::invalid_argument);
  if (_sequences.contains(id)) return infer::fail(std::errc::file_exists);
  std::vector<StorageId> ids;
  ids.reserve(_cfg.layers);
  auto rollback = [&]() noexcept {
    for (StorageId sid : ids) _storage->free(sid);
  };
  for (std::size_t l = 0; l < _cfg.layers; ++l) {
    auto sid = _storage->alloc(l, _cfg.max_tokens_per_sequence);
    if (!sid) {
      rollback();
      return infer::unexpected(sid.error());
    }
    ids.push_back(*sid);
  }
  _sequences.emplace(id, std::move(ids));
  return {};
}

infer::expected<void, std::error_code> ContiguousKVStrategy::reserve_append(SequenceId id,
                                                                           TokenRange range) {
  if (id == kInvalidSequenceId || !_sequences.contains(id))
    return infer::fail(std::errc::invalid_argument);
  // Overflow is an error: no truncation, no sliding window.
  if (!fits(range)) return infer::fail(std::errc::not_enough_memory);
  return {};
}

infer::expected<KVMapping, std::error_code> ContiguousKVStrategy::lookup(SequenceId id,
                                                                         std::size_t layer,
                                                                         TokenRange range) const {
  if (id == kInvalidSequenceId) return infer::fail(std::errc::invalid_argument);
  auto it = _sequences.find(id);
  if (it == _sequences.end() || layer >= it->second.size())
    return infer::fail(std::errc::invalid_argument);
  if (!fits(range)) return infer::fail(std::errc::not_enough_memory);
  if (range.empty()) return KVMapping{};
  const KVSlice slice{.storage_id = it->second[layer], .token_offset = range.begin,
                      .token_count = range.count};
  return KVMapping{.k = {slice}, .v = {slice}};
}

infer::expected<void, std::error_code> ContiguousKVStrategy::commit_append(SequenceId id,
                                                                          TokenRange range) {
  if (!_sequences.contains(id)) return infer::fail(std::errc::invalid_argument);
  if (!fits(range)) return infer::fail(std::errc::not_enough_memory);
  return {};
}

infer::expected<void, std::error_code> ContiguousKVStrategy::abort_append(SequenceId id,
                                                                         TokenRange range) {
  // The rows written by the aborted step stay in memory; they lie beyond the
  // committed length and are overwritten by the next append.
  if (!_sequences.contains(id)) return infer::fail(std::errc::invalid_argument);
  if (!fits(range)) return infer::fail(std::errc::not_enough_memory);
  return {};
}

infer::expected<void, std::error_code> ContiguousKVStrategy::release_sequence(SequenceId id) {
  auto it = _sequences.find(id);
  if (it == _sequences.end()) return infer::fail(std::errc::invalid_argument);
  for (StorageId sid : it->second) _storage->free(sid);
  _sequences.erase(it);
  return {};
}

infer::expected<void, std::error_code> ContiguousKVStrategy::clear_sequence() {
  for (auto &[id, ids] : _sequences)
    for (StorageId sid : ids) _storage->free(sid);
  _sequences.clear();
  return {};
}
