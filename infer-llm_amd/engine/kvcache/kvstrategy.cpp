#include "kvstrategy.hpp"

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <limits>
#include <string>

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

  // Per object, in its own rows: the rows written (the pending slices) and the
  // history read before them (the readable slices up to the first written row).
  std::unordered_map<StorageId, KVObjectAccessRequest> requests;
  std::unordered_map<StorageId, std::size_t> read_end;
  for (const auto *slices : {&read_map->k, &read_map->v})
    for (const KVSlice &sl : *slices) {
      std::size_t &e = read_end[sl.storage_id];
      e = std::max(e, sl.token_offset + sl.token_count);
    }
  for (const auto *slices : {&write_map->k, &write_map->v})
    for (const KVSlice &sl : *slices) {
      auto [it, fresh] = requests.try_emplace(sl.storage_id, KVObjectAccessRequest{.id = sl.storage_id,
                                                                                  .layer = layer,
                                                                                  .ranges_known = true});
      TokenRange &w = it->second.writable;
      const std::size_t b = fresh ? sl.token_offset : std::min(w.begin, sl.token_offset);
      const std::size_t e = fresh ? sl.token_offset + sl.token_count
                                  : std::max(w.end(), sl.token_offset + sl.token_count);
      w = TokenRange{.begin = b, .count = e - b};
    }
  for (const auto &[sid, e] : read_end) {
    auto [it, fresh] = requests.try_emplace(sid, KVObjectAccessRequest{.id = sid, .layer = layer,
                                                                       .ranges_known = true});
    it->second.history_tokens = fresh ? e : std::min(e, it->second.writable.begin);
  }

  KVLayerAccess access;
  access._owner = this;
  access.n_past = n_past;
  access.n_new = n_new;
  std::unordered_map<StorageId, KVStorageObject> objects;
  auto readable = make_KVRangeAccess(*read_map, read_range, layer, objects, access, &requests);
  if (!readable) {
    (void)release_layer(access);
    return infer::unexpected(readable.error());
  }
  auto writable = make_KVRangeAccess(*write_map, pending, layer, objects, access, &requests);
  if (!writable) {
    (void)release_layer(access);
    return infer::unexpected(writable.error());
  }
  access.readable = std::move(*readable);
  access.writable = std::move(*writable);
  if (!objects.empty()) access.backend = objects.begin()->second.backend;
  describe(access, id, layer);
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
  access.pages = KVPages{};
  return {};
}

// Slices -> Tensor views [head_dim, n_kv_heads, count, 1] whose data starts at
// base + token_offset * token_bytes (reference src/kvcache/kvstrategy.cpp:
// 73-168). Each storage object is acquired once per access.
infer::expected<KVRangeAccess, std::error_code> KVStrategy::make_KVRangeAccess(
    const KVMapping &mapping, TokenRange range, std::size_t layer,
    std::unordered_map<StorageId, KVStorageObject> &objects, KVLayerAccess &access,
    const std::unordered_map<StorageId, KVObjectAccessRequest> *requests) {
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
        const KVObjectAccessRequest *req = nullptr;
        if (requests) {
          auto r = requests->find(slice.storage_id);
          if (r != requests->end()) req = &r->second;
        }
        auto acquired = _storage->acquire(slice.storage_id, layer, req);
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

// ---------------------------------------------------------------------------
// PagedKVStrategy

PagedKVStrategy::PagedKVStrategy(std::unique_ptr<BlockPoolKVStorage> storage) noexcept
    : KVStrategy(std::move(storage)) {
  _pool = static_cast<BlockPoolKVStorage *>(_storage.get());
}

PagedKVStrategy::~PagedKVStrategy() {
  for (auto &[id, layers] : _sequences) drop(layers);
}

void PagedKVStrategy::drop(std::vector<Layer> &layers) noexcept {
  for (std::size_t l = 0; l < layers.size(); ++l) {
    for (StorageId sid : layers[l].blocks) _storage->free(sid);
    layers[l].blocks.clear();
    if (layers[l].device_table && layers[l].device_table->data && l < _backend_layer.size())
      _backend_layer[l]->free(BufferKind::KVCACHE, layers[l].device_table->data);
    layers[l].device_table.reset();
  }
}

infer::expected<void, std::error_code> PagedKVStrategy::init(std::span<const KVLayerSpec> layers,
                                                            std::span<Backend *const> backend_layer,
                                                            const KVCacheConfig &config) {
  if (!_pool || layers.size() != backend_layer.size() || config.layers != layers.size() ||
      config.block_tokens == 0 || config.block_tokens != _pool->block_tokens() ||
      config.max_tokens_per_sequence == 0)
    return infer::fail(std::errc::invalid_argument);
  const std::size_t max_blocks =
      (config.max_tokens_per_sequence + config.block_tokens - 1) / config.block_tokens;
  if (max_blocks > static_cast<std::size_t>(INT32_MAX)) return infer::fail(std::errc::value_too_large);
  auto r = _storage->init(layers, backend_layer);
  if (!r) return infer::unexpected(r.error());
  _layers.assign(layers.begin(), layers.end());
  _backend_layer.assign(backend_layer.begin(), backend_layer.end());
  _cfg = config;
  _max_blocks = max_blocks;
  return {};
}

infer::expected<void, std::error_code> PagedKVStrategy::create_sequence(SequenceId id) {
  if (id == kInvalidSequenceId) return infer::fail(std::errc::invalid_argument);
  if (_sequences.contains(id)) return infer::fail(std::errc::file_exists);
  std::vector<Layer> layers(_cfg.layers);
  for (std::size_t l = 0; l < _cfg.layers; ++l) {
    Backend *backend = _backend_layer[l];
    auto mem = backend->alloc(BufferKind::KVCACHE, _max_blocks * sizeof(int32_t));
    if (!mem) {
      drop(layers);
      return infer::unexpected(mem.error());
    }
    auto t = std::make_unique<Tensor>("kv_block_table_" + std::to_string(l), GGML_TYPE_I32,
                                      std::initializer_list<int64_t>{static_cast<int64_t>(_max_blocks)});
    t->data = *mem;
    t->backend = backend;
    t->device = backend->device_type();
    t->tensorRole = TensorRole::TENSOR_ROLE_KVCACHE;
    layers[l].device_table = std::move(t);
  }
  _sequences.emplace(id, std::move(layers));
  return {};
}

infer::expected<void, std::error_code> PagedKVStrategy::reserve_append(SequenceId id,
                                                                      TokenRange range) {
  auto it = _sequences.find(id);
  if (id == kInvalidSequenceId || it == _sequences.end()) return infer::fail(std::errc::invalid_argument);
  if (!fits(range)) return infer::fail(std::errc::not_enough_memory);
  const std::size_t bt = _cfg.block_tokens;
  const std::size_t need = (range.end() + bt - 1) / bt;
  std::vector<Layer> &layers = it->second;
  // Take every new block first, so that running out of pool leaves the
  // sequence as it was.
  std::vector<std::vector<StorageId>> fresh(layers.size());
  auto undo = [&]() noexcept {
    for (auto &v : fresh)
      for (StorageId sid : v) _storage->free(sid);
  };
  for (std::size_t l = 0; l < layers.size(); ++l) {
    for (std::size_t b = layers[l].blocks.size(); b < need; ++b) {
      auto sid = _pool->alloc(l, bt);
      if (!sid) {
        undo();
        return infer::unexpected(sid.error());
      }
      fresh[l].push_back(*sid);
    }
  }
  for (std::size_t l = 0; l < layers.size(); ++l) {
    if (fresh[l].empty()) continue;
    Layer &L = layers[l];
    const std::size_t first = L.blocks.size();
    for (StorageId sid : fresh[l]) {
      L.blocks.push_back(sid);
      L.table.push_back(static_cast<int32_t>(_pool->block_of(sid)));
    }
    auto up = _backend_layer[l]->copy_tensor_set(L.device_table.get(), L.table.data() + first,
                                                 first * sizeof(int32_t),
                                                 fresh[l].size() * sizeof(int32_t));
    if (!up) return infer::unexpected(up.error());
  }
  return {};
}

infer::expected<KVMapping, std::error_code> PagedKVStrategy::lookup(SequenceId id,
                                                                   std::size_t layer,
                                                                   TokenRange range) const {
  if (id == kInvalidSequenceId) return infer::fail(std::errc::invalid_argument);
  auto it = _sequences.find(id);
  if (it == _sequences.end() || layer >= it->second.size())
    return infer::fail(std::errc::invalid_argument);
  if (!fits(range)) return infer::fail(std::errc::not_enough_memory);
  KVMapping m;
  if (range.empty()) return m;
  const std::size_t bt = _cfg.block_tokens;
  const auto &blocks = it->second[layer].blocks;
  if ((range.end() + bt - 1) / bt > blocks.size()) return infer::fail(std::errc::invalid_argument);
  for (std::size_t t = range.begin; t < range.end();) {
    const std::size_t b = t / bt, off = t - b * bt;
    const std::size_t n = std::min(bt - off, range.end() - t);
    const KVSlice slice{.storage_id = blocks[b], .token_offset = off, .token_count = n};
    m.k.push_back(slice);
    m.v.push_back(slice);
    t += n;
  }
  return m;
}

void PagedKVStrategy::describe(KVLayerAccess &access, SequenceId id, std::size_t layer) const {
  auto it = _sequences.find(id);
  if (it == _sequences.end() || layer >= it->second.size()) return;
  access.pages = KVPages{.block_table = it->second[layer].device_table.get(),
                         .block_tokens = _cfg.block_tokens,
                         .pool_blocks = _pool->blocks_per_layer(),
                         .k_pool = _pool->k_pool(layer),
                         .v_pool = _pool->v_pool(layer)};
}

infer::expected<void, std::error_code> PagedKVStrategy::commit_append(SequenceId id,
                                                                     TokenRange range) {
  if (!_sequences.contains(id)) return infer::fail(std::errc::invalid_argument);
  if (!fits(range)) return infer::fail(std::errc::not_enough_memory);
  return {};
}

infer::expected<void, std::error_code> PagedKVStrategy::abort_append(SequenceId id,
                                                                    TokenRange range) {
  auto it = _sequences.find(id);
  if (it == _sequences.end()) return infer::fail(std::errc::invalid_argument);
  if (!fits(range)) return infer::fail(std::errc::not_enough_memory);
  // Blocks past the one holding the last committed token go back to the pool
  // (an object still in use is returned by its last release).
  const std::size_t bt = _cfg.block_tokens;
  const std::size_t keep = (range.begin + bt - 1) / bt;
  for (Layer &L : it->second) {
    while (L.blocks.size() > keep) {
      _storage->free(L.blocks.back());
      L.blocks.pop_back();
      L.table.pop_back();
    }
  }
  return {};
}

infer::expected<void, std::error_code> PagedKVStrategy::release_sequence(SequenceId id) {
  auto it = _sequences.find(id);
  if (it == _sequences.end()) return infer::fail(std::errc::invalid_argument);
  drop(it->second);
  _sequences.erase(it);
  return {};
}

infer::expected<void, std::error_code> PagedKVStrategy::clear_sequence() {
  for (auto &[id, layers] : _sequences) drop(layers);
  _sequences.clear();
  return {};
}

std::vector<int64_t> PagedKVStrategy::blocks(SequenceId id, std::size_t layer) const {
  std::vector<int64_t> out;
  auto it = _sequences.find(id);
  if (it == _sequences.end() || layer >= it->second.size()) return out;
  for (StorageId sid : it->second[layer].blocks) out.push_back(_pool->block_of(sid));
  return out;
}

