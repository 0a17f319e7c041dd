#include "kvcache_manager.hpp"

infer::expected<void, std::error_code> KVCacheManager::init(std::span<const KVLayerSpec> layers,
                                                            std::span<Backend *const> backend_layer,
                                                            const KVCacheConfig &config) {
  return _strategy->init(layers, backend_layer, config);
}

infer::expected<SequenceId, std::error_code> KVCacheManager::create_sequence() {
  const SequenceId id = _next_sequence_id++;
  auto [it, inserted] = _sequences.try_emplace(id);
  if (!inserted) return infer::fail(std::errc::file_exists);
  auto r = _strategy->create_sequence(id);
  if (!r) {
    _sequences.erase(id);
    return infer::unexpected(r.error());
  }
  return id;
}

infer::expected<void, std::error_code> KVCacheManager::reserve_append(SequenceId id,
                                                                     std::size_t n_tokens) {
  auto it = _sequences.find(id);
  if (it == _sequences.end()) return infer::fail(std::errc::invalid_argument);
  SequenceState &st = it->second;
  if (st.pending) return infer::fail(std::errc::device_or_resource_busy);
  const TokenRange range{.begin = st.committed_length, .count = n_tokens};
  auto r = _strategy->reserve_append(id, range);
  if (!r) return infer::unexpected(r.error());
  st.pending = range;
  return {};
}

infer::expected<KVLayerAccess, std::error_code> KVCacheManager::acquire_layer(SequenceId id,
                                                                              std::size_t layer) {
  auto it = _sequences.find(id);
  if (it == _sequences.end() || !it->second.pending) return infer::fail(std::errc::invalid_argument);
  return _strategy->acquire_layer(id, layer, *it->second.pending);
}

infer::expected<void, std::error_code> KVCacheManager::release_layer(KVLayerAccess &access) noexcept {
  return _strategy->release_layer(access);
}

infer::expected<void, std::error_code> KVCacheManager::commit_append(SequenceId id) {
  auto it = _sequences.find(id);
  if (it == _sequences.end() || !it->second.pending) return infer::fail(std::errc::invalid_argument);
  const TokenRange range = *it->second.pending;
  auto r = _strategy->commit_append(id, range);
  if (!r) return infer::unexpected(r.error());
  it->second.committed_length = range.end();
  it->second.pending.reset();
  return {};
}

infer::expected<void, std::error_code> KVCacheManager::abort_append(SequenceId id) {
  auto it = _sequences.find(id);
  if (it == _sequences.end() || !it->second.pending) return infer::fail(std::errc::invalid_argument);
  auto r = _strategy->abort_append(id, *it->second.pending);
  if (!r) return infer::unexpected(r.error());
  it->second.pending.reset();  // committed_length unchanged
  return {};
}

infer::expected<std::size_t, std::error_code> KVCacheManager::length(SequenceId id) const {
  auto it = _sequences.find(id);
  if (it == _sequences.end()) return infer::fail(std::errc::invalid_argument);
  return it->second.committed_length;
}

infer::expected<void, std::error_code> KVCacheManager::release_sequence(SequenceId id) {
  if (!_sequences.contains(id)) return infer::fail(std::errc::invalid_argument);
  auto r = _strategy->release_sequence(id);
  if (!r) return infer::unexpected(r.error());
  _sequences.erase(id);
  return {};
}

infer::expected<void, std::error_code> KVCacheManager::clear_sequence() {
  auto r = _strategy->clear_sequence();
  if (!r) return infer::unexpected(r.error());
  _sequences.clear();
  return {};
}
