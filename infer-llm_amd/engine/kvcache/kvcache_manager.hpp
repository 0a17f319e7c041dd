// kvcache_manager.hpp — per-sequence append transactions over a strategy
// (reference include/kvcache/kvcacheManager.hpp:19-72,
// src/kvcache/kvcacheManager.cpp:9-142).
//
//   reserve_append(id, n)  pending = {committed, n}; busy if one is pending;
//                          not_enough_memory beyond capacity
//   acquire_layer(id, l)   views for the pending step (invalid_argument
//                          without a pending reserve)
//   release_layer(access)  hand the access back once kernels are done
//   commit_append(id)      committed = pending.end()
//   abort_append(id)       drop the pending range; committed unchanged
#pragma once

#include <memory>
#include <optional>
#include <span>
#include <system_error>
#include <unordered_map>

#include "../expected.hpp"
#include "kvstrategy.hpp"
#include "kvutil.hpp"

struct SequenceState {
  std::size_t committed_length = 0;
  std::optional<TokenRange> pending;
};

class KVCacheManager {
 public:
  explicit KVCacheManager(std::unique_ptr<KVStrategy> strategy) noexcept
      : _strategy(std::move(strategy)) {}
  KVCacheManager(const KVCacheManager &) = delete;
  KVCacheManager &operator=(const KVCacheManager &) = delete;

  infer::expected<void, std::error_code> init(std::span<const KVLayerSpec> layers,
                                              std::span<Backend *const> backend_layer,
                                              const KVCacheConfig &config);
  infer::expected<SequenceId, std::error_code> create_sequence();
  infer::expected<void, std::error_code> reserve_append(SequenceId id, std::size_t n_tokens);
  infer::expected<KVLayerAccess, std::error_code> acquire_layer(SequenceId id, std::size_t layer);
  infer::expected<void, std::error_code> release_layer(KVLayerAccess &access) noexcept;
  infer::expected<void, std::error_code> commit_append(SequenceId id);
  infer::expected<void, std::error_code> abort_append(SequenceId id);
  infer::expected<std::size_t, std::error_code> length(SequenceId id) const;
  infer::expected<void, std::error_code> release_sequence(SequenceId id);
  infer::expected<void, std::error_code> clear_sequence();

  KVStrategy *strategy() const { return _strategy.get(); }

 private:
  std::unique_ptr<KVStrategy> _strategy;
  std::unordered_map<SequenceId, SequenceState> _sequences;
  SequenceId _next_sequence_id = 1;
};
