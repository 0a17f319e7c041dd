// kvstrategy.hpp — token -> storage mapping and the guarded layer views
// (reference include/kvcache/kvstrategy.hpp:29-77, src/kvcache/kvstrategy.cpp
// and src/kvcache/KVStrategys/contiguousKVStrategy.cpp).
//
// Contract (as in the reference): sequence lengths and the pending append are
// owned by KVCacheManager; strategy methods take explicit TokenRanges;
// lookup() sees ranges reserved but not yet committed; one uncommitted
// append per sequence at a time.
#pragma once

#include <memory>
#include <span>
#include <system_error>
#include <unordered_map>
#include <vector>

#include "../expected.hpp"
#include "kvstorage.hpp"
#include "kvutil.hpp"

class KVStrategy {
 public:
  explicit KVStrategy(std::unique_ptr<KVStorage> storage) noexcept : _storage(std::move(storage)) {}
  virtual ~KVStrategy() = default;
  KVStrategy(const KVStrategy &) = delete;
  KVStrategy &operator=(const KVStrategy &) = delete;

  virtual infer::expected<void, std::error_code> init(std::span<const KVLayerSpec> layers,
                                                      std::span<Backend *const> backend_layer,
                                                      const KVCacheConfig &config) = 0;
  virtual infer::expected<void, std::error_code> create_sequence(SequenceId id) = 0;
  virtual infer::expected<void, std::error_code> reserve_append(SequenceId id, TokenRange range) = 0;

  // Readable view [0, pending.end()) and writable view `pending`, each
  // storage object acquired once (reference src/kvcache/kvstrategy.cpp:7-55).
  infer::expected<KVLayerAccess, std::error_code> acquire_layer(SequenceId id, std::size_t layer,
                                                                TokenRange pending);
  infer::expected<void, std::error_code> release_layer(KVLayerAccess &access) noexcept;

  virtual infer::expected<void, std::error_code> commit_append(SequenceId id, TokenRange range) = 0;
  virtual infer::expected<void, std::error_code> abort_append(SequenceId id, TokenRange range) = 0;
  virtual infer::expected<void, std::error_code> release_sequence(SequenceId id) = 0;
  virtual infer::expected<void, std::error_code> clear_sequence() = 0;

  KVStorage *storage() const { return _storage.get(); }

 protected:
  // Lets a strategy attach what its kernels need beyond the views (a paged
  // strategy's block table) to an access it has built.
  virtual void describe(KVLayerAccess &, SequenceId, std::size_t) const {}

  virtual infer::expected<KVMapping, std::error_code> lookup(SequenceId id, std::size_t layer,
                                                             TokenRange range) const = 0;
  // requests: per object, the rows this access reads and writes (passed to
  // the storage's acquire; NULL or a missing entry: unknown).
  infer::expected<KVRangeAccess, std::error_code> make_KVRangeAccess(
      const KVMapping &mapping, TokenRange range, std::size_t layer,
      std::unordered_map<StorageId, KVStorageObject> &objects, KVLayerAccess &access,
      const std::unordered_map<StorageId, KVObjectAccessRequest> *requests = nullptr);

  std::unique_ptr<KVStorage> _storage;
  std::vector<KVLayerSpec> _layers;
  KVCacheConfig _cfg = {};
};

// One storage object per (sequence, layer) of max_tokens_per_sequence tokens;
// a token's offset in it is its absolute position.
class ContiguousKVStrategy : public KVStrategy {
 public:
  explicit ContiguousKVStrategy(std::unique_ptr<KVStorage> storage) noexcept
      : KVStrategy(std::move(storage)) {}

  infer::expected<void, std::error_code> init(std::span<const KVLayerSpec> layers,
                                              std::span<Backend *const> backend_layer,
                                              const KVCacheConfig &config) override;
  infer::expected<void, std::error_code> create_sequence(SequenceId id) override;
  infer::expected<void, std::error_code> reserve_append(SequenceId id, TokenRange range) override;
  infer::expected<void, std::error_code> commit_append(SequenceId id, TokenRange range) override;
  infer::expected<void, std::error_code> abort_append(SequenceId id, TokenRange range) override;
  infer::expected<void, std::error_code> release_sequence(SequenceId id) override;
  infer::expected<void, std::error_code> clear_sequence() override;

 protected:
  infer::expected<KVMapping, std::error_code> lookup(SequenceId id, std::size_t layer,
                                                     TokenRange range) const override;

 private:
  bool fits(TokenRange r) const {
    const auto cap = _cfg.max_tokens_per_sequence;
    return r.begin <= cap && r.count <= cap - r.begin;
  }
  std::unordered_map<SequenceId, std::vector<StorageId>> _sequences;  // index = layer
};

// Paged strategy (KVCacheConfig::block_tokens > 0) over a BlockPoolKVStorage:
// a sequence's layer is a list of pool blocks, grown by reserve_append,
// trimmed by abort_append to the blocks that hold committed tokens, and
// returned by release_sequence. lookup() yields one slice per block touched,
// and every access carries the sequence's device block table (one int32 per
// block, kept on the layer's backend and updated only when blocks are added),
// so the attention kernels follow the blocks without a per-step upload.
class PagedKVStrategy : public KVStrategy {
 public:
  explicit PagedKVStrategy(std::unique_ptr<BlockPoolKVStorage> storage) noexcept;
  ~PagedKVStrategy() override;

  infer::expected<void, std::error_code> init(std::span<const KVLayerSpec> layers,
                                              std::span<Backend *const> backend_layer,
                                              const KVCacheConfig &config) override;
  infer::expected<void, std::error_code> create_sequence(SequenceId id) override;
  infer::expected<void, std::error_code> reserve_append(SequenceId id, TokenRange range) override;
  infer::expected<void, std::error_code> commit_append(SequenceId id, TokenRange range) override;
  infer::expected<void, std::error_code> abort_append(SequenceId id, TokenRange range) override;
  infer::expected<void, std::error_code> release_sequence(SequenceId id) override;
  infer::expected<void, std::error_code> clear_sequence() override;

  // Pool blocks of (sequence, layer), in token order (tests, tools).
  std::vector<int64_t> blocks(SequenceId id, std::size_t layer) const;

 protected:
  infer::expected<KVMapping, std::error_code> lookup(SequenceId id, std::size_t layer,
                                                     TokenRange range) const override;
  void describe(KVLayerAccess &access, SequenceId id, std::size_t layer) const override;

 private:
  struct Layer {
    std::vector<StorageId> blocks;
    std::vector<int32_t> table;            // host mirror of the device table
    std::unique_ptr<Tensor> device_table;  // I32 [max_blocks] on the layer's backend
  };
  bool fits(TokenRange r) const {
    const auto cap = _cfg.max_tokens_per_sequence;
    return r.begin <= cap && r.count <= cap - r.begin;
  }
  void drop(std::vector<Layer> &layers) noexcept;

  BlockPoolKVStorage *_pool;
  std::vector<Backend *> _backend_layer;
  std::size_t _max_blocks = 0;
  std::unordered_map<SequenceId, std::vector<Layer>> _sequences;
};

