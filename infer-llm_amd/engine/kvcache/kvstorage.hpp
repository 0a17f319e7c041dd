// kvstorage.hpp — physical KV objects and their use counts (reference
// include/kvcache/kvstorage.hpp:39-76, src/kvcache/kvstorage.cpp:5-57).
//
// The base class owns the object table: acquire() prepares an object for its
// layer's backend and counts an active user; release_access() drops it; free()
// defers destruction while users remain. Derived storages allocate and
// destroy the memory.
#pragma once

#include <cstddef>
#include <span>
#include <system_error>
#include <unordered_map>
#include <vector>

#include "../backend.hpp"
#include "../expected.hpp"
#include "kvutil.hpp"

// What one access does with an object, in the object's own token rows:
// reads rows [0, history_tokens) written by earlier accesses, and writes
// rows `writable`. ranges_known false: unknown (treated as any row read or
// written).
struct KVObjectAccessRequest {
  StorageId id = kInvalidStorageId;
  std::size_t layer = 0;
  std::size_t history_tokens = 0;
  TokenRange writable;
  bool ranges_known = false;
};

struct KVStorageObject {
  StorageId id = kInvalidStorageId;
  Backend *backend = nullptr;
  std::size_t capacity_tokens = 0;
  void *k_base = nullptr;
  void *v_base = nullptr;
};

// active_users counts outstanding accesses, not ownership.
struct StorageState {
  KVStorageObject object;
  std::size_t layer = 0;
  std::size_t active_users = 0;
  bool pending_free = false;
};

class KVStorage {
 public:
  virtual ~KVStorage() = default;

  virtual infer::expected<void, std::error_code> init(std::span<const KVLayerSpec> layers,
                                                      std::span<Backend *const> backend_layer) = 0;
  // Allocates one object for `layer`; ids are never reused by one storage.
  virtual infer::expected<StorageId, std::error_code> alloc(std::size_t layer,
                                                           std::size_t capacity_tokens) = 0;
  // Gives up ownership: destroyed now, or when the last user releases it.
  void free(StorageId id) noexcept;
  // Prepares the object for its layer's backend; on success active_users++.
  // request, if not NULL, says which rows this access reads and writes (its
  // id and layer must match).
  infer::expected<KVStorageObject, std::error_code> acquire(StorageId id, std::size_t layer,
                                                          const KVObjectAccessRequest *request = nullptr);
  void release_access(StorageId id) noexcept;

  // Introspection for tests and tools.
  const StorageState *state(StorageId id) const {
    auto it = _states.find(id);
    return it == _states.end() ? nullptr : &it->second;
  }
  std::size_t object_count() const { return _states.size(); }

 protected:
  // Called only with active_users == 0; the object is ready when it returns.
  // (The reference declares this with a request struct in the base and a
  // (StorageId, layer) pair in NaiveKVStorage, which does not override it —
  // kvstorage.hpp:66 vs naiveKVStorage.hpp:52 — one signature is used here.)
  virtual infer::expected<void, std::error_code> prepare_object(const KVObjectAccessRequest &req) = 0;
  // Called only with active_users == 0; the base erases the entry after it.
  virtual void destroy_object(StorageId id) noexcept = 0;
  // Called on every successful acquire, with that acquire's request
  // (recency for eviction policies, rows written for write-back).
  virtual void record_access(const KVObjectAccessRequest &) noexcept {}

  std::unordered_map<StorageId, StorageState> _states;
  std::vector<KVLayerSpec> _layers;
  std::vector<Backend *> _backend_layer;
  StorageId _next_storage_id = 1;
};

// One backend allocation per (sequence, layer): the K region
// [capacity][n_kv_heads][k_head_dim] followed by the V region
// (reference src/kvcache/KVStorages/naiveKVStorage.cpp:17-54).
class NaiveKVStorage : public KVStorage {
 public:
  ~NaiveKVStorage() override;
  infer::expected<void, std::error_code> init(std::span<const KVLayerSpec> layers,
                                              std::span<Backend *const> backend_layer) override;
  infer::expected<StorageId, std::error_code> alloc(std::size_t layer,
                                                   std::size_t capacity_tokens) override;

 protected:
  infer::expected<void, std::error_code> prepare_object(const KVObjectAccessRequest &req) override;
  void destroy_object(StorageId id) noexcept override;
};

// Paged storage: per layer one backend allocation holding a K pool and a V
// pool of `blocks_per_layer` blocks of `block_tokens` token rows each
// ([blocks][block_tokens][n_kv_heads][head_dim] per pool), sized once for
// the device (an MI355X holds 288 GB of HBM). alloc() hands out one block as
// one storage object (capacity_tokens == block_tokens) from the layer's free
// list; destroying the object returns the block. No backend call per block.
class BlockPoolKVStorage : public KVStorage {
 public:
  BlockPoolKVStorage(std::size_t blocks_per_layer, std::size_t block_tokens) noexcept
      : _blocks(blocks_per_layer), _block_tokens(block_tokens) {}
  ~BlockPoolKVStorage() override;
  infer::expected<void, std::error_code> init(std::span<const KVLayerSpec> layers,
                                              std::span<Backend *const> backend_layer) override;
  infer::expected<StorageId, std::error_code> alloc(std::size_t layer,
                                                   std::size_t capacity_tokens) override;

  std::size_t block_tokens() const { return _block_tokens; }
  std::size_t blocks_per_layer() const { return _blocks; }
  std::size_t free_blocks(std::size_t layer) const {
    return layer < _pools.size() ? _pools[layer].free.size() : 0;
  }
  void *k_pool(std::size_t layer) const { return layer < _pools.size() ? _pools[layer].k : nullptr; }
  void *v_pool(std::size_t layer) const { return layer < _pools.size() ? _pools[layer].v : nullptr; }
  // Pool block of an object, or -1 for an unknown id.
  int64_t block_of(StorageId id) const;

 protected:
  infer::expected<void, std::error_code> prepare_object(const KVObjectAccessRequest &req) override;
  void destroy_object(StorageId id) noexcept override;

 private:
  struct Pool {
    void *base = nullptr;  // the allocation: K pool, then V pool
    void *k = nullptr;
    void *v = nullptr;
    std::size_t k_block_bytes = 0, v_block_bytes = 0;
    std::vector<std::size_t> free;  // block indices, taken from the back
  };
  std::size_t _blocks, _block_tokens;
  std::vector<Pool> _pools;
  std::unordered_map<StorageId, std::size_t> _block;  // object -> pool block
};

