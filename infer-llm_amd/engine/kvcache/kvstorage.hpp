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

struct KVObjectAccessRequest {
  StorageId id = kInvalidStorageId;
  std::size_t layer = 0;
  std::size_t history_tokens = 0;
  TokenRange writable;
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
  infer::expected<KVStorageObject, std::error_code> acquire(StorageId id, std::size_t layer);
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
