// offload_storage.hpp — the HBM <-> host tier of the KV cache (reference
// include/kvcache/KVStorages/offloadKVStorage.hpp, kvEvictionPolicy.hpp,
// kvPrefetchPolicy.hpp; the reference's implementation is unfinished:
// src/kvcache/KVStorages/offloadKVStorage.cpp leaves prepare_object, evict,
// prefetch and writeback unimplemented).
//
// Every storage object (one (sequence, layer) cache, K region then V region)
// may hold two copies: one in pinned host memory on the host backend and one
// in HBM on its layer's backend. The HBM copy is the only one kernels see:
// acquire() makes it resident (uploading the host copy), under a hard
// per-device byte budget; when the budget is full, the eviction policy picks
// an object nobody holds, its HBM copy is written back to the host (if
// kernels may have written it since it was uploaded) and freed.
//
// Only token rows that hold data move (the reference's per-copy valid_tokens,
// offloadKVStorage.hpp:113-160): a host copy holds rows [0, host_valid) as of
// its last write-back (0 when new), and an upload copies those rows of K and
// of V; each access names the rows it writes (KVObjectAccessRequest), and a
// write-back copies the rows written since the HBM copy was made, from
// min(first written row, host_valid) on. So a new sequence's first step
// uploads nothing, and a switch between sequences moves each cache's
// committed rows in, and only the rows written since, out. An access whose
// rows are not known marks the whole object written. Copies use the
// backend's synchronous copies, so the stream's queued kernels finish before
// any copy or free. No disk tier (the reference declares one and implements
// none of it).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>
#include <span>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "kvstorage.hpp"

// What an eviction policy sees: objects on one device that no access holds.
struct KVEvictionCandidate {
  StorageId id = kInvalidStorageId;
  std::size_t resident_bytes = 0;
  std::size_t writeback_bytes = 0;  // 0 when the host copy is current
  std::uint64_t last_access_order = 0;
  std::uint64_t admission_order = 0;
};

class KVEvictionPolicy {
 public:
  virtual ~KVEvictionPolicy() = default;
  virtual std::string name() const = 0;
  // One victim among the candidates, or nullopt for none.
  virtual std::optional<StorageId> select_victim(std::span<const KVEvictionCandidate> candidates) const = 0;
};

// Least recently acquired first; ties go to the earlier admitted.
class LRUKVEvictionPolicy final : public KVEvictionPolicy {
 public:
  std::string name() const override { return "LRU"; }
  std::optional<StorageId> select_victim(std::span<const KVEvictionCandidate> candidates) const override;
};

// history_tokens: the committed prefix the next access reads (an upload
// copies the rows the host copy holds, so it only orders and filters
// requests).
struct KVPrefetchRequest {
  StorageId id = kInvalidStorageId;
  std::size_t history_tokens = 0;
};

struct KVPrefetchContext {
  StorageId current = kInvalidStorageId;
  std::span<const KVPrefetchRequest> upcoming;
};

class KVPrefetchPolicy {
 public:
  virtual ~KVPrefetchPolicy() = default;
  virtual std::string name() const = 0;
  // Requests in priority order, taken from context.upcoming only.
  virtual std::vector<KVPrefetchRequest> plan(const KVPrefetchContext &context) const = 0;
};

class NoKVPrefetchPolicy final : public KVPrefetchPolicy {
 public:
  std::string name() const override { return "None"; }
  std::vector<KVPrefetchRequest> plan(const KVPrefetchContext &) const override { return {}; }
};

// The next `lookahead` upcoming objects, in order.
class NextAccessKVPrefetchPolicy final : public KVPrefetchPolicy {
 public:
  explicit NextAccessKVPrefetchPolicy(std::size_t lookahead) : _lookahead(lookahead) {}
  std::string name() const override { return "NextAccess"; }
  std::vector<KVPrefetchRequest> plan(const KVPrefetchContext &context) const override;

 private:
  std::size_t _lookahead;
};

struct KVDeviceBudget {
  Backend *backend = nullptr;      // not owned
  std::size_t resident_bytes = 0;  // hard cap of HBM copies on this device
  std::size_t prefetch_bytes = 0;  // part of the cap prefetch may fill; 0 = no prefetch
};

enum class KVFirstAllocPlacement {
  CPU,           // alloc() creates the host copy; the first acquire uploads it
  LayerBackend,  // alloc() creates the HBM copy (within the budget); no host copy yet
};

struct OffloadKVStorageConfig {
  Backend *host_backend = nullptr;  // is_host(); outlives the storage
  std::vector<KVDeviceBudget> device_budgets;
  KVFirstAllocPlacement first_alloc = KVFirstAllocPlacement::CPU;
};

struct OffloadStats {
  std::uint64_t page_ins = 0, page_outs = 0, evictions = 0, prefetches = 0;
  std::uint64_t bytes_in = 0, bytes_out = 0;
};

class OffloadKVStorage final : public KVStorage {
 public:
  OffloadKVStorage(OffloadKVStorageConfig config, std::unique_ptr<KVEvictionPolicy> eviction,
                   std::unique_ptr<KVPrefetchPolicy> prefetch);
  ~OffloadKVStorage() override;

  infer::expected<void, std::error_code> init(std::span<const KVLayerSpec> layers,
                                              std::span<Backend *const> backend_layer) override;
  infer::expected<StorageId, std::error_code> alloc(std::size_t layer,
                                                   std::size_t capacity_tokens) override;

  // Drops the HBM copy (writing it back first when needed). busy while an
  // access holds the object; a failed write-back keeps the HBM copy.
  infer::expected<void, std::error_code> evict(StorageId id);
  // Uploads the objects the prefetch policy picks from context, as far as
  // each device's prefetch budget allows without evicting anything. Returns
  // how many were uploaded.
  infer::expected<std::size_t, std::error_code> prefetch(const KVPrefetchContext &context);

  bool resident(StorageId id) const;
  std::size_t resident_bytes(const Backend *backend) const;
  const OffloadStats &stats() const { return _stats; }

 protected:
  infer::expected<void, std::error_code> prepare_object(const KVObjectAccessRequest &req) override;
  void destroy_object(StorageId id) noexcept override;
  void record_access(const KVObjectAccessRequest &req) noexcept override;

 private:
  struct Copy {
    Backend *backend = nullptr;
    void *base = nullptr;  // K region, then V region
    std::size_t bytes = 0;
  };
  struct ObjectState {
    std::optional<Copy> host, dev;
    std::size_t host_valid = 0;  // rows [0, host_valid) of the host copy hold data
    // Rows [dirty_lo, dirty_hi) of the HBM copy may have been written by
    // kernels since it was made or last written back (empty: lo >= hi).
    std::size_t dirty_lo = SIZE_MAX, dirty_hi = 0;
    std::uint64_t last_access_order = 0, admission_order = 0;
    bool dirty() const { return dirty_lo < dirty_hi; }
  };
  // The byte range of rows [lo, hi) within the K region and within the V
  // region of an object of this storage's layer `layer`.
  struct RowBytes {
    std::size_t k_off, v_off, k_len, v_len;
  };
  RowBytes row_bytes(StorageId id, std::size_t lo, std::size_t hi) const;
  // The rows a write-back of this object would copy: [lo, hi), empty if none,
  // and their bytes (K and V).
  std::pair<std::size_t, std::size_t> writeback_rows(StorageId id, const ObjectState &st) const;
  std::size_t writeback_bytes(StorageId id, const ObjectState &st) const;

  const KVDeviceBudget *budget_for(const Backend *backend) const;
  infer::expected<void, std::error_code> ensure_resident(StorageId id, bool may_evict);
  infer::expected<void, std::error_code> make_room(Backend &backend, std::size_t bytes,
                                                  StorageId protected_id);
  infer::expected<void, std::error_code> writeback(StorageId id);
  void point_object_at(StorageId id, const Copy *c);
  void release_copy(std::optional<Copy> &c) noexcept;

  OffloadKVStorageConfig _config;
  std::unique_ptr<KVEvictionPolicy> _eviction;
  std::unique_ptr<KVPrefetchPolicy> _prefetch;
  std::unordered_map<StorageId, ObjectState> _objects;
  std::uint64_t _clock = 0;
  OffloadStats _stats;
};
