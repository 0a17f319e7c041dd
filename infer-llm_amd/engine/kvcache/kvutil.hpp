// kvutil.hpp — shared types of the KV-cache subsystem (reference
// include/kvcache/kvutil.hpp:16-131): layer specs, token ranges, storage
// slices, and the non-owning K/V views handed to the graph.
#pragma once

#include <cassert>
#include <cstddef>
#include <cstdint>
#include <utility>
#include <vector>

#include "../tensor.hpp"
#include "../util.hpp"

class KVStrategy;
class Backend;

using StorageId = std::uint64_t;
constexpr StorageId kInvalidStorageId = 0;
using SequenceId = std::uint64_t;
constexpr SequenceId kInvalidSequenceId = 0;

struct KVLayerSpec {
  std::size_t n_kv_heads = 0;
  std::size_t k_head_dim = 0;
  std::size_t v_head_dim = 0;
  DataType k_type = GGML_TYPE_F32;
  DataType v_type = GGML_TYPE_F32;
};

struct KVCacheConfig {
  std::size_t layers = 0;
  std::size_t max_tokens_per_sequence = 0;  // capacity of one (sequence, layer)
  std::size_t block_tokens = 0;             // 0: contiguous (the only strategy built)
  std::size_t alignment = 256;
};

// Token positions [begin, begin + count), numbered from 0 per sequence.
struct TokenRange {
  std::size_t begin = 0;
  std::size_t count = 0;
  std::size_t end() const noexcept { return begin + count; }
  bool empty() const noexcept { return count == 0; }
};

struct KVSlice {
  StorageId storage_id = kInvalidStorageId;
  std::size_t token_offset = 0;
  std::size_t token_count = 0;
};

struct KVMapping {
  std::vector<KVSlice> k;
  std::vector<KVSlice> v;
};

// Non-owning view of one slice; view.data points at its first token.
struct KVSegmentView {
  Tensor view;
  std::size_t token_begin = 0;
  std::size_t token_count = 0;
};

// A paged layer as one kernel sees it: the layer's K and V block pools
// ([pool_blocks * block_tokens][n_kv_heads][head_dim] each) and the
// sequence's device block table (entry i = pool block of tokens
// [i * block_tokens, (i + 1) * block_tokens)). The readable and writable
// segments of the access are the same rows, one segment per block.
struct KVPages {
  Tensor *block_table = nullptr;  // I32 [entries], device; owned by the strategy
  std::size_t block_tokens = 0;
  std::size_t pool_blocks = 0;
  void *k_pool = nullptr;
  void *v_pool = nullptr;
  explicit operator bool() const noexcept { return block_table != nullptr; }
};

struct KVRangeAccess {
  std::vector<KVSegmentView> k;
  std::vector<KVSegmentView> v;
};

// Guarded access to one layer for one step: readable [0, n_past + n_new),
// writable [n_past, n_past + n_new). Must be handed back with release_layer
// of the same strategy once the step's kernels are done.
struct KVLayerAccess {
 private:
  friend class KVStrategy;
  std::vector<StorageId> _storage_ids;  // deduplicated acquires to hand back
  KVStrategy *_owner = nullptr;

 public:
  KVLayerAccess() = default;
  KVLayerAccess(const KVLayerAccess &) = delete;
  KVLayerAccess &operator=(const KVLayerAccess &) = delete;
  KVLayerAccess(KVLayerAccess &&o) noexcept
      : _storage_ids(std::move(o._storage_ids)),
        _owner(std::exchange(o._owner, nullptr)),
        backend(std::exchange(o.backend, nullptr)),
        n_past(std::exchange(o.n_past, 0)),
        n_new(std::exchange(o.n_new, 0)),
        readable(std::move(o.readable)),
        writable(std::move(o.writable)),
        pages(std::exchange(o.pages, KVPages{})) {
    o._storage_ids.clear();
    o.readable.k.clear();
    o.readable.v.clear();
    o.writable.k.clear();
    o.writable.v.clear();
  }
  KVLayerAccess &operator=(KVLayerAccess &&) = delete;
  ~KVLayerAccess() { assert(_owner == nullptr && "release_layer must be called"); }

  bool released() const noexcept { return _owner == nullptr; }

  Backend *backend = nullptr;
  std::size_t n_past = 0;
  std::size_t n_new = 0;
  KVRangeAccess readable;
  KVRangeAccess writable;
  // Set by a paged strategy (block_tokens > 0); empty for contiguous storage.
  KVPages pages;
};
