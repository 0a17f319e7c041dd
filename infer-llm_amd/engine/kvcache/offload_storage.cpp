#include "offload_storage.hpp"

#include <algorithm>
#include <limits>

namespace {

// The bytes of one copy as a tensor, for the backends' copy calls.
Tensor bytes_view(void *base, std::size_t bytes) {
  Tensor t("kv_offload_copy", GGML_TYPE_F32, {static_cast<int64_t>(bytes / sizeof(float))});
  t.data = base;
  return t;
}

}  // namespace

std::optional<StorageId> LRUKVEvictionPolicy::select_victim(
    std::span<const KVEvictionCandidate> candidates) const {
  const KVEvictionCandidate *best = nullptr;
  for (const auto &c : candidates) {
    if (!best || c.last_access_order < best->last_access_order ||
        (c.last_access_order == best->last_access_order && c.admission_order < best->admission_order))
      best = &c;
  }
  if (!best) return std::nullopt;
  return best->id;
}

std::vector<KVPrefetchRequest> NextAccessKVPrefetchPolicy::plan(const KVPrefetchContext &context) const {
  std::vector<KVPrefetchRequest> out;
  for (const auto &r : context.upcoming) {
    if (out.size() >= _lookahead) break;
    if (r.id != kInvalidStorageId && r.id != context.current) out.push_back(r);
  }
  return out;
}

// ---------------------------------------------------------------------------

OffloadKVStorage::OffloadKVStorage(OffloadKVStorageConfig config,
                                   std::unique_ptr<KVEvictionPolicy> eviction,
                                   std::unique_ptr<KVPrefetchPolicy> prefetch)
    : _config(std::move(config)), _eviction(std::move(eviction)), _prefetch(std::move(prefetch)) {}

OffloadKVStorage::~OffloadKVStorage() {
  for (auto &[id, st] : _objects) {
    release_copy(st.dev);
    release_copy(st.host);
  }
}

void OffloadKVStorage::release_copy(std::optional<Copy> &c) noexcept {
  if (c && c->backend && c->base) c->backend->free(BufferKind::KVCACHE, c->base);
  c.reset();
}

infer::expected<void, std::error_code> OffloadKVStorage::init(std::span<const KVLayerSpec> layers,
                                                             std::span<Backend *const> backend_layer) {
  if (layers.size() != backend_layer.size() || !_eviction || !_prefetch || !_config.host_backend ||
      !_config.host_backend->is_host())
    return infer::fail(std::errc::invalid_argument);
  for (Backend *b : backend_layer) {
    if (!b) return infer::fail(std::errc::invalid_argument);
    // every device a layer computes on needs its budget
    if (!b->is_host() && !budget_for(b)) return infer::fail(std::errc::invalid_argument);
  }
  for (std::size_t i = 0; i < _config.device_budgets.size(); ++i)
    for (std::size_t j = 0; j < i; ++j)
      if (_config.device_budgets[i].backend == _config.device_budgets[j].backend)
        return infer::fail(std::errc::invalid_argument);  // one budget per device
  _layers.assign(layers.begin(), layers.end());
  _backend_layer.assign(backend_layer.begin(), backend_layer.end());
  return {};
}

const KVDeviceBudget *OffloadKVStorage::budget_for(const Backend *backend) const {
  for (const auto &b : _config.device_budgets)
    if (b.backend == backend) return &b;
  return nullptr;
}

std::size_t OffloadKVStorage::resident_bytes(const Backend *backend) const {
  std::size_t n = 0;
  for (const auto &[id, st] : _objects)
    if (st.dev && st.dev->backend == backend) n += st.dev->bytes;
  return n;
}

bool OffloadKVStorage::resident(StorageId id) const {
  auto it = _objects.find(id);
  return it != _objects.end() && it->second.dev.has_value();
}

void OffloadKVStorage::point_object_at(StorageId id, const Copy *c) {
  auto it = _states.find(id);
  if (it == _states.end()) return;
  KVStorageObject &o = it->second.object;
  const KVLayerSpec &sp = _layers[it->second.layer];
  const std::size_t k_bytes = sp.n_kv_heads * sp.k_head_dim * dataType_size(sp.k_type) * o.capacity_tokens;
  o.k_base = c ? c->base : nullptr;
  o.v_base = c ? static_cast<std::byte *>(c->base) + k_bytes : nullptr;
}

infer::expected<StorageId, std::error_code> OffloadKVStorage::alloc(std::size_t layer,
                                                                   std::size_t capacity_tokens) {
  if (layer >= _layers.size()) return infer::fail(std::errc::invalid_argument);
  Backend *backend = _backend_layer[layer];
  const KVLayerSpec &sp = _layers[layer];
  const std::size_t row = sp.n_kv_heads * (sp.k_head_dim * dataType_size(sp.k_type) +
                                           sp.v_head_dim * dataType_size(sp.v_type));
  if (capacity_tokens && row > std::numeric_limits<std::size_t>::max() / capacity_tokens)
    return infer::fail(std::errc::value_too_large);
  const std::size_t bytes = row * capacity_tokens;
  const StorageId id = _next_storage_id++;
  ObjectState st;
  st.admission_order = ++_clock;
  const bool on_device = !backend->is_host() && _config.first_alloc == KVFirstAllocPlacement::LayerBackend;
  if (on_device) {
    if (auto r = make_room(*backend, bytes, kInvalidStorageId); !r) return infer::unexpected(r.error());
    auto mem = backend->alloc(BufferKind::KVCACHE, bytes);
    if (!mem) return infer::unexpected(mem.error());
    st.dev = Copy{backend, *mem, bytes};
  } else {
    auto mem = _config.host_backend->alloc(BufferKind::KVCACHE, bytes);
    if (!mem) return infer::unexpected(mem.error());
    st.host = Copy{_config.host_backend, *mem, bytes};
  }
  KVStorageObject obj{.id = id, .backend = backend, .capacity_tokens = capacity_tokens};
  if (!_states.try_emplace(id, StorageState{.object = obj, .layer = layer}).second) {
    release_copy(st.dev);
    release_copy(st.host);
    return infer::fail(std::errc::file_exists);
  }
  auto [it, ok] = _objects.emplace(id, std::move(st));
  const Copy *compute = it->second.dev ? &*it->second.dev : (backend->is_host() ? &*it->second.host : nullptr);
  point_object_at(id, compute);
  return id;
}

infer::expected<void, std::error_code> OffloadKVStorage::make_room(Backend &backend, std::size_t bytes,
                                                                  StorageId protected_id) {
  const KVDeviceBudget *b = budget_for(&backend);
  if (!b || bytes > b->resident_bytes) return infer::fail(std::errc::not_enough_memory);
  while (resident_bytes(&backend) + bytes > b->resident_bytes) {
    std::vector<KVEvictionCandidate> cands;
    for (const auto &[id, st] : _objects) {
      if (!st.dev || st.dev->backend != &backend || id == protected_id) continue;
      auto s = _states.find(id);
      if (s == _states.end() || s->second.active_users != 0) continue;
      cands.push_back({.id = id,
                       .resident_bytes = st.dev->bytes,
                       .writeback_bytes = writeback_bytes(id, st),
                       .last_access_order = st.last_access_order,
                       .admission_order = st.admission_order});
    }
    auto victim = _eviction->select_victim(cands);
    if (!victim) return infer::fail(std::errc::not_enough_memory);
    if (std::none_of(cands.begin(), cands.end(), [&](const auto &c) { return c.id == *victim; }))
      return infer::fail(std::errc::invalid_argument);  // the policy named a non-candidate
    if (auto r = evict(*victim); !r) return r;
  }
  return {};
}

infer::expected<void, std::error_code> OffloadKVStorage::writeback(StorageId id) {
  auto it = _objects.find(id);
  if (it == _objects.end() || !it->second.dev) return infer::fail(std::errc::invalid_argument);
  ObjectState &st = it->second;
  if (!st.host) {
    auto mem = _config.host_backend->alloc(BufferKind::KVCACHE, st.dev->bytes);
    if (!mem) return infer::unexpected(mem.error());
    st.host = Copy{_config.host_backend, *mem, st.dev->bytes};
    st.host_valid = 0;
  }
  const auto [lo, hi] = writeback_rows(id, st);
  if (lo < hi) {
    // The device backend's copies are ordered after its queued kernels.
    const RowBytes rb = row_bytes(id, lo, hi);
    const Tensor dev = bytes_view(st.dev->base, st.dev->bytes);
    auto *h = static_cast<std::byte *>(st.host->base);
    if (auto r = st.dev->backend->copy_tensor_get(&dev, h + rb.k_off, rb.k_off, rb.k_len); !r) return r;
    if (auto r = st.dev->backend->copy_tensor_get(&dev, h + rb.v_off, rb.v_off, rb.v_len); !r) return r;
    st.host_valid = std::max(st.host_valid, hi);
    ++_stats.page_outs;
    _stats.bytes_out += rb.k_len + rb.v_len;
  }
  st.dirty_lo = SIZE_MAX;
  st.dirty_hi = 0;
  return {};
}

infer::expected<void, std::error_code> OffloadKVStorage::evict(StorageId id) {
  auto it = _objects.find(id);
  auto s = _states.find(id);
  if (it == _objects.end() || s == _states.end()) return infer::fail(std::errc::invalid_argument);
  ObjectState &st = it->second;
  if (!st.dev) return {};
  if (s->second.active_users != 0) return infer::fail(std::errc::device_or_resource_busy);
  if (st.dirty() || !st.host) {
    if (auto r = writeback(id); !r) return r;  // the HBM copy stays on failure
  }
  // No queued kernel may still read the HBM copy when it is freed.
  if (auto r = st.dev->backend->synchronize(); !r) return r;
  release_copy(st.dev);
  point_object_at(id, nullptr);
  ++_stats.evictions;
  return {};
}

infer::expected<void, std::error_code> OffloadKVStorage::ensure_resident(StorageId id, bool may_evict) {
  auto it = _objects.find(id);
  auto s = _states.find(id);
  if (it == _objects.end() || s == _states.end()) return infer::fail(std::errc::invalid_argument);
  ObjectState &st = it->second;
  Backend *backend = _backend_layer[s->second.layer];
  if (backend->is_host()) {  // a host-computed layer works on the host copy
    point_object_at(id, st.host ? &*st.host : nullptr);
    return st.host ? infer::expected<void, std::error_code>{} : infer::fail(std::errc::invalid_argument);
  }
  if (st.dev) {
    point_object_at(id, &*st.dev);
    return {};
  }
  const std::size_t bytes = st.host ? st.host->bytes : 0;
  if (!st.host) return infer::fail(std::errc::invalid_argument);
  if (may_evict) {
    if (auto r = make_room(*backend, bytes, id); !r) return r;
  } else {
    const KVDeviceBudget *b = budget_for(backend);
    if (!b || resident_bytes(backend) + bytes > std::min(b->prefetch_bytes, b->resident_bytes))
      return infer::fail(std::errc::not_enough_memory);
  }
  auto mem = backend->alloc(BufferKind::KVCACHE, bytes);
  if (!mem) return infer::unexpected(mem.error());
  if (st.host_valid > 0) {  // the rows the host copy holds, of K and of V
    const RowBytes rb = row_bytes(id, 0, st.host_valid);
    Tensor dev = bytes_view(*mem, bytes);
    const auto *h = static_cast<const std::byte *>(st.host->base);
    auto r = backend->copy_tensor_set(&dev, h + rb.k_off, rb.k_off, rb.k_len);
    if (r) r = backend->copy_tensor_set(&dev, h + rb.v_off, rb.v_off, rb.v_len);
    if (!r) {
      backend->free(BufferKind::KVCACHE, *mem);
      return r;
    }
    ++_stats.page_ins;
    _stats.bytes_in += rb.k_len + rb.v_len;
  }
  st.dev = Copy{backend, *mem, bytes};
  st.dirty_lo = SIZE_MAX;
  st.dirty_hi = 0;
  point_object_at(id, &*st.dev);
  return {};
}

infer::expected<void, std::error_code> OffloadKVStorage::prepare_object(const KVObjectAccessRequest &req) {
  if (req.layer >= _layers.size() || !_states.contains(req.id))
    return infer::fail(std::errc::invalid_argument);
  return ensure_resident(req.id, true);
}

void OffloadKVStorage::record_access(const KVObjectAccessRequest &req) noexcept {
  auto it = _objects.find(req.id);
  auto s = _states.find(req.id);
  if (it == _objects.end() || s == _states.end()) return;
  ObjectState &st = it->second;
  st.last_access_order = ++_clock;
  // The rows this access may write; not known: all of them.
  const std::size_t cap = s->second.object.capacity_tokens;
  std::size_t lo = 0, hi = cap;
  if (req.ranges_known) {
    if (req.writable.empty()) return;
    lo = std::min(req.writable.begin, cap);
    hi = std::min(req.writable.end(), cap);
  }
  if (st.dev) {
    st.dirty_lo = std::min(st.dirty_lo, lo);
    st.dirty_hi = std::max(st.dirty_hi, hi);
  } else if (st.host) {  // a host-computed layer writes its host copy
    st.host_valid = std::max(st.host_valid, hi);
  }
}

OffloadKVStorage::RowBytes OffloadKVStorage::row_bytes(StorageId id, std::size_t lo, std::size_t hi) const {
  const StorageState &ss = _states.at(id);
  const KVLayerSpec &sp = _layers[ss.layer];
  const std::size_t k_row = sp.n_kv_heads * sp.k_head_dim * dataType_size(sp.k_type);
  const std::size_t v_row = sp.n_kv_heads * sp.v_head_dim * dataType_size(sp.v_type);
  const std::size_t k_bytes = k_row * ss.object.capacity_tokens;
  return {.k_off = lo * k_row, .v_off = k_bytes + lo * v_row, .k_len = (hi - lo) * k_row,
          .v_len = (hi - lo) * v_row};
}

std::pair<std::size_t, std::size_t> OffloadKVStorage::writeback_rows(StorageId id, const ObjectState &st) const {
  if (!st.dirty()) return {0, 0};
  // Rows the host copy lacks that the HBM copy may hold start at host_valid
  // at the latest (everything below it was uploaded unchanged unless dirty).
  const std::size_t cap = _states.at(id).object.capacity_tokens;
  const std::size_t hi = std::min(st.dirty_hi, cap);
  const std::size_t lo = std::min({st.dirty_lo, st.host ? st.host_valid : 0, hi});
  return {lo, hi};
}

std::size_t OffloadKVStorage::writeback_bytes(StorageId id, const ObjectState &st) const {
  const auto [lo, hi] = writeback_rows(id, st);
  if (lo >= hi) return 0;
  const RowBytes rb = row_bytes(id, lo, hi);
  return rb.k_len + rb.v_len;
}

infer::expected<std::size_t, std::error_code> OffloadKVStorage::prefetch(const KVPrefetchContext &context) {
  std::size_t done = 0;
  for (const KVPrefetchRequest &r : _prefetch->plan(context)) {
    auto it = _objects.find(r.id);
    auto s = _states.find(r.id);
    if (it == _objects.end() || s == _states.end() || s->second.pending_free || it->second.dev) continue;
    auto up = ensure_resident(r.id, false);
    if (!up) {
      if (up.error() == std::make_error_code(std::errc::not_enough_memory)) continue;  // no room: skip
      return infer::unexpected(up.error());
    }
    ++done;
    ++_stats.prefetches;
  }
  return done;
}

void OffloadKVStorage::destroy_object(StorageId id) noexcept {
  auto it = _objects.find(id);
  if (it == _objects.end()) return;
  if (it->second.dev) (void)it->second.dev->backend->synchronize();
  release_copy(it->second.dev);
  release_copy(it->second.host);
  _objects.erase(it);
}
