#include "backend.hpp"

#include <algorithm>
#include <cstdlib>

void Backend::init_pools(std::unique_ptr<PhysicalAllocator> phys) {
  _phys_allocator = std::move(phys);
  // Only the naive strategy exists; BUMP and CACHING fall back to it (the
  // reference leaves them unimplemented, include/backend.hpp:71-74).
  _weights_pool = std::make_unique<NaivePool>(*_phys_allocator);
  _activation_pool = std::make_unique<NaivePool>(*_phys_allocator);
  _kvcache_pool = std::make_unique<NaivePool>(*_phys_allocator);
}

MemoryPool *Backend::pool(BufferKind kind) {
  switch (kind) {
    case BufferKind::WEIGHTS: return _weights_pool.get();
    case BufferKind::ACTIVATION: return _activation_pool.get();
    case BufferKind::KVCACHE: return _kvcache_pool.get();
  }
  return nullptr;
}

infer::expected<void *, std::error_code> Backend::alloc(BufferKind kind, size_t bytes) {
  MemoryPool *p = pool(kind);
  if (!p) return infer::fail(std::errc::invalid_argument);
  return p->alloc(bytes);
}

void Backend::free(BufferKind kind, void *ptr) {
  if (!ptr) return;
  if (MemoryPool *p = pool(kind)) p->free(ptr);
}

// ---------------------------------------------------------------------------

BackendRegistry &BackendRegistry::instance() {
  static BackendRegistry reg;
  return reg;
}

void BackendRegistry::register_backend(std::string type_name, ProbeFunc probe, CreateFunc creator) {
  _entries[std::move(type_name)] = Entry{std::move(probe), std::move(creator)};
}

void BackendRegistry::probe_all() {
  _devices.clear();
  for (auto &[name, entry] : _entries)
    for (auto &info : entry.probe()) _devices.push_back(std::move(info));
}

infer::expected<std::unique_ptr<Backend>, std::error_code> BackendRegistry::create(
    std::string_view name, const PoolConfig &cfg) const {
  auto dev = std::find_if(_devices.begin(), _devices.end(),
                          [&](const DeviceInfo &d) { return d.name == name; });
  if (dev == _devices.end()) return infer::fail(std::errc::no_such_device);
  auto entry = _entries.find(extract_type(name));
  if (entry == _entries.end()) return infer::fail(std::errc::no_such_device);
  return entry->second.create(extract_device_id(name), *dev, cfg);
}

infer::expected<std::unique_ptr<Backend>, std::error_code> BackendRegistry::create_default(
    const PoolConfig &cfg) const {
  if (const char *env = std::getenv("INFERLLM_DEVICE")) return create(env, cfg);
  for (DeviceType t : {DeviceType::HIP, DeviceType::CUDA, DeviceType::METAL, DeviceType::CPU})
    for (const auto &d : _devices)
      if (d.type == t) return create(d.name, cfg);
  return infer::fail(std::errc::no_such_device);
}

infer::expected<DeviceInfo, std::error_code> BackendRegistry::device_info(std::string_view name) const {
  for (const auto &d : _devices)
    if (d.name == name) return d;
  return infer::fail(std::errc::invalid_argument);
}

std::string BackendRegistry::extract_type(std::string_view name) {
  const auto colon = name.find(':');
  return std::string(colon == std::string_view::npos ? name : name.substr(0, colon));
}

int BackendRegistry::extract_device_id(std::string_view name) {
  const auto colon = name.find(':');
  if (colon == std::string_view::npos) return 0;
  return std::atoi(std::string(name.substr(colon + 1)).c_str());
}
