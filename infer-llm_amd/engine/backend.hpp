// backend.hpp — the device plugin interface and its registry (reference
// include/backend.hpp:17-171, src/backend.cpp:1-104).
//
// A backend owns three pools (weights, activations, KV cache) over one
// physical allocator, copies tensors to/from host memory, and computes a
// topologically ordered subgraph. Devices are named "type:id"; the registry
// probes each registered type and creates backends by name.
#pragma once

#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

#include "expected.hpp"
#include "memory_pool.hpp"
#include "tensor.hpp"
#include "util.hpp"

class Graph;

struct DeviceInfo {
  std::string name;  // "cpu", "hip:0"
  DeviceType type = DeviceType::CPU;
  size_t memory_bytes = 0;
};

enum class BufferKind : uint8_t {
  WEIGHTS = 0,  // resident for the model's lifetime
  ACTIVATION,   // one graph execution
  KVCACHE,      // one request (sequence)
};

enum class Strategy { NAIVE, BUMP, CACHING };

struct PoolConfig {
  Strategy weights = Strategy::NAIVE;
  Strategy activation = Strategy::NAIVE;
  Strategy kvcache = Strategy::NAIVE;
};

class Backend {
 public:
  Backend(int device_id, DeviceInfo info, const PoolConfig &cfg)
      : _device_id(device_id), _info(std::move(info)), _pool_config(cfg) {}
  virtual ~Backend() = default;

  void init_pools(std::unique_ptr<PhysicalAllocator> phys);
  const DeviceInfo &get_info() const { return _info; }
  int device_id() const { return _device_id; }

  virtual DeviceType device_type() const = 0;
  virtual std::string device_name() const = 0;
  virtual bool supports_op(OperationType op, const Tensor &t) const = 0;

  virtual infer::expected<void *, std::error_code> alloc(BufferKind kind, size_t bytes);
  virtual void free(BufferKind kind, void *ptr);

  virtual bool is_host() const = 0;
  // host memory -> tensor's buffer
  virtual infer::expected<void, std::error_code> copy_tensor_set(Tensor *tensor, const void *data,
                                                                 size_t offset, size_t size) = 0;
  // tensor's buffer -> host memory
  virtual infer::expected<void, std::error_code> copy_tensor_get(const Tensor *tensor, void *data,
                                                                 size_t offset, size_t size) = 0;
  // device-side copy into dst's buffer; false = not supported (caller bounces
  // through host memory)
  virtual infer::expected<bool, std::error_code> copy_tensor_high(const Tensor *src,
                                                                  Tensor *dst) const = 0;
  virtual infer::expected<void, std::error_code> compute(Graph &sub_graph) = 0;
  // Waits for this backend's queued work (scheduler boundary / result reads).
  virtual infer::expected<void, std::error_code> synchronize() { return {}; }
  // True when the op at `node` reads src[src_index] from host memory itself,
  // so the scheduler must not stage a device copy of it.
  virtual bool accepts_host_src(const Tensor &node, int src_index) const {
    (void)node;
    (void)src_index;
    return false;
  }

 protected:
  MemoryPool *pool(BufferKind kind);

  int _device_id;
  DeviceInfo _info;
  PoolConfig _pool_config;
  std::unique_ptr<PhysicalAllocator> _phys_allocator;
  std::unique_ptr<MemoryPool> _weights_pool;
  std::unique_ptr<MemoryPool> _activation_pool;
  std::unique_ptr<MemoryPool> _kvcache_pool;
};

class BackendRegistry {
 public:
  using ProbeFunc = std::function<std::vector<DeviceInfo>()>;
  using CreateFunc =
      std::function<std::unique_ptr<Backend>(int device_id, const DeviceInfo info, const PoolConfig &cfg)>;

  static BackendRegistry &instance();
  void register_backend(std::string type_name, ProbeFunc probe, CreateFunc creator);
  void probe_all();
  infer::expected<std::unique_ptr<Backend>, std::error_code> create(std::string_view name,
                                                                     const PoolConfig &cfg) const;
  // INFERLLM_DEVICE when set, else HIP > CUDA > Metal > CPU.
  infer::expected<std::unique_ptr<Backend>, std::error_code> create_default(const PoolConfig &cfg) const;
  const std::vector<DeviceInfo> &available_devices() const { return _devices; }
  infer::expected<DeviceInfo, std::error_code> device_info(std::string_view name) const;

  static std::string extract_type(std::string_view name);
  static int extract_device_id(std::string_view name);

 private:
  BackendRegistry() = default;
  struct Entry {
    ProbeFunc probe;
    CreateFunc create;
  };
  std::unordered_map<std::string, Entry> _entries;
  std::vector<DeviceInfo> _devices;
};

void register_hip_backend();
