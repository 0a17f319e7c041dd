// memory_pool.hpp — physical allocators and the per-kind pools every backend
// owns (reference include/memoryPool.hpp:9-73, include/memoryPools/
// naivePool.hpp:6-21). The host allocator keeps the engine testable without
// a device; the HIP allocator puts WEIGHTS / ACTIVATION / KVCACHE in HBM.
#pragma once

#include <cstddef>
#include <cstdlib>
#include <system_error>

#include "expected.hpp"

class PhysicalAllocator {
 public:
  virtual ~PhysicalAllocator() = default;
  virtual infer::expected<void *, std::error_code> raw_alloc(size_t bytes) = 0;
  virtual void raw_free(void *ptr) = 0;
};

// malloc-backed, as CPUPhysicalAllocator (include/memoryPool.hpp:16-34).
class HostPhysicalAllocator : public PhysicalAllocator {
 public:
  infer::expected<void *, std::error_code> raw_alloc(size_t bytes) override {
    if (bytes == 0) return static_cast<void *>(nullptr);
    void *p = std::malloc(bytes);
    if (!p) return infer::fail(std::errc::not_enough_memory);
    return p;
  }
  void raw_free(void *ptr) override { std::free(ptr); }
};

// hipMalloc-backed device memory (the CUDAPhysicalAllocator of
// include/memoryPool.hpp:37-54). The caller must have selected the device.
class HIPPhysicalAllocator : public PhysicalAllocator {
 public:
  infer::expected<void *, std::error_code> raw_alloc(size_t bytes) override;
  void raw_free(void *ptr) override;
};

// hipHostMalloc-backed pinned host memory: the host tier of the KV offload
// storage, which the DMA engines copy to and from HBM directly.
class PinnedHostAllocator : public PhysicalAllocator {
 public:
  infer::expected<void *, std::error_code> raw_alloc(size_t bytes) override;
  void raw_free(void *ptr) override;
};

class MemoryPool {
 public:
  explicit MemoryPool(PhysicalAllocator &a) : _phys_allocator(&a) {}
  virtual ~MemoryPool() = default;
  virtual infer::expected<void *, std::error_code> alloc(size_t bytes) = 0;
  virtual void free(void *ptr) = 0;

 protected:
  PhysicalAllocator *_phys_allocator;
};

// Forwards every request to the physical allocator (no strategy).
class NaivePool : public MemoryPool {
 public:
  explicit NaivePool(PhysicalAllocator &a) : MemoryPool(a) {}
  infer::expected<void *, std::error_code> alloc(size_t bytes) override {
    return _phys_allocator->raw_alloc(bytes);
  }
  void free(void *ptr) override { _phys_allocator->raw_free(ptr); }
};
