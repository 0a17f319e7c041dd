// scheduler.hpp — runs a graph whose ops all live on one device backend, the
// case of the KV-cache hot path (the reference's five-pass, multi-backend
// splitter is src/scheduler.cpp:33-302).
//
// execute(): orders the graph, assigns unplaced nodes to the device backend
// (KV CPY/VIEW nodes arrive pinned to the KV storage's backend), stages
// host-resident leaf inputs (positions) into device memory unless the op
// reads them from the host itself (RoPE angle tables), binds activations in
// one reusable device arena (RESHAPE of a contiguous tensor aliases its
// source), and hands the graph to the backend. Work is asynchronous; call
// the backend's synchronize() before reading results.
#pragma once

#include <system_error>
#include <unordered_map>

#include "backend.hpp"
#include "expected.hpp"
#include "graph.hpp"

class Scheduler {
 public:
  explicit Scheduler(Backend *device) : _device(device) {}
  ~Scheduler();
  Scheduler(const Scheduler &) = delete;
  Scheduler &operator=(const Scheduler &) = delete;

  infer::expected<void, std::error_code> execute(Graph &g);
  size_t arena_bytes() const { return _arena_bytes; }

 private:
  Backend *_device;
  void *_arena = nullptr;
  size_t _arena_bytes = 0;
};
