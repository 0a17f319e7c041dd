#include "scheduler.hpp"

#include <vector>

namespace {
size_t align256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

// A VIEW node without memory of its own (OpFactory::view_rows): it takes its
// source's bytes at its offset. KV-cache views are placed by their storage
// when the graph is built and never reach this test.
bool aliases_src(const Tensor *n) {
  return n->op == OperationType::GGML_OP_VIEW && !n->data && n->src[0];
}
}  // namespace

Scheduler::~Scheduler() {
  if (_arena) _device->free(BufferKind::ACTIVATION, _arena);
}

infer::expected<void, std::error_code> Scheduler::execute(Graph &g) {
  if (!_device) return infer::fail(std::errc::invalid_argument);
  if (auto r = g.compute(); !r) return r;

  // placement
  for (Tensor *n : g.nodes()) {
    if (!n->backend) {
      if (!_device->supports_op(n->op, *n)) return infer::fail(std::errc::not_supported);
      n->backend = _device;
      n->device = _device->device_type();
    } else if (n->backend != _device) {
      return infer::fail(std::errc::not_supported);  // one device per graph here
    }
  }

  // host leaves read by device ops: staged copies (one per leaf)
  std::unordered_map<Tensor *, Tensor *> staged;
  std::vector<Tensor *> to_upload;
  for (Tensor *n : g.nodes()) {
    for (int i = 0; i < TENSOR_MAX_SRC; ++i) {
      Tensor *s = n->src[i];
      if (!s) break;
      if (s->op != OperationType::GGML_OP_NONE || s->device != DeviceType::CPU) continue;
      if (_device->accepts_host_src(*n, i)) continue;
      auto it = staged.find(s);
      if (it == staged.end()) {
        auto copy = std::make_unique<Tensor>(*s);
        copy->name = s->name + "_dev";
        copy->data = nullptr;
        copy->src.fill(nullptr);
        copy->set_contiguous_strides();
        copy->backend = _device;
        copy->device = _device->device_type();
        Tensor *c = g.adopt(std::move(copy));
        it = staged.emplace(s, c).first;
        to_upload.push_back(s);
      }
      n->src[i] = it->second;
    }
  }

  // arena layout: staged inputs, then activations in topological order
  size_t total = 0;
  for (Tensor *s : to_upload) total += align256(staged[s]->byte_size());
  for (Tensor *n : g.nodes()) {
    if (n->data) continue;
    if (n->op == OperationType::GGML_OP_RESHAPE && n->src[0] && n->src[0]->is_contiguous()) continue;
    if (aliases_src(n)) continue;
    total += align256(n->byte_size());
  }
  if (total > _arena_bytes) {
    if (auto r = _device->synchronize(); !r) return r;
    if (_arena) _device->free(BufferKind::ACTIVATION, _arena);
    _arena = nullptr;
    _arena_bytes = 0;
    auto mem = _device->alloc(BufferKind::ACTIVATION, total);
    if (!mem) return infer::unexpected(mem.error());
    _arena = *mem;
    _arena_bytes = total;
  }
  char *cursor = static_cast<char *>(_arena);
  for (Tensor *s : to_upload) {
    staged[s]->data = cursor;
    cursor += align256(staged[s]->byte_size());
  }
  for (Tensor *n : g.nodes()) {
    if (n->data) continue;
    if (n->op == OperationType::GGML_OP_RESHAPE && n->src[0] && n->src[0]->is_contiguous()) {
      n->data = n->src[0]->data;  // same bytes, new shape
      continue;
    }
    if (aliases_src(n)) {
      n->data = static_cast<char *>(n->src[0]->data) + n->offset;  // rows of the source
      continue;
    }
    n->data = cursor;
    cursor += align256(n->byte_size());
  }
  for (Tensor *s : to_upload)
    if (auto r = _device->copy_tensor_set(staged[s], s->data, 0, s->byte_size()); !r) return r;

  return _device->compute(g);
}
