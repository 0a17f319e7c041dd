#include "hip_backend.hpp"

#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/ikv.h"
#include "../../include/ikv_model.h"
#include "op_params.hpp"

namespace {

// C-ABI return code -> error_code: negative errno as std::errc, positive
// hipError_t as io_error (the mapping of check_cuda, reference
// include/cuda_util.hpp:7-16).
infer::expected<void, std::error_code> check_ikv(int rc, const char *what) {
  if (rc == 0) return {};
  if (rc < 0) return infer::unexpected(std::make_error_code(static_cast<std::errc>(-rc)));
  std::fprintf(stderr, "[hip] %s: %s\n", what, hipGetErrorString(static_cast<hipError_t>(rc)));
  return infer::fail(std::errc::io_error);
}

infer::expected<void, std::error_code> check_hip(hipError_t e, const char *what) {
  if (e == hipSuccess) return {};
  std::fprintf(stderr, "[hip] %s: %s\n", what, hipGetErrorString(e));
  return infer::fail(std::errc::io_error);
}

// Host -> device copies this small ride in a kernel's arguments: the runtime
// takes the bytes at launch, so the caller's buffer is free on return and the
// write is ordered on the stream like any launch, with no stream
// synchronisation (a paged cache's block-table entries, written when a step
// opens a block, are the common case: 28 synchronous copies there stalled the
// decode pipeline every time a block opened).
constexpr size_t kArgCopyBytes = 256;
struct ArgBytes {
  unsigned char b[kArgCopyBytes];
};
__global__ void set_bytes_kernel(unsigned char *dst, ArgBytes src, int n) {
  const int i = static_cast<int>(threadIdx.x);
  if (i < n) dst[i] = src.b[i];
}

bool contiguous_f32(const Tensor *t) {
  return t && t->data && t->dataType == GGML_TYPE_F32 && t->is_contiguous();
}

// A KV CPY or VIEW node of a paged layer (append_kv_paged): the block table
// rides in src[1], (block_tokens, pool blocks, first token) in op_params.
bool is_paged(const Tensor *t) {
  return t && (t->op == OperationType::GGML_OP_CPY || t->op == OperationType::GGML_OP_VIEW) &&
         t->src[1] && t->src[1]->dataType == GGML_TYPE_I32 && t->src[1]->data;
}

ikv_kv_pages pages_of(const Tensor *t, int *status) {
  return ikv_kv_pages{static_cast<const int32_t *>(t->src[1]->data), t->op_params[0],
                      t->op_params[1], status};
}

}  // namespace

// ---------------------------------------------------------------------------
// HBM allocator

infer::expected<void *, std::error_code> HIPPhysicalAllocator::raw_alloc(size_t bytes) {
  if (bytes == 0) return static_cast<void *>(nullptr);
  void *p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess || !p) {
    (void)hipGetLastError();
    return infer::fail(std::errc::not_enough_memory);
  }
  return p;
}

void HIPPhysicalAllocator::raw_free(void *ptr) {
  if (ptr) (void)hipFree(ptr);
}

infer::expected<void *, std::error_code> PinnedHostAllocator::raw_alloc(size_t bytes) {
  if (bytes == 0) return static_cast<void *>(nullptr);
  void *p = nullptr;
  if (hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess || !p) {
    (void)hipGetLastError();
    return infer::fail(std::errc::not_enough_memory);
  }
  return p;
}

void PinnedHostAllocator::raw_free(void *ptr) {
  if (ptr) (void)hipHostFree(ptr);
}

// ---------------------------------------------------------------------------
// pinned host backend: the host tier of OffloadKVStorage

PinnedHostBackend::PinnedHostBackend(int device_id)
    : Backend(device_id, {"host:" + std::to_string(device_id), DeviceType::CPU, 0}, {}) {
  init_pools(std::make_unique<PinnedHostAllocator>());
}

infer::expected<void, std::error_code> PinnedHostBackend::copy_tensor_set(Tensor *t, const void *d,
                                                                          size_t off, size_t n) {
  if (!t || !t->data || !d || off + n > t->byte_size()) return infer::fail(std::errc::invalid_argument);
  std::memcpy(static_cast<char *>(t->data) + off, d, n);
  return {};
}

infer::expected<void, std::error_code> PinnedHostBackend::copy_tensor_get(const Tensor *t, void *d,
                                                                          size_t off, size_t n) {
  if (!t || !t->data || !d || off + n > t->byte_size()) return infer::fail(std::errc::invalid_argument);
  std::memcpy(d, static_cast<const char *>(t->data) + off, n);
  return {};
}

// ---------------------------------------------------------------------------
// registration

std::vector<DeviceInfo> probe_hip_devices() {
  std::vector<DeviceInfo> devices;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess) {
    (void)hipGetLastError();
    return devices;
  }
  int prev = 0;
  const bool restore = hipGetDevice(&prev) == hipSuccess;
  for (int i = 0; i < count; ++i) {
    if (hipSetDevice(i) != hipSuccess) continue;
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) continue;
    devices.push_back({"hip:" + std::to_string(i), DeviceType::HIP, free_b});
  }
  if (restore) (void)hipSetDevice(prev);
  return devices;
}

void register_hip_backend() {
  BackendRegistry::instance().register_backend(
      "hip", [] { return probe_hip_devices(); },
      [](int device_id, DeviceInfo info, const PoolConfig &cfg) -> std::unique_ptr<Backend> {
        return std::make_unique<HIPBackend>(device_id, std::move(info), cfg);
      });
}

// ---------------------------------------------------------------------------

HIPBackend::HIPBackend(int device_id, DeviceInfo info, const PoolConfig &cfg)
    : Backend(device_id, std::move(info), cfg) {
  init_pools(std::make_unique<HIPPhysicalAllocator>());
  (void)hipSetDevice(_device_id);
  (void)hipStreamCreate(&_stream);
  if (hipMalloc(reinterpret_cast<void **>(&_status), sizeof(int)) == hipSuccess)
    (void)hipMemset(_status, 0, sizeof(int));
}

HIPBackend::~HIPBackend() {
  (void)hipSetDevice(_device_id);
  if (_stream) (void)hipStreamSynchronize(_stream);
  for (auto &t : _tables) {
    (void)hipFree(t.sin);
    (void)hipFree(t.cos);
  }
  if (_workspace) (void)hipFree(_workspace);
  if (_status) (void)hipFree(_status);
  if (_stream) (void)hipStreamDestroy(_stream);
}

infer::expected<void, std::error_code> HIPBackend::set_device() const {
  return check_hip(hipSetDevice(_device_id), "hipSetDevice");
}

bool HIPBackend::supports_op(OperationType op, const Tensor &t) const {
  (void)t;
  switch (op) {
    case OperationType::GGML_OP_NONE:
    case OperationType::GGML_OP_CPY:
    case OperationType::GGML_OP_VIEW:
    case OperationType::GGML_OP_RESHAPE:
    case OperationType::GGML_OP_RMS_NORM:
    case OperationType::GGML_OP_ROPE:
    case OperationType::GGML_OP_FLASH_ATTN_EXT:
    case OperationType::GGML_OP_GET_ROWS:
    case OperationType::GGML_OP_MUL_MAT:
    case OperationType::GGML_OP_ADD:
    case OperationType::GGML_OP_MUL:
      return true;
    case OperationType::GGML_OP_UNARY: {
      uint32_t sub = 0;
      std::memcpy(&sub, &t.op_params[0], sizeof(sub));
      return sub == static_cast<uint32_t>(UnaryOp::GGML_UNARY_OP_SILU);
    }
    default:
      return false;
  }
}

bool HIPBackend::accepts_host_src(const Tensor &node, int src_index) const {
  return node.op == OperationType::GGML_OP_ROPE && src_index == 2;
}

infer::expected<void *, std::error_code> HIPBackend::alloc(BufferKind kind, size_t bytes) {
  if (auto r = set_device(); !r) return infer::unexpected(r.error());
  return Backend::alloc(kind, bytes);
}

void HIPBackend::free(BufferKind kind, void *ptr) {
  (void)hipSetDevice(_device_id);
  Backend::free(kind, ptr);
}

infer::expected<void, std::error_code> HIPBackend::copy_tensor_set(Tensor *tensor, const void *data,
                                                                   size_t offset, size_t size) {
  if (!tensor || !tensor->data || !data) return infer::fail(std::errc::invalid_argument);
  if (offset + size > tensor->byte_size()) return infer::fail(std::errc::invalid_argument);
  if (auto r = set_device(); !r) return r;
  if (size == 0) return {};
  if (size <= kArgCopyBytes) {
    ArgBytes a;
    std::memcpy(a.b, data, size);
    set_bytes_kernel<<<1, kArgCopyBytes, 0, _stream>>>(
        static_cast<unsigned char *>(tensor->data) + offset, a, static_cast<int>(size));
    return check_hip(hipGetLastError(), "copy_tensor_set (kernel argument)");
  }
  auto r = check_hip(hipMemcpyAsync(static_cast<char *>(tensor->data) + offset, data, size,
                                    hipMemcpyHostToDevice, _stream),
                     "copy_tensor_set");
  if (!r) return r;
  return check_hip(hipStreamSynchronize(_stream), "copy_tensor_set sync");
}

infer::expected<void, std::error_code> HIPBackend::copy_tensor_get(const Tensor *tensor, void *data,
                                                                   size_t offset, size_t size) {
  if (!tensor || !tensor->data || !data) return infer::fail(std::errc::invalid_argument);
  if (offset + size > tensor->byte_size()) return infer::fail(std::errc::invalid_argument);
  if (auto r = set_device(); !r) return r;
  auto r = check_hip(hipMemcpyAsync(data, static_cast<const char *>(tensor->data) + offset, size,
                                    hipMemcpyDeviceToHost, _stream),
                     "copy_tensor_get");
  if (!r) return r;
  return check_hip(hipStreamSynchronize(_stream), "copy_tensor_get sync");
}

infer::expected<bool, std::error_code> HIPBackend::copy_tensor_high(const Tensor *src,
                                                                    Tensor *dst) const {
  if (!src || !dst || !src->backend || !dst->data || !src->data) return false;
  if (src->device != DeviceType::HIP) return false;  // host sources go through copy_tensor_set
  const auto *peer = dynamic_cast<const HIPBackend *>(src->backend);
  if (!peer) return infer::fail(std::errc::invalid_argument);
  if (src->byte_size() != dst->byte_size()) return infer::fail(std::errc::invalid_argument);
  if (auto r = set_device(); !r) return infer::unexpected(r.error());
  hipError_t e;
  if (peer->_device_id == _device_id)
    e = hipMemcpyAsync(dst->data, src->data, src->byte_size(), hipMemcpyDeviceToDevice, _stream);
  else  // over xGMI when peer access is enabled, staged by the runtime otherwise
    e = hipMemcpyPeerAsync(dst->data, _device_id, src->data, peer->_device_id, src->byte_size(),
                           _stream);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return true;
}

infer::expected<void, std::error_code> HIPBackend::synchronize() {
  if (auto r = set_device(); !r) return r;
  if (auto r = check_hip(hipStreamSynchronize(_stream), "synchronize"); !r) return r;
  int status = 0;
  if (_status) {
    if (auto r = check_hip(hipMemcpy(&status, _status, sizeof(int), hipMemcpyDeviceToHost), "status");
        !r)
      return r;
  }
  if (status != 0) {
    (void)hipMemset(_status, 0, sizeof(int));
    if (status & IKV_STATUS_POSITION)
      std::fprintf(stderr, "[hip] RoPE position outside the angle table\n");
    if (status & IKV_STATUS_BLOCK)
      std::fprintf(stderr, "[hip] paged block-table entry outside the pool (its rows were "
                           "read from block 0 and its writes dropped)\n");
    if (status & IKV_STATUS_TOKEN)
      std::fprintf(stderr, "[hip] token id outside the embedding table\n");
    return infer::fail(std::errc::invalid_argument);
  }
  return {};
}

infer::expected<void, std::error_code> HIPBackend::ensure_workspace(size_t bytes) {
  if (bytes <= _workspace_bytes) return {};
  if (_workspace) {
    (void)hipStreamSynchronize(_stream);
    (void)hipFree(_workspace);
    _workspace = nullptr;
    _workspace_bytes = 0;
  }
  if (hipMalloc(&_workspace, bytes) != hipSuccess) {
    (void)hipGetLastError();
    _workspace = nullptr;
    return infer::fail(std::errc::not_enough_memory);
  }
  // The decode kernel's arrival counters live in the workspace and must start
  // at zero; every launch leaves them at zero again.
  if (hipMemset(_workspace, 0, bytes) != hipSuccess) {
    (void)hipGetLastError();
    (void)hipFree(_workspace);
    _workspace = nullptr;
    return infer::fail(std::errc::io_error);
  }
  _workspace_bytes = bytes;
  return {};
}

infer::expected<void, std::error_code> HIPBackend::reserve_decode_workspace(int n_head,
                                                                           int n_head_kv,
                                                                           int head_dim,
                                                                           int64_t max_kv) {
  if (auto r = set_device(); !r) return r;
  return ensure_workspace(decode_workspace_reservation(n_head, n_head_kv, head_dim, max_kv));
}

size_t HIPBackend::decode_workspace_reservation(int n_head, int n_head_kv, int head_dim,
                                                int64_t max_kv) {
  // The split count is not monotone in n_kv (it peaks where a split's tile
  // count steps down), so every context is asked; a few ns each, once.
  size_t need = 0;
  for (int64_t n = 1; n <= max_kv; ++n)
    need = std::max(need, ikv_attn_decode_workspace_bytes(n_head, n_head_kv, head_dim, n));
  return need;
}

infer::expected<const HIPBackend::RopeTables *, std::error_code> HIPBackend::rope_tables(
    const Tensor &theta) {
  if (auto it = _rope.find(theta.data); it != _rope.end()) return &_tables[it->second];
  if (theta.dataType != GGML_TYPE_F32 || !theta.data) return infer::fail(std::errc::invalid_argument);
  const int64_t half = theta.dims[0];
  const int64_t n_ctx = theta.dims[1];
  if (half <= 0 || n_ctx <= 0) return infer::fail(std::errc::invalid_argument);
  const size_t count = static_cast<size_t>(half * n_ctx);
  const bool on_host = theta.device == DeviceType::CPU;

  // Content key: the dims and row 1 (the frequencies, which fix theta_base
  // and head_dim). A table staged to the device at a new address each step
  // then maps to the sin/cos tables already built for it.
  std::vector<float> row1(static_cast<size_t>(half), 0.f);
  if (n_ctx > 1) {
    const float *src = static_cast<const float *>(theta.data) + half;
    if (on_host)
      std::memcpy(row1.data(), src, row1.size() * sizeof(float));
    else if (auto r = check_hip(hipMemcpy(row1.data(), src, row1.size() * sizeof(float),
                                          hipMemcpyDeviceToHost),
                                "rope table key");
             !r)
      return infer::unexpected(r.error());
  }
  std::string key(reinterpret_cast<const char *>(&half), sizeof(half));
  key.append(reinterpret_cast<const char *>(&n_ctx), sizeof(n_ctx));
  key.append(reinterpret_cast<const char *>(row1.data()), row1.size() * sizeof(float));
  if (auto it = _rope_by_content.find(key); it != _rope_by_content.end()) {
    _rope.emplace(theta.data, it->second);
    return &_tables[it->second];
  }

  std::vector<float> host(count), s(count), c(count);
  if (on_host) {
    std::memcpy(host.data(), theta.data, count * sizeof(float));
  } else if (auto r = check_hip(hipMemcpy(host.data(), theta.data, count * sizeof(float),
                                          hipMemcpyDeviceToHost),
                                "rope table");
             !r) {
    return infer::unexpected(r.error());
  }
  if (auto r = check_ikv(ikv_rope_sincos_table_f32(host.data(), count, s.data(), c.data()), "sincos");
      !r)
    return infer::unexpected(r.error());
  RopeTables t;
  t.half = half;
  t.n_ctx = n_ctx;
  if (hipMalloc(reinterpret_cast<void **>(&t.sin), count * sizeof(float)) != hipSuccess ||
      hipMalloc(reinterpret_cast<void **>(&t.cos), count * sizeof(float)) != hipSuccess) {
    (void)hipGetLastError();
    (void)hipFree(t.sin);
    return infer::fail(std::errc::not_enough_memory);
  }
  if (auto r = check_hip(hipMemcpy(t.sin, s.data(), count * sizeof(float), hipMemcpyHostToDevice),
                         "sin upload");
      !r)
    return infer::unexpected(r.error());
  if (auto r = check_hip(hipMemcpy(t.cos, c.data(), count * sizeof(float), hipMemcpyHostToDevice),
                         "cos upload");
      !r)
    return infer::unexpected(r.error());
  _tables.push_back(t);
  const size_t idx = _tables.size() - 1;
  _rope_by_content.emplace(std::move(key), idx);
  _rope.emplace(theta.data, idx);
  return &_tables[idx];
}

infer::expected<void, std::error_code> HIPBackend::compute(Graph &graph) {
  if (auto r = set_device(); !r) return r;
  _stats = Stats{};
  _norm_into_rope.clear();
  _append_into_attn.clear();
  _swiglu.clear();
  _silu_mul.clear();
  _residual.clear();
  _qkv.clear();
  _norm_into_mm.clear();
  _rope_into_attn.clear();
  _qkv_attn.clear();
  _attn_done.clear();
  _out_into_cpy.clear();
  _skip.clear();

  if (_fusion) {
    std::unordered_map<const Tensor *, int> uses;
    for (Tensor *n : graph.nodes())
      for (Tensor *s : n->src)
        if (s) ++uses[s];
    for (Tensor *o : graph.outputs()) ++uses[o];
    for (Tensor *n : graph.nodes()) {
      if (n->op == OperationType::GGML_OP_ROPE) {
        const Tensor *nm = n->src[0];
        if (nm && nm->op == OperationType::GGML_OP_RMS_NORM && uses[nm] == 1 &&
            nm->dims == n->dims && nm->src[1] && nm->src[1]->element_count() == size_t(n->dims[0])) {
          _norm_into_rope[n] = nm;
          _skip[nm] = true;
        }
      }
      if (n->op == OperationType::GGML_OP_FLASH_ATTN_EXT && n->src[0] && n->src[0]->dims[2] == 1) {
        const Tensor *kv = n->src[1], *vv = n->src[2];
        if (!kv || !vv || kv->op != OperationType::GGML_OP_VIEW || vv->op != OperationType::GGML_OP_VIEW)
          continue;
        const Tensor *kc = kv->src[0], *vc = vv->src[0];
        if (!kc || !vc || kc->op != OperationType::GGML_OP_CPY || vc->op != OperationType::GGML_OP_CPY)
          continue;
        if (uses[kv] != 1 || uses[vv] != 1 || uses[kc] != 1 || uses[vc] != 1) continue;
        const int64_t n_kv = kv->dims[2];
        AttnParams p;
        std::memcpy(&p, n->op_params, sizeof(p));
        const size_t row = static_cast<size_t>(kv->dims[0] * kv->dims[1]) * 4;
        // the copies write exactly the last row the views read: by address
        // for a contiguous cache, by logical token for a paged one
        auto last_row = [&](const Tensor *c, const Tensor *view) {
          if (c->dims[2] != 1 || c->dims[3] != 1 || is_paged(c) != is_paged(view)) return false;
          if (is_paged(c))
            return c->src[1] == view->src[1] && c->data == view->data &&
                   int64_t(c->op_params[2]) == n_kv - 1;
          return c->data == static_cast<char *>(view->data) + (n_kv - 1) * row;
        };
        const bool last_row_k = last_row(kc, kv);
        const bool last_row_v = last_row(vc, vv);
        if (!last_row_k || !last_row_v || int64_t(p.n_ctx) + 1 != n_kv) continue;
        if (!contiguous_f32(kc->src[0]) || !contiguous_f32(vc->src[0])) continue;
        _append_into_attn[n] = {kc->src[0], vc->src[0]};
        _skip[kc] = true;
        _skip[vc] = true;
      }
    }
    plan_model_fusions(graph, uses);
  }

  for (Tensor *node : graph.nodes()) {
    if (node->op == OperationType::GGML_OP_NONE) continue;
    if (_skip.count(node)) continue;
    if (auto r = dispatch(node); !r) {
      std::fprintf(stderr, "[hip] compute failed at node %s op=%u\n", node->name.c_str(),
                   static_cast<unsigned>(node->op));
      return r;
    }
  }
  return {};
}

namespace {

bool is_mm(const Tensor *t) { return t && t->op == OperationType::GGML_OP_MUL_MAT; }

bool is_silu(const Tensor *t) {
  if (!t || t->op != OperationType::GGML_OP_UNARY) return false;
  uint32_t sub = 0;
  std::memcpy(&sub, &t->op_params[0], sizeof(sub));
  return sub == static_cast<uint32_t>(UnaryOp::GGML_UNARY_OP_SILU);
}

// Weight [K, N] times activation [K, M] with contiguous F32 operands.
bool mm_operands_ok(const Tensor *mm) {
  const Tensor *w = mm->src[0], *x = mm->src[1];
  return contiguous_f32(w) && contiguous_f32(x) && w->dims[0] == x->dims[0] && w->dims[2] == 1 &&
         w->dims[3] == 1 && x->dims[2] == 1 && x->dims[3] == 1;
}

}  // namespace

// Model-level fusions of the Qwen3 graph (src/models/Qwen3.cpp:53-113):
//  * MUL(up, SILU(gate)) with gate = MUL_MAT(w_gate, x), up = MUL_MAT(w_up, x)
//    and one token -> one ikv_gemv_swiglu_f32; with several tokens the SILU
//    and MUL -> one ikv_silu_mul_f32 pass;
//  * ADD(MUL_MAT(w, x), r) -> the product with the residual added in its
//    epilogue (o_proj and ffn_down);
//  * three single-token MUL_MATs of one input (q, k, v) -> one ikv_gemv3_f32.
// Every fused intermediate has exactly one use.
void HIPBackend::plan_model_fusions(Graph &graph, std::unordered_map<const Tensor *, int> &uses) {
  for (Tensor *n : graph.nodes()) {
    if (n->op != OperationType::GGML_OP_MUL || !n->src[0] || !n->src[1]) continue;
    for (int side = 0; side < 2; ++side) {
      const Tensor *up = n->src[side], *act = n->src[1 - side];
      if (!is_mm(up) || !is_silu(act) || !is_mm(act->src[0])) continue;
      const Tensor *gate = act->src[0];
      if (up->src[1] != gate->src[1] || up->src[1]->dims[1] != 1) continue;
      if (uses[up] != 1 || uses[act] != 1 || uses[gate] != 1) continue;
      if (!mm_operands_ok(up) || !mm_operands_ok(gate) || up->dims != gate->dims) continue;
      _swiglu[n] = {gate, up};
      _skip[up] = _skip[act] = _skip[gate] = true;
      break;
    }
  }
  // The remaining MUL(up, SILU(gate)) pairs (several tokens: the projections
  // are separate GEMMs) -> one elementwise pass, up * silu(gate).
  for (Tensor *n : graph.nodes()) {
    if (n->op != OperationType::GGML_OP_MUL || _swiglu.count(n) || !n->src[0] || !n->src[1]) continue;
    for (int side = 0; side < 2; ++side) {
      const Tensor *act = n->src[1 - side], *up = n->src[side];
      if (!is_silu(act) || uses[act] != 1 || !act->src[0]) continue;
      const Tensor *gate = act->src[0];
      if (!contiguous_f32(gate) || !contiguous_f32(up) || gate->dims != n->dims || up->dims != n->dims)
        continue;
      _silu_mul[n] = {gate, up};
      _skip[act] = true;
      break;
    }
  }
  for (Tensor *n : graph.nodes()) {
    if (n->op != OperationType::GGML_OP_ADD || !n->src[0] || !n->src[1]) continue;
    for (int side = 0; side < 2; ++side) {
      const Tensor *mm = n->src[side], *res = n->src[1 - side];
      if (!is_mm(mm) || _skip.count(mm) || uses[mm] != 1 || !mm_operands_ok(mm)) continue;
      if (!contiguous_f32(res) || res->dims != mm->dims) continue;
      _residual[n] = {mm, res};
      _skip[mm] = true;
      break;
    }
  }
  std::unordered_map<const Tensor *, std::vector<const Tensor *>> by_input;
  std::vector<const Tensor *> order;
  for (Tensor *n : graph.nodes()) {
    if (!is_mm(n) || _skip.count(n) || !mm_operands_ok(n) || n->src[1]->dims[1] != 1) continue;
    auto &v = by_input[n->src[1]];
    if (v.empty()) order.push_back(n->src[1]);
    v.push_back(n);
  }
  for (const Tensor *x : order) {
    const auto &v = by_input[x];
    if (v.size() != 3) continue;
    _qkv[v[0]] = {v[0], v[1], v[2]};
    _skip[v[1]] = _skip[v[2]] = true;
  }
  // The single-row RMS_NORM feeding a q/k/v group (attn_norm) or a SwiGLU
  // pair (ffn_norm), and nothing else, is folded into that launch.
  auto foldable_norm = [&](const Tensor *x, int consumers) {
    if (!x || x->op != OperationType::GGML_OP_RMS_NORM || uses[x] != consumers) return false;
    const Tensor *in = x->src[0], *w = x->src[1];
    return contiguous_f32(in) && contiguous_f32(w) && in->dims == x->dims && x->dims[1] == 1 &&
           x->dims[2] == 1 && x->dims[3] == 1 && x->dims[0] % 1024 == 0 &&
           w->element_count() == static_cast<size_t>(x->dims[0]);
  };
  for (const auto &[first, group] : _qkv) {
    const Tensor *x = first->src[1];
    if (foldable_norm(x, 3)) {
      _norm_into_mm[first] = x;
      _skip[x] = true;
    }
  }
  for (const auto &[mul, pair] : _swiglu) {
    const Tensor *x = pair.first->src[1];
    if (foldable_norm(x, 2)) {
      _norm_into_mm[mul] = x;
      _skip[x] = true;
    }
  }
  // qk-RMSNorm + RoPE of a one-token step folded into its decode launch.
  for (const auto &[attn, kv_src] : _append_into_attn) {
    const Tensor *qr = attn->src[0], *kr = kv_src.first;
    if (!qr || !kr || qr->op != OperationType::GGML_OP_ROPE || kr->op != OperationType::GGML_OP_ROPE)
      continue;
    if (!_norm_into_rope.count(qr) || !_norm_into_rope.count(kr) || uses[qr] != 1 || uses[kr] != 1)
      continue;
    if (qr->src[1] != kr->src[1] || qr->src[2] != kr->src[2]) continue;  // same positions, table
    const Tensor *qn = _norm_into_rope[qr], *kn = _norm_into_rope[kr];
    if (std::memcmp(&qn->op_params[0], &kn->op_params[0], sizeof(float)) != 0) continue;  // same eps
    if (!contiguous_f32(qn->src[0]) || !contiguous_f32(kn->src[0])) continue;
    _rope_into_attn[attn] = {qr, kr};
    _skip[qr] = _skip[kr] = true;
  }
  // A q/k/v group whose three outputs are exactly that decode's q, k and v
  // inputs (contiguous cache): the decode may run inside the q/k/v launch.
  for (const auto &[attn, ropes] : _rope_into_attn) {
    const Tensor *k = attn->src[1], *v = attn->src[2];
    if (!k || !v || is_paged(k) || is_paged(v)) continue;
    const Tensor *qsrc = _norm_into_rope[ropes.first]->src[0];
    const Tensor *ksrc = _norm_into_rope[ropes.second]->src[0];
    const Tensor *vsrc = _append_into_attn[attn].second;
    for (const auto &[first, group] : _qkv) {
      if (group[0]->data == qsrc->data && group[1]->data == ksrc->data &&
          group[2]->data == vsrc->data) {
        _qkv_attn[first] = attn;
        break;
      }
    }
  }
  // A cache append (CPY into a contiguous cache view) whose source is a RoPE
  // output or a product, through aliasing reshapes, and read by nothing else:
  // the producer writes the cache rows itself (src/model.cpp:602-625's CPY
  // folded into the k RoPE and the v projection of a prefill).
  for (Tensor *c : graph.nodes()) {
    if (c->op != OperationType::GGML_OP_CPY || _skip.count(c) || is_paged(c) || !c->is_contiguous())
      continue;
    const Tensor *p = c->src[0];
    bool sole = p && uses[p] == 1;
    while (sole && p->op == OperationType::GGML_OP_RESHAPE && p->src[0] && p->data == p->src[0]->data) {
      p = p->src[0];
      sole = uses[p] == 1;
    }
    if (!sole || _skip.count(p) || p->byte_size() != c->byte_size() || !p->is_contiguous()) continue;
    const bool rope = p->op == OperationType::GGML_OP_ROPE;
    const bool plain_mm = is_mm(p) && !_qkv.count(p) && mm_operands_ok(p);
    if (!rope && !plain_mm) continue;
    _out_into_cpy[p] = c;
    _skip[c] = true;
  }
}

infer::expected<HIPBackend::DecodeRopeArgs, std::error_code> HIPBackend::decode_rope_args(
    const Tensor *attn) {
  const auto rf = _rope_into_attn.find(attn);
  const auto ap = _append_into_attn.find(attn);
  if (rf == _rope_into_attn.end() || ap == _append_into_attn.end())
    return infer::fail(std::errc::invalid_argument);
  const Tensor *qr = rf->second.first, *kr = rf->second.second;
  const Tensor *qn = _norm_into_rope[qr], *kn = _norm_into_rope[kr];
  const Tensor *pos = qr->src[1];
  if (!pos || !pos->data || pos->dataType != GGML_TYPE_I32 || !qr->src[2])
    return infer::fail(std::errc::invalid_argument);
  auto tab = rope_tables(*qr->src[2]);
  if (!tab) return infer::unexpected(tab.error());
  DecodeRopeArgs a;
  a.q_raw = static_cast<const float *>(qn->src[0]->data);
  a.k_raw = static_cast<const float *>(kn->src[0]->data);
  a.v_new = static_cast<const float *>(ap->second.second->data);
  a.q_norm_w = static_cast<const float *>(qn->src[1]->data);
  a.k_norm_w = static_cast<const float *>(kn->src[1]->data);
  std::memcpy(&a.eps, &qn->op_params[0], sizeof(a.eps));
  a.pos = static_cast<const int32_t *>(pos->data);
  a.tab = *tab;
  return a;
}

infer::expected<void, std::error_code> HIPBackend::dispatch_qkv_decode(const Tensor *first,
                                                                       const Tensor *attn) {
  const auto g = _qkv.find(first);
  if (g == _qkv.end()) return infer::fail(std::errc::invalid_argument);
  const Tensor *a = g->second[0], *b = g->second[1], *c = g->second[2];
  const Tensor *q = attn->src[0], *k = attn->src[1], *v = attn->src[2];
  AttnParams p;
  std::memcpy(&p, attn->op_params, sizeof(p));
  const int64_t D = q->dims[0], Hq = q->dims[1], nkv = k->dims[2], Hkv = k->dims[1];
  if (q->dims[2] != 1 || nkv != static_cast<int64_t>(p.n_ctx) + 1 || !attn->data)
    return infer::fail(std::errc::not_supported);
  const Tensor *xin = first->src[1], *nw = nullptr;
  float attn_eps = 0.f;
  if (const auto f = _norm_into_mm.find(first); f != _norm_into_mm.end()) {
    xin = f->second->src[0];
    nw = f->second->src[1];
    std::memcpy(&attn_eps, &f->second->op_params[0], sizeof(attn_eps));
  }
  auto args = decode_rope_args(attn);
  if (!args) return infer::unexpected(args.error());
  if (_replay_max > 0 && (is_paged(k) || nkv > _replay_max)) return infer::fail(std::errc::not_supported);
  const int64_t plan_kv = _replay_max > 0 ? _replay_max : nkv;
  const size_t need = ikv_attn_decode_workspace_bytes(int(Hq), int(Hkv), int(D), plan_kv);
  if (auto r = ensure_workspace(need); !r) return r;
  const int rc = (_replay_max > 0 ? ikv_qkv_attn_decode_replay_f32 : ikv_qkv_attn_decode_f32)(
      static_cast<const float *>(a->src[0]->data), static_cast<const float *>(b->src[0]->data),
      static_cast<const float *>(c->src[0]->data), static_cast<const float *>(xin->data),
      nw ? static_cast<const float *>(nw->data) : nullptr, attn_eps, static_cast<float *>(a->data),
      static_cast<float *>(b->data), static_cast<float *>(c->data), first->src[0]->dims[0],
      static_cast<float *>(k->data), static_cast<float *>(v->data),
      static_cast<float *>(attn->data), int(Hq), int(Hkv), int(D), plan_kv, p.scale,
      args->q_norm_w, args->k_norm_w, args->eps, args->pos, args->tab->sin, args->tab->cos,
      args->tab->n_ctx, _status, _workspace, _workspace_bytes, _stream);
  if (rc == -ENOTSUP) return infer::fail(std::errc::not_supported);
  if (auto r = check_ikv(rc, "qkv_attn_decode"); !r) return r;
  _attn_done[attn] = true;
  ++_stats.fused_qkv;
  ++_stats.fused_qkv_decode;
  ++_stats.fused_rope_decode;
  ++_stats.fused_append_decode;
  if (nw) ++_stats.fused_norm_mm;
  return {};
}

infer::expected<void, std::error_code> HIPBackend::dispatch(Tensor *node) {
  void *s = _stream;
  switch (node->op) {
    case OperationType::GGML_OP_VIEW:
      return {};

    case OperationType::GGML_OP_CPY: {
      const Tensor *src = node->src[0];
      if (!src || !src->data || !node->data || src->dataType != node->dataType || src->dims != node->dims)
        return infer::fail(std::errc::invalid_argument);
      if (!src->is_contiguous() || !node->is_contiguous()) return infer::fail(std::errc::not_supported);
      const size_t rows = static_cast<size_t>(node->dims[2] * node->dims[3]);
      const size_t row_bytes = static_cast<size_t>(node->dims[0] * node->dims[1]) * dataType_size(node->dataType);
      ++_stats.launches;
      if (is_paged(node)) {
        const ikv_kv_pages pg = pages_of(node, _status);
        return check_ikv(ikv_append_paged_f32(node->data, src->data, &pg, node->op_params[2], rows,
                                              row_bytes, s),
                         "append_paged");
      }
      return check_ikv(ikv_append_f32(node->data, src->data, rows, row_bytes, s), "append");
    }

    case OperationType::GGML_OP_RESHAPE: {
      const Tensor *src = node->src[0];
      if (!src || !src->data || !node->data || src->byte_size() != node->byte_size())
        return infer::fail(std::errc::invalid_argument);
      if (node->data == src->data) return {};
      ++_stats.launches;
      return check_ikv(ikv_append_f32(node->data, src->data, 1, src->byte_size(), s), "reshape");
    }

    case OperationType::GGML_OP_RMS_NORM: {
      const Tensor *x = node->src[0], *w = node->src[1];
      if (!contiguous_f32(x) || !contiguous_f32(w) || !node->data || x->dims != node->dims ||
          w->element_count() != static_cast<size_t>(x->dims[0]))
        return infer::fail(std::errc::invalid_argument);
      float eps;
      std::memcpy(&eps, &node->op_params[0], sizeof(eps));
      ++_stats.launches;
      return check_ikv(ikv_rms_norm_f32(static_cast<const float *>(x->data),
                                        static_cast<const float *>(w->data),
                                        static_cast<float *>(node->data),
                                        static_cast<int64_t>(x->element_count() / x->dims[0]),
                                        x->dims[0], eps, s),
                       "rms_norm");
    }

    case OperationType::GGML_OP_ROPE: {
      const Tensor *pos = node->src[1], *theta = node->src[2];
      const auto fused = _norm_into_rope.find(node);
      const Tensor *x = fused != _norm_into_rope.end() ? fused->second->src[0] : node->src[0];
      if (!contiguous_f32(x) || !pos || !pos->data || pos->dataType != GGML_TYPE_I32 || !theta ||
          !node->data || x->dims != node->dims || pos->element_count() != static_cast<size_t>(x->dims[2]))
        return infer::fail(std::errc::invalid_argument);
      if (theta->dims[0] * 2 != x->dims[0]) return infer::fail(std::errc::invalid_argument);
      auto tab = rope_tables(*theta);
      if (!tab) return infer::unexpected(tab.error());
      const RopeTables &t = **tab;
      ++_stats.launches;
      float *rope_out = static_cast<float *>(node->data);
      if (const auto oc = _out_into_cpy.find(node); oc != _out_into_cpy.end()) {
        rope_out = static_cast<float *>(oc->second->data);
        ++_stats.fused_append;
      }
      if (fused != _norm_into_rope.end()) {
        const Tensor *w = fused->second->src[1];
        float eps;
        std::memcpy(&eps, &fused->second->op_params[0], sizeof(eps));
        ++_stats.fused_norm_rope;
        return check_ikv(ikv_qk_norm_rope_f32(static_cast<const float *>(x->data),
                                              static_cast<const float *>(w->data), rope_out,
                                              static_cast<const int32_t *>(pos->data), x->dims[2],
                                              static_cast<int>(x->dims[1]), static_cast<int>(x->dims[0]),
                                              eps, t.sin, t.cos, t.n_ctx, _status, s),
                         "qk_norm_rope");
      }
      return check_ikv(ikv_rope_neox_f32(static_cast<const float *>(x->data), rope_out,
                                         static_cast<const int32_t *>(pos->data), x->dims[2],
                                         static_cast<int>(x->dims[1]), static_cast<int>(x->dims[0]),
                                         t.sin, t.cos, t.n_ctx, _status, s),
                       "rope");
    }

    case OperationType::GGML_OP_FLASH_ATTN_EXT: {
      const Tensor *q = node->src[0], *k = node->src[1], *v = node->src[2];
      if (!contiguous_f32(q) || !contiguous_f32(k) || !contiguous_f32(v) || !node->data)
        return infer::fail(std::errc::invalid_argument);
      AttnParams p;
      std::memcpy(&p, node->op_params, sizeof(p));
      const int64_t D = q->dims[0], Hq = q->dims[1], nq = q->dims[2];
      const int64_t Hkv = k->dims[1], nkv = k->dims[2];
      if (k->dims[0] != D || v->dims[0] != D || v->dims[1] != Hkv || v->dims[2] != nkv || Hkv <= 0 ||
          Hq % Hkv != 0)
        return infer::fail(std::errc::invalid_argument);
      if (_attn_done.count(node)) return {};  // ran inside its q/k/v launch
      ++_stats.launches;
      if (nq == 1 && nkv == static_cast<int64_t>(p.n_ctx) + 1) {
        const auto fused = _append_into_attn.find(node);
        const void *kn = nullptr, *vn = nullptr;
        if (fused != _append_into_attn.end()) {
          kn = fused->second.first->data;
          vn = fused->second.second->data;
          ++_stats.fused_append_decode;
        }
        const bool paged = is_paged(k) && is_paged(v);
        if (_replay_max > 0 && (!_rope_into_attn.count(node) || nkv > _replay_max))
          return infer::fail(std::errc::not_supported);
        const int64_t plan_kv = _replay_max > 0 ? _replay_max : nkv;
        const size_t need = ikv_attn_decode_workspace_bytes(int(Hq), int(Hkv), int(D), plan_kv);
        if (auto r = ensure_workspace(need); !r) return r;
        const ikv_kv_pages pg = paged ? pages_of(k, _status) : ikv_kv_pages{};
        if (_rope_into_attn.count(node)) {
          auto a = decode_rope_args(node);
          if (!a) return infer::unexpected(a.error());
          const RopeTables *tab = a->tab;
          ++_stats.fused_rope_decode;
          if (_replay_max > 0 && paged)
            return check_ikv(ikv_attn_decode_rope_paged_replay_f32(
                                 a->q_raw, a->k_raw, a->v_new, static_cast<float *>(k->data),
                                 static_cast<float *>(v->data), &pg, static_cast<float *>(node->data),
                                 int(Hq), int(Hkv), int(D), plan_kv, p.scale, a->q_norm_w,
                                 a->k_norm_w, a->eps, a->pos, tab->sin, tab->cos, tab->n_ctx,
                                 _status, _workspace, _workspace_bytes, s),
                             "attn_decode_rope_paged_replay");
          if (_replay_max > 0)
            return check_ikv(ikv_attn_decode_rope_replay_f32(
                                 a->q_raw, a->k_raw, a->v_new, static_cast<float *>(k->data),
                                 static_cast<float *>(v->data), static_cast<float *>(node->data),
                                 int(Hq), int(Hkv), int(D), plan_kv, p.scale, a->q_norm_w,
                                 a->k_norm_w, a->eps, a->pos, tab->sin, tab->cos, tab->n_ctx,
                                 _status, _workspace, _workspace_bytes, s),
                             "attn_decode_rope_replay");
          if (paged)
            return check_ikv(ikv_attn_decode_rope_paged_f32(
                                 a->q_raw, a->k_raw, a->v_new, static_cast<float *>(k->data),
                                 static_cast<float *>(v->data), &pg, static_cast<float *>(node->data),
                                 int(Hq), int(Hkv), int(D), nkv, p.scale, a->q_norm_w, a->k_norm_w,
                                 a->eps, a->pos, tab->sin, tab->cos, tab->n_ctx, _status, _workspace,
                                 _workspace_bytes, s),
                             "attn_decode_rope_paged");
          return check_ikv(ikv_attn_decode_rope_f32(
                               a->q_raw, a->k_raw, a->v_new, static_cast<float *>(k->data),
                               static_cast<float *>(v->data), static_cast<float *>(node->data),
                               int(Hq), int(Hkv), int(D), nkv, p.scale, a->q_norm_w, a->k_norm_w,
                               a->eps, a->pos, tab->sin, tab->cos, tab->n_ctx, _status, _workspace,
                               _workspace_bytes, s),
                           "attn_decode_rope");
        }
        if (paged)
          return check_ikv(ikv_attn_decode_paged_f32(
                               static_cast<const float *>(q->data), static_cast<float *>(k->data),
                               static_cast<float *>(v->data), &pg, static_cast<const float *>(kn),
                               static_cast<const float *>(vn), static_cast<float *>(node->data),
                               int(Hq), int(Hkv), int(D), nkv, p.scale, _workspace,
                               _workspace_bytes, s),
                           "attn_decode_paged");
        return check_ikv(ikv_attn_decode_f32(static_cast<const float *>(q->data),
                                             static_cast<float *>(k->data), static_cast<float *>(v->data),
                                             static_cast<const float *>(kn), static_cast<const float *>(vn),
                                             static_cast<float *>(node->data), int(Hq), int(Hkv), int(D),
                                             nkv, p.scale, _workspace, _workspace_bytes, s),
                         "attn_decode");
      }
      if (is_paged(k) && is_paged(v)) {
        const ikv_kv_pages pg = pages_of(k, _status);
        return check_ikv(ikv_attn_prefill_paged_f32(static_cast<const float *>(q->data),
                                                    static_cast<const float *>(k->data),
                                                    static_cast<const float *>(v->data), &pg,
                                                    static_cast<float *>(node->data), int(Hq),
                                                    int(Hkv), int(D), nq, nkv, p.n_ctx, p.scale, s),
                         "attn_prefill_paged");
      }
      return check_ikv(ikv_attn_prefill_f32(static_cast<const float *>(q->data),
                                            static_cast<const float *>(k->data),
                                            static_cast<const float *>(v->data),
                                            static_cast<float *>(node->data), int(Hq), int(Hkv), int(D),
                                            nq, nkv, p.n_ctx, p.scale, s),
                       "attn_prefill");
    }

    case OperationType::GGML_OP_GET_ROWS: {
      const Tensor *table = node->src[0], *ids = node->src[1];
      if (!contiguous_f32(table) || !ids || !ids->data || ids->dataType != GGML_TYPE_I32 ||
          !node->data || table->dims[0] != node->dims[0] ||
          ids->element_count() != static_cast<size_t>(node->dims[1]))
        return infer::fail(std::errc::invalid_argument);
      ++_stats.launches;
      return check_ikv(ikv_get_rows_f32(static_cast<const float *>(table->data),
                                        static_cast<const int32_t *>(ids->data),
                                        static_cast<float *>(node->data), node->dims[1],
                                        table->dims[0], table->dims[1], _status, s),
                       "get_rows");
    }

    case OperationType::GGML_OP_MUL_MAT: {
      if (!mm_operands_ok(node) || !node->data) return infer::fail(std::errc::invalid_argument);
      const Tensor *w = node->src[0], *x = node->src[1];
      ++_stats.launches;
      if (const auto g = _qkv.find(node); g != _qkv.end()) {
        if (const auto qa = _qkv_attn.find(node); qa != _qkv_attn.end()) {
          auto r = dispatch_qkv_decode(node, qa->second);
          if (r) return r;
          if (r.error() != std::make_error_code(std::errc::not_supported)) return r;
        }
        const Tensor *a = g->second[0], *b = g->second[1], *c = g->second[2];
        const Tensor *xin = x, *nw = nullptr;
        float eps = 0.f;
        if (const auto f = _norm_into_mm.find(node); f != _norm_into_mm.end()) {
          xin = f->second->src[0];
          nw = f->second->src[1];
          std::memcpy(&eps, &f->second->op_params[0], sizeof(eps));
          ++_stats.fused_norm_mm;
        }
        ++_stats.fused_qkv;
        return check_ikv(
            ikv_gemv3_f32(static_cast<const float *>(a->src[0]->data),
                          static_cast<const float *>(b->src[0]->data),
                          static_cast<const float *>(c->src[0]->data),
                          static_cast<const float *>(xin->data), static_cast<float *>(a->data),
                          static_cast<float *>(b->data), static_cast<float *>(c->data),
                          a->dims[0], b->dims[0], c->dims[0], w->dims[0],
                          nw ? static_cast<const float *>(nw->data) : nullptr, eps, s),
            "gemv3");
      }
      float *mm_out = static_cast<float *>(node->data);
      if (const auto oc = _out_into_cpy.find(node); oc != _out_into_cpy.end()) {
        mm_out = static_cast<float *>(oc->second->data);
        ++_stats.fused_append;
      }
      return check_ikv(ikv_mul_mat_f32(static_cast<const float *>(w->data),
                                       static_cast<const float *>(x->data), mm_out, w->dims[1],
                                       w->dims[0], x->dims[1], nullptr, s),
                       "mul_mat");
    }

    case OperationType::GGML_OP_ADD: {
      const Tensor *a = node->src[0], *b = node->src[1];
      if (!node->data) return infer::fail(std::errc::invalid_argument);
      ++_stats.launches;
      if (const auto f = _residual.find(node); f != _residual.end()) {
        const Tensor *mm = f->second.first, *res = f->second.second;
        const Tensor *w = mm->src[0], *x = mm->src[1];
        ++_stats.fused_residual;
        return check_ikv(ikv_mul_mat_f32(static_cast<const float *>(w->data),
                                         static_cast<const float *>(x->data),
                                         static_cast<float *>(node->data), w->dims[1], w->dims[0],
                                         x->dims[1], static_cast<const float *>(res->data), s),
                         "mul_mat+add");
      }
      if (!contiguous_f32(a) || !contiguous_f32(b) || a->dims != node->dims || b->dims != node->dims)
        return infer::fail(std::errc::invalid_argument);
      return check_ikv(ikv_add_f32(static_cast<const float *>(a->data), static_cast<const float *>(b->data),
                                   static_cast<float *>(node->data), int64_t(node->element_count()), s),
                       "add");
    }

    case OperationType::GGML_OP_MUL: {
      const Tensor *a = node->src[0], *b = node->src[1];
      if (!node->data) return infer::fail(std::errc::invalid_argument);
      ++_stats.launches;
      if (const auto f = _swiglu.find(node); f != _swiglu.end()) {
        const Tensor *gate = f->second.first, *up = f->second.second;
        const Tensor *xin = gate->src[1], *nw = nullptr;
        float eps = 0.f;
        if (const auto n = _norm_into_mm.find(node); n != _norm_into_mm.end()) {
          xin = n->second->src[0];
          nw = n->second->src[1];
          std::memcpy(&eps, &n->second->op_params[0], sizeof(eps));
          ++_stats.fused_norm_mm;
        }
        ++_stats.fused_swiglu;
        return check_ikv(ikv_gemv_swiglu_f32(static_cast<const float *>(gate->src[0]->data),
                                             static_cast<const float *>(up->src[0]->data),
                                             static_cast<const float *>(xin->data),
                                             static_cast<float *>(node->data), gate->dims[0],
                                             gate->src[0]->dims[0],
                                             nw ? static_cast<const float *>(nw->data) : nullptr,
                                             eps, s),
                         "gemv_swiglu");
      }
      if (const auto f = _silu_mul.find(node); f != _silu_mul.end()) {
        const Tensor *gate = f->second.first, *up = f->second.second;
        return check_ikv(ikv_silu_mul_f32(static_cast<const float *>(gate->data),
                                          static_cast<const float *>(up->data),
                                          static_cast<float *>(node->data),
                                          int64_t(node->element_count()), s),
                         "silu_mul");
      }
      if (!contiguous_f32(a) || !contiguous_f32(b) || a->dims != node->dims || b->dims != node->dims)
        return infer::fail(std::errc::invalid_argument);
      return check_ikv(ikv_mul_f32(static_cast<const float *>(a->data), static_cast<const float *>(b->data),
                                   static_cast<float *>(node->data), int64_t(node->element_count()), s),
                       "mul");
    }

    case OperationType::GGML_OP_UNARY: {
      const Tensor *x = node->src[0];
      if (!is_silu(node) || !contiguous_f32(x) || !node->data || x->dims != node->dims)
        return infer::fail(std::errc::not_supported);
      ++_stats.launches;
      return check_ikv(ikv_silu_f32(static_cast<const float *>(x->data), static_cast<float *>(node->data),
                                    int64_t(node->element_count()), s),
                       "silu");
    }

    default:
      std::fprintf(stderr, "[hip] unsupported op %u\n", static_cast<unsigned>(node->op));
      return infer::fail(std::errc::not_supported);
  }
}
