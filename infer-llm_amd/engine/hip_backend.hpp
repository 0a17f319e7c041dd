// hip_backend.hpp — the MI355X backend behind the engine's Backend interface
// (the slot of CUDABackend, reference include/backends/cuda_backend.hpp:15-97,
// src/backends/cuda_backend.cpp:6-241).
//
// * Registered as "hip"; devices are probed with hipGetDeviceCount /
//   hipMemGetInfo and named "hip:<id>".
// * WEIGHTS / ACTIVATION / KVCACHE pools allocate with hipMalloc, so the KV
//   cache of NaiveKVStorage lives in HBM.
// * One stream per backend (default priority); every entry point selects the
//   device first.
// * compute() walks the subgraph in topological order and calls the C-ABI
//   of include/ikv.h. Two fusions are applied when the graph has the shape
//   the Qwen3 attention slice builds: RMS_NORM -> ROPE becomes one
//   qk-norm+RoPE launch, and CPY (K), CPY (V) -> VIEW -> FLASH_ATTN_EXT for
//   one query token becomes one decode launch with the append inside.
// * RoPE reads device-resident sin/cos tables built once, with the host's
//   sinf/cosf, from the angle table the graph supplies (host memory); the
//   reference copied that 10.5 MB table to the device every step.
#pragma once

#include <hip/hip_runtime.h>

#include <array>
#include <string>
#include <unordered_map>
#include <vector>

#include "backend.hpp"
#include "graph.hpp"

std::vector<DeviceInfo> probe_hip_devices();

class HIPBackend : public Backend {
 public:
  HIPBackend(int device_id, DeviceInfo info, const PoolConfig &cfg);
  ~HIPBackend() override;

  DeviceType device_type() const override { return DeviceType::HIP; }
  std::string device_name() const override { return "HIP:" + std::to_string(_device_id); }
  bool supports_op(OperationType op, const Tensor &t) const override;
  infer::expected<void *, std::error_code> alloc(BufferKind kind, size_t bytes) override;
  void free(BufferKind kind, void *ptr) override;
  bool is_host() const override { return false; }
  infer::expected<void, std::error_code> copy_tensor_set(Tensor *tensor, const void *data,
                                                         size_t offset, size_t size) override;
  infer::expected<void, std::error_code> copy_tensor_get(const Tensor *tensor, void *data,
                                                         size_t offset, size_t size) override;
  infer::expected<bool, std::error_code> copy_tensor_high(const Tensor *src,
                                                          Tensor *dst) const override;
  infer::expected<void, std::error_code> compute(Graph &sub_graph) override;
  // Waits for the stream, then reports the data errors the kernels recorded
  // since the last call (IKV_STATUS_* bits: RoPE positions, paged block
  // entries, token ids), each by name, as invalid_argument.
  infer::expected<void, std::error_code> synchronize() override;
  bool accepts_host_src(const Tensor &node, int src_index) const override;

  hipStream_t stream() const { return _stream; }
  // Sizes the decode workspace for contexts up to max_kv keys, so that no
  // allocation happens inside compute() (e.g. under graph capture).
  infer::expected<void, std::error_code> reserve_decode_workspace(int n_head, int n_head_kv,
                                                                  int head_dim, int64_t max_kv);
  // The bytes reserve_decode_workspace allocates: the largest decode
  // workspace of any context of 1..max_kv keys (host arithmetic only).
  static size_t decode_workspace_reservation(int n_head, int n_head_kv, int head_dim,
                                             int64_t max_kv);
  void set_fusion(bool on) { _fusion = on; }
  bool fusion() const { return _fusion; }
  // n_kv_max > 0: one-token decodes launch in their replay form (the context
  // read from the position on the device, planned for n_kv_max keys), so
  // that the step can be captured once and replayed at later positions; 0
  // restores the per-context launches. Decodes with the qk-norm / RoPE
  // fusion only, contiguous or paged (other decodes then fail with
  // not_supported).
  void set_decode_replay(int64_t n_kv_max) { _replay_max = n_kv_max; }
  struct Stats {
    int launches = 0;
    int fused_norm_rope = 0;
    int fused_append_decode = 0;
    int fused_swiglu = 0;
    int fused_residual = 0;
    int fused_qkv = 0;
    int fused_norm_mm = 0;      // RMSNorm folded into q/k/v or SwiGLU
    int fused_rope_decode = 0;  // qk-norm + RoPE folded into the decode launch
    int fused_qkv_decode = 0;   // short-context decode folded into the q/k/v launch
    int fused_append = 0;       // cache appends written by their producer (prefill K and V)
  };
  const Stats &last_stats() const { return _stats; }

 private:
  struct RopeTables {
    float *sin = nullptr;
    float *cos = nullptr;
    int64_t n_ctx = 0;
    int64_t half = 0;
  };
  infer::expected<const RopeTables *, std::error_code> rope_tables(const Tensor &theta);
  infer::expected<void, std::error_code> ensure_workspace(size_t bytes);
  infer::expected<void, std::error_code> dispatch(Tensor *node);
  // The arguments of a one-token decode with qk-norm + RoPE folded in.
  struct DecodeRopeArgs {
    const float *q_raw, *k_raw, *v_new, *q_norm_w, *k_norm_w;
    float eps;
    const int32_t *pos;
    const RopeTables *tab;
  };
  infer::expected<DecodeRopeArgs, std::error_code> decode_rope_args(const Tensor *attn);
  // The q/k/v group `first` with its layer's decode folded in, when the
  // context allows (else not_supported and nothing was launched).
  infer::expected<void, std::error_code> dispatch_qkv_decode(const Tensor *first, const Tensor *attn);
  void plan_model_fusions(Graph &graph, std::unordered_map<const Tensor *, int> &uses);
  infer::expected<void, std::error_code> set_device() const;

  hipStream_t _stream = nullptr;
  int *_status = nullptr;  // device flag raised by RoPE on a bad position
  void *_workspace = nullptr;
  size_t _workspace_bytes = 0;
  std::vector<RopeTables> _tables;                            // device sin/cos tables
  std::unordered_map<const void *, size_t> _rope;             // angle-table address -> table
  std::unordered_map<std::string, size_t> _rope_by_content;   // dims + row 1 -> table
  bool _fusion = true;
  int64_t _replay_max = 0;
  Stats _stats;
  // per-compute() fusion plan
  std::unordered_map<const Tensor *, const Tensor *> _norm_into_rope;  // rope -> its rms_norm
  std::unordered_map<const Tensor *, std::pair<const Tensor *, const Tensor *>> _append_into_attn;
  std::unordered_map<const Tensor *, std::pair<const Tensor *, const Tensor *>> _swiglu;    // mul -> gate, up
  std::unordered_map<const Tensor *, std::pair<const Tensor *, const Tensor *>> _silu_mul;  // mul -> gate, up (SILU input, other factor)
  std::unordered_map<const Tensor *, std::pair<const Tensor *, const Tensor *>> _residual;  // add -> mm, r
  std::unordered_map<const Tensor *, std::array<const Tensor *, 3>> _qkv;  // first mm -> group
  std::unordered_map<const Tensor *, const Tensor *> _norm_into_mm;  // qkv first mm / swiglu mul -> norm
  std::unordered_map<const Tensor *, std::pair<const Tensor *, const Tensor *>> _rope_into_attn;  // attn -> q, k rope
  std::unordered_map<const Tensor *, const Tensor *> _qkv_attn;  // qkv first mm -> the decode it feeds
  std::unordered_map<const Tensor *, bool> _attn_done;           // decodes run by a q/k/v launch
  std::unordered_map<const Tensor *, const Tensor *> _out_into_cpy;  // rope / mul_mat -> the cache copy it writes
  std::unordered_map<const Tensor *, bool> _skip;
};

// Host memory as a backend: pinned (hipHostMalloc) pools, memcpy copies, no
// compute. The host tier of OffloadKVStorage, so that its page-in and
// write-back copies are DMA transfers from page-locked memory.
class PinnedHostBackend final : public Backend {
 public:
  explicit PinnedHostBackend(int device_id = 0);
  DeviceType device_type() const override { return DeviceType::CPU; }
  std::string device_name() const override { return "PINNED_HOST"; }
  bool supports_op(OperationType, const Tensor &) const override { return false; }
  bool is_host() const override { return true; }
  infer::expected<void, std::error_code> copy_tensor_set(Tensor *t, const void *d, size_t off,
                                                         size_t n) override;
  infer::expected<void, std::error_code> copy_tensor_get(const Tensor *t, void *d, size_t off,
                                                         size_t n) override;
  infer::expected<bool, std::error_code> copy_tensor_high(const Tensor *, Tensor *) const override {
    return false;
  }
  infer::expected<void, std::error_code> compute(Graph &) override {
    return infer::fail(std::errc::not_supported);
  }
};

