// op_params.hpp — parameters of the attention op, stored byte-for-byte in
// Tensor::op_params (reference include/op_params.hpp:5-21; 36 bytes).
#pragma once

#include <cstdint>

struct AttnParams {
  uint32_t n_head = 0;          // query heads
  uint32_t n_head_kv = 0;       // KV heads (GQA)
  uint32_t head_dim = 0;        // 128 for Qwen3
  float scale = 0.0f;           // softmax scale; <= 0 means 1/sqrt(head_dim)
  bool causal = true;           // key j visible to query t iff j <= n_ctx + t
  uint32_t n_ctx = 0;           // tokens already in the cache (n_past)
  uint32_t sliding_window = 0;  // 0 = disabled (ignored, as in the reference)
  uint32_t _pad[2] = {0, 0};
};

static_assert(sizeof(AttnParams) == 36, "AttnParams must keep the reference layout");
