// tensor.hpp — the Tensor descriptor every op reads (reference
// include/tensor.hpp:12-91): dims[0] innermost, byte strides, up to four
// sources, 64 bytes of op parameters, role, placement.
#pragma once

#include <array>
#include <initializer_list>
#include <string>
#include <string_view>

#include "util.hpp"

class Backend;

struct Tensor {
  Tensor() = default;
  Tensor(std::string_view name_, DataType type, std::initializer_list<int64_t> shape)
      : name(name_), dataType(type) {
    size_t i = 0;
    for (int64_t e : shape) {
      if (i >= TENSOR_MAX_DIMS) break;
      dims[i++] = e;
    }
    set_contiguous_strides();
  }

  std::string name;
  int layer = 0;
  int64_t offset = 0;
  void *data = nullptr;
  std::array<int64_t, TENSOR_MAX_DIMS> dims{1, 1, 1, 1};
  std::array<int64_t, TENSOR_MAX_DIMS> strides{0, 0, 0, 0};
  std::array<Tensor *, TENSOR_MAX_SRC> src{nullptr, nullptr, nullptr, nullptr};
  int32_t op_params[OP_PARAMS_MAX * sizeof(int32_t)] = {0};
  DataType dataType = GGML_TYPE_F32;
  TensorRole tensorRole = TensorRole::TENSOR_ROLE_NONE;
  OperationType op = OperationType::GGML_OP_NONE;
  DeviceType device = DeviceType::CPU;
  Backend *backend = nullptr;
  bool pinned = false;

  // Byte strides of a contiguous layout (include/tensor.hpp:26-29).
  void set_contiguous_strides() {
    const int64_t es = static_cast<int64_t>(dataType_size(dataType));
    strides[0] = es;
    strides[1] = es * dims[0];
    strides[2] = es * dims[0] * dims[1];
    strides[3] = es * dims[0] * dims[1] * dims[2];
  }
  size_t element_count() const {
    return static_cast<size_t>(dims[0] * dims[1] * dims[2] * dims[3]);
  }
  size_t byte_size() const { return element_count() * dataType_size(dataType); }
  bool is_contiguous() const {
    int64_t s = static_cast<int64_t>(dataType_size(dataType));
    for (int i = 0; i < TENSOR_MAX_DIMS; ++i) {
      if (dims[i] <= 0 || strides[i] != s) return false;
      s *= dims[i];
    }
    return true;
  }
};
