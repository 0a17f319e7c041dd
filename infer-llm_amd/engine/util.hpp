// util.hpp — the enums and helpers of the engine's data contract, restated
// from the reference (include/util.hpp:27-310) for the ops this build uses.
//
// Numeric values are the reference's (ggml numbering), so a Tensor built by
// the reference's OpFactory and one built here carry the same op ids:
//   DataType       include/util.hpp:27-72
//   TensorRole     include/util.hpp:74-82
//   OperationType  include/util.hpp:85-198 (only the values used are named)
//   DeviceType     include/util.hpp:227-233, plus HIP for this backend
#pragma once

#include <cstddef>
#include <cstdint>

#define TENSOR_MAX_DIMS 4
#define TENSOR_MAX_SRC 4
#define OP_PARAMS_MAX 4

enum DataType : int32_t {
  GGML_TYPE_F32 = 0,
  GGML_TYPE_F16 = 1,
  GGML_TYPE_I8 = 24,
  GGML_TYPE_I16 = 25,
  GGML_TYPE_I32 = 26,
  GGML_TYPE_I64 = 27,
  GGML_TYPE_F64 = 28,
  GGML_TYPE_BF16 = 30,
};

enum class TensorRole : uint8_t {
  TENSOR_ROLE_NONE = 0,
  TNESOR_ROLE_INPUT = 1 << 0,  // the reference's spelling
  TENSOR_ROLE_OUTPUT = 1 << 1,
  TENSOR_ROLE_WEIGHT = 1 << 2,
  TENSOR_ROLE_ACTIVATION = 1 << 3,
  TENSOR_ROLE_VIEW = 1 << 4,
  TENSOR_ROLE_KVCACHE = 1 << 5,
};

enum class OperationType : uint32_t {
  GGML_OP_NONE = 0,
  GGML_OP_ADD = 2,
  GGML_OP_MUL = 7,
  GGML_OP_RMS_NORM = 25,
  GGML_OP_MUL_MAT = 29,
  GGML_OP_CPY = 34,
  GGML_OP_RESHAPE = 36,
  GGML_OP_VIEW = 37,
  GGML_OP_GET_ROWS = 40,
  GGML_OP_ROPE = 48,
  GGML_OP_FLASH_ATTN_EXT = 74,
  GGML_OP_UNARY = 91,
  GGML_OP_COUNT = 101,
};

// Sub-op ids of GGML_OP_UNARY (include/util.hpp:198-215).
enum class UnaryOp : uint32_t {
  GGML_UNARY_OP_ABS = 0,
  GGML_UNARY_OP_SGN,
  GGML_UNARY_OP_NEG,
  GGML_UNARY_OP_STEP,
  GGML_UNARY_OP_TANH,
  GGML_UNARY_OP_ELU,
  GGML_UNARY_OP_RELU,
  GGML_UNARY_OP_SIGMOID,
  GGML_UNARY_OP_GELU,
  GGML_UNARY_OP_GELU_QUICK,
  GGML_UNARY_OP_SILU,
};

enum class DeviceType : uint8_t {
  CPU = 0,
  CUDA = 1,
  SYCL = 2,
  VULKAN = 3,
  METAL = 4,
  HIP = 5,
};

size_t dataType_size(DataType t);
const char *device_type_name(DeviceType t);
