#include "util.hpp"

// Element sizes of the element-wise types (reference src/util.cpp:78-121).
size_t dataType_size(DataType t) {
  switch (t) {
    case GGML_TYPE_F32: return 4;
    case GGML_TYPE_F16: return 2;
    case GGML_TYPE_I8: return 1;
    case GGML_TYPE_I16: return 2;
    case GGML_TYPE_I32: return 4;
    case GGML_TYPE_I64: return 8;
    case GGML_TYPE_F64: return 8;
    case GGML_TYPE_BF16: return 2;
  }
  return 0;
}

const char *device_type_name(DeviceType t) {
  switch (t) {
    case DeviceType::CPU: return "CPU";
    case DeviceType::CUDA: return "CUDA";
    case DeviceType::SYCL: return "SYCL";
    case DeviceType::VULKAN: return "VULKAN";
    case DeviceType::METAL: return "METAL";
    case DeviceType::HIP: return "HIP";
  }
  return "UNKNOWN";
}
