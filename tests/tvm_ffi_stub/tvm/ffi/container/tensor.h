// Test stand-in, not tvm-ffi: the DLPack types (values as the DLPack standard
// defines them) and the members of tvm::ffi::TensorView that the shims under
// gdn_kernel_amd/csrc/tvm_ffi use, so that tests/test_tvm_ffi_shim.py can compile
// and run the shims' argument checks on the CPU where tvm-ffi is not installed.
#pragma once

#include <cstdint>
#include <utility>
#include <vector>

typedef enum { kDLInt = 0U, kDLUInt = 1U, kDLFloat = 2U, kDLBfloat = 4U } DLDataTypeCode;
typedef enum { kDLCPU = 1, kDLCUDA = 2, kDLROCM = 10 } DLDeviceType;
typedef struct {
  uint8_t code;
  uint8_t bits;
  uint16_t lanes;
} DLDataType;
typedef struct {
  DLDeviceType device_type;
  int32_t device_id;
} DLDevice;

namespace tvm {
namespace ffi {

// A view of a strided tensor; strides in elements (empty: row-major).
class TensorView {
 public:
  TensorView(void* data, DLDataType dtype, DLDevice device, std::vector<int64_t> shape,
             std::vector<int64_t> strides = {})
      : data_(data), dtype_(dtype), device_(device), shape_(std::move(shape)), strides_(std::move(strides)) {
    if (strides_.empty()) {
      strides_.assign(shape_.size(), 1);
      for (int i = static_cast<int>(shape_.size()) - 2; i >= 0; --i) strides_[i] = strides_[i + 1] * shape_[i + 1];
    }
  }
  void* data_ptr() const { return data_; }
  DLDataType dtype() const { return dtype_; }
  DLDevice device() const { return device_; }
  int32_t ndim() const { return static_cast<int32_t>(shape_.size()); }
  int64_t size(int64_t i) const { return shape_[static_cast<size_t>(i)]; }
  int64_t stride(int64_t i) const { return strides_[static_cast<size_t>(i)]; }

 private:
  void* data_;
  DLDataType dtype_;
  DLDevice device_;
  std::vector<int64_t> shape_, strides_;
};

}  // namespace ffi
}  // namespace tvm
