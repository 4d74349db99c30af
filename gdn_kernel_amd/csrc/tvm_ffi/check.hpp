// Argument checks of the TVM-FFI shims (host code): the dtype, rank, extents,
// device and contiguity of every tensor, as the Python binding checks them
// (gdn_kernel_amd/binding.py), before any pointer reaches the C ABI.  The
// reference's exports check nothing (solution/cuda/kernel.cu:101-148,
// kernel_prefill.cu:300-337).  A failed check throws a TVM-FFI ValueError.
#pragma once

#include <tvm/ffi/container/tensor.h>
#include <tvm/ffi/error.h>

#include <cstdint>
#include <vector>

namespace gdn_tvm_ffi {

enum class DType { kBF16, kF32, kIndex /* int32 or int64 */ };

inline const char* dtype_name(DType d) {
  return d == DType::kBF16 ? "bfloat16" : d == DType::kF32 ? "float32" : "int32 or int64";
}

inline bool dtype_ok(DLDataType t, DType want) {
  if (t.lanes != 1) return false;
  switch (want) {
    case DType::kBF16: return t.code == kDLBfloat && t.bits == 16;
    case DType::kF32: return t.code == kDLFloat && t.bits == 32;
    default: return t.code == kDLInt && (t.bits == 32 || t.bits == 64);
  }
}

// `shape` lists the expected extents; -1 accepts any extent.
inline void check_tensor(const tvm::ffi::TensorView& t, const char* name, DType want,
                         const std::vector<int64_t>& shape, DLDevice device) {
  if (!dtype_ok(t.dtype(), want)) TVM_FFI_THROW(ValueError) << name << " must be " << dtype_name(want);
  if (t.ndim() != static_cast<int>(shape.size()))
    TVM_FFI_THROW(ValueError) << name << " must have " << shape.size() << " dims (got " << t.ndim() << ")";
  int i = 0;
  for (const int64_t want_size : shape) {
    if (want_size >= 0 && t.size(i) != want_size)
      TVM_FFI_THROW(ValueError) << name << " dim " << i << " must be " << want_size << " (got " << t.size(i) << ")";
    ++i;
  }
  const DLDevice d = t.device();
  if (d.device_type != device.device_type || d.device_id != device.device_id)
    TVM_FFI_THROW(ValueError) << name << " is on another device than q";
  int64_t expect = 1;  // row-major (C-contiguous) strides, in elements
  for (int j = t.ndim() - 1; j >= 0; --j) {
    if (t.size(j) != 1 && t.stride(j) != expect) TVM_FFI_THROW(ValueError) << name << " must be contiguous";
    expect *= t.size(j);
  }
}

}  // namespace gdn_tvm_ffi
