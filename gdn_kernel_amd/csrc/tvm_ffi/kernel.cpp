// TVM-FFI export of the decode kernel over the gdn_kernel_amd C ABI: the symbol
// `kernel` with the reference's signature (solution/cuda/kernel.cu:101-113,
// exported at :150), so a FlashInfer-Bench config with binding = "tvm-ffi" and
// entry_point = "kernel.cu::kernel" can bind this library unchanged.  Host code
// only; built by gdn_kernel_amd.build when the tvm-ffi headers are found.
#include <tvm/ffi/container/tensor.h>
#include <tvm/ffi/error.h>
#include <tvm/ffi/extra/c_env_api.h>
#include <tvm/ffi/function.h>

#include "check.hpp"
#include "gdn_kernel_amd.h"

namespace {

// q, k [B, 1, Hq|Hk, 128] bf16; v [B, 1, Hv, 128] bf16; state / new_state
// [B, Hv, 128, 128] fp32 (state may be a null tensor: zeros); A_log, dt_bias [Hv]
// fp32; a, b [B, 1, Hv] bf16; output [B, 1, Hv, 128] bf16.  scale 0 => 1/sqrt(128).
// Every tensor is checked (dtype, rank, extents, device, contiguity) first.
void GDNDecodeKernel(tvm::ffi::TensorView q, tvm::ffi::TensorView k, tvm::ffi::TensorView v,
                     tvm::ffi::TensorView state, tvm::ffi::TensorView A_log, tvm::ffi::TensorView a,
                     tvm::ffi::TensorView dt_bias, tvm::ffi::TensorView b, double scale,
                     tvm::ffi::TensorView output, tvm::ffi::TensorView new_state) {
  using gdn_tvm_ffi::check_tensor;
  using gdn_tvm_ffi::DType;
  const DLDevice dev = q.device();
  if (q.ndim() != 4 || k.ndim() != 4 || v.ndim() != 4)
    TVM_FFI_THROW(ValueError) << "q, k, v must be 4-D [B, 1, H, d]";
  const int64_t B = q.size(0), Hq = q.size(2), Hk = k.size(2), Hv = v.size(2), dk = q.size(3), dv = v.size(3);
  check_tensor(q, "q", DType::kBF16, {B, 1, Hq, dk}, dev);
  check_tensor(k, "k", DType::kBF16, {B, 1, Hk, dk}, dev);
  check_tensor(v, "v", DType::kBF16, {B, 1, Hv, dv}, dev);
  if (state.data_ptr() != nullptr) check_tensor(state, "state", DType::kF32, {B, Hv, dv, dk}, dev);
  check_tensor(A_log, "A_log", DType::kF32, {Hv}, dev);
  check_tensor(a, "a", DType::kBF16, {B, 1, Hv}, dev);
  check_tensor(dt_bias, "dt_bias", DType::kF32, {Hv}, dev);
  check_tensor(b, "b", DType::kBF16, {B, 1, Hv}, dev);
  check_tensor(output, "output", DType::kBF16, {B, 1, Hv, dv}, dev);
  check_tensor(new_state, "new_state", DType::kF32, {B, Hv, dv, dk}, dev);
  void* stream = TVMFFIEnvGetStream(dev.device_type, dev.device_id);  // the caller's hipStream_t
  const int rc = gdn_decode(
      static_cast<const gdn_bf16*>(q.data_ptr()), static_cast<const gdn_bf16*>(k.data_ptr()),
      static_cast<const gdn_bf16*>(v.data_ptr()), static_cast<const float*>(state.data_ptr()),
      static_cast<const float*>(A_log.data_ptr()), static_cast<const gdn_bf16*>(a.data_ptr()),
      static_cast<const float*>(dt_bias.data_ptr()), static_cast<const gdn_bf16*>(b.data_ptr()), scale,
      static_cast<gdn_bf16*>(output.data_ptr()), static_cast<float*>(new_state.data_ptr()), B,
      static_cast<int32_t>(Hq), static_cast<int32_t>(Hk), static_cast<int32_t>(Hv), static_cast<int32_t>(dk),
      static_cast<int32_t>(dv), stream);
  if (rc != GDN_OK) TVM_FFI_THROW(RuntimeError) << gdn_last_error();
}

}  // namespace

TVM_FFI_DLL_EXPORT_TYPED_FUNC(kernel, GDNDecodeKernel);
