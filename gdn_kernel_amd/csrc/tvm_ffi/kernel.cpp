// TVM-FFI export of the decode kernel over the gdn_kernel_amd C ABI: the symbol
// `kernel` with the reference's signature (solution/cuda/kernel.cu:101-113,
// exported at :150), so a FlashInfer-Bench config with binding = "tvm-ffi" and
// entry_point = "kernel.cu::kernel" can bind this library unchanged.  Host code
// only; built by gdn_kernel_amd.build when the tvm-ffi headers are found.
#include <tvm/ffi/container/tensor.h>
#include <tvm/ffi/error.h>
#include <tvm/ffi/extra/c_env_api.h>
#include <tvm/ffi/function.h>

#include "gdn_kernel_amd.h"

namespace {

// q, k [B, 1, Hq|Hk, 128] bf16; v [B, 1, Hv, 128] bf16; state / new_state
// [B, Hv, 128, 128] fp32 (state may be a null tensor: zeros); A_log, dt_bias [Hv]
// fp32; a, b [B, 1, Hv] bf16; output [B, 1, Hv, 128] bf16.  scale 0 => 1/sqrt(128).
void GDNDecodeKernel(tvm::ffi::TensorView q, tvm::ffi::TensorView k, tvm::ffi::TensorView v,
                     tvm::ffi::TensorView state, tvm::ffi::TensorView A_log, tvm::ffi::TensorView a,
                     tvm::ffi::TensorView dt_bias, tvm::ffi::TensorView b, double scale,
                     tvm::ffi::TensorView output, tvm::ffi::TensorView new_state) {
  const DLDevice dev = q.device();
  void* stream = TVMFFIEnvGetStream(dev.device_type, dev.device_id);  // the caller's hipStream_t
  const int nd = static_cast<int>(q.ndim());
  const int rc = gdn_decode(
      static_cast<const gdn_bf16*>(q.data_ptr()), static_cast<const gdn_bf16*>(k.data_ptr()),
      static_cast<const gdn_bf16*>(v.data_ptr()), static_cast<const float*>(state.data_ptr()),
      static_cast<const float*>(A_log.data_ptr()), static_cast<const gdn_bf16*>(a.data_ptr()),
      static_cast<const float*>(dt_bias.data_ptr()), static_cast<const gdn_bf16*>(b.data_ptr()), scale,
      static_cast<gdn_bf16*>(output.data_ptr()), static_cast<float*>(new_state.data_ptr()), q.size(0),
      static_cast<int32_t>(q.size(nd - 2)), static_cast<int32_t>(k.size(nd - 2)),
      static_cast<int32_t>(v.size(nd - 2)), static_cast<int32_t>(q.size(nd - 1)),
      static_cast<int32_t>(v.size(nd - 1)), stream);
  if (rc != GDN_OK) TVM_FFI_THROW(RuntimeError) << gdn_last_error();
}

}  // namespace

TVM_FFI_DLL_EXPORT_TYPED_FUNC(kernel, GDNDecodeKernel);
