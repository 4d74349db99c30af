// TVM-FFI export of the varlen chunked prefill over the gdn_kernel_amd C ABI: the
// symbol `kernel` with the reference's signature (solution/cuda/
// kernel_prefill.cu:300-306, exported at :339).  Host code only; built by
// gdn_kernel_amd.build when the tvm-ffi headers are found.
#include <tvm/ffi/container/tensor.h>
#include <tvm/ffi/error.h>
#include <tvm/ffi/extra/c_env_api.h>
#include <tvm/ffi/function.h>

#include "gdn_kernel_amd.h"

namespace {

// q, k [T, Hq|Hk, 128] bf16 and v [T, Hv, 128] bf16 (packed tokens; a leading
// dim of 1 is accepted); state / new_state [N, Hv, 128, 128] fp32 (state may be a
// null tensor: zeros); A_log, dt_bias [Hv] fp32; a, b [T, Hv] bf16; cu_seqlens
// [N + 1] int64 (as the reference) or int32; output [T, Hv, 128] bf16.
void GDNPrefillKernel(tvm::ffi::TensorView q, tvm::ffi::TensorView k, tvm::ffi::TensorView v,
                      tvm::ffi::TensorView state, tvm::ffi::TensorView A_log, tvm::ffi::TensorView a,
                      tvm::ffi::TensorView dt_bias, tvm::ffi::TensorView b, tvm::ffi::TensorView cu_seqlens,
                      double scale, tvm::ffi::TensorView output, tvm::ffi::TensorView new_state) {
  const DLDevice dev = q.device();
  void* stream = TVMFFIEnvGetStream(dev.device_type, dev.device_id);  // the caller's hipStream_t
  const int nd = static_cast<int>(q.ndim());
  const int64_t total_tokens = q.size(nd - 3);
  const int64_t num_seqs = cu_seqlens.size(0) - 1;
  const int32_t cu_dtype = cu_seqlens.dtype().bits == 64 ? GDN_INDEX_INT64 : GDN_INDEX_INT32;
  const int rc = gdn_prefill(
      static_cast<const gdn_bf16*>(q.data_ptr()), static_cast<const gdn_bf16*>(k.data_ptr()),
      static_cast<const gdn_bf16*>(v.data_ptr()), static_cast<const float*>(state.data_ptr()),
      static_cast<const float*>(A_log.data_ptr()), static_cast<const gdn_bf16*>(a.data_ptr()),
      static_cast<const float*>(dt_bias.data_ptr()), static_cast<const gdn_bf16*>(b.data_ptr()),
      cu_seqlens.data_ptr(), cu_dtype, num_seqs, total_tokens, scale, static_cast<gdn_bf16*>(output.data_ptr()),
      static_cast<float*>(new_state.data_ptr()), static_cast<int32_t>(q.size(nd - 2)),
      static_cast<int32_t>(k.size(nd - 2)), static_cast<int32_t>(v.size(nd - 2)),
      static_cast<int32_t>(q.size(nd - 1)), static_cast<int32_t>(v.size(nd - 1)), stream);
  if (rc != GDN_OK) TVM_FFI_THROW(RuntimeError) << gdn_last_error();
}

}  // namespace

TVM_FFI_DLL_EXPORT_TYPED_FUNC(kernel, GDNPrefillKernel);
