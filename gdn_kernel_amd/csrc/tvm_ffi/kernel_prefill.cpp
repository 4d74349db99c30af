// TVM-FFI export of the varlen chunked prefill over the gdn_kernel_amd C ABI: the
// symbol `kernel` with the reference's signature (solution/cuda/
// kernel_prefill.cu:300-306, exported at :339).  Host code only; built by
// gdn_kernel_amd.build when the tvm-ffi headers are found.
#include <tvm/ffi/container/tensor.h>
#include <tvm/ffi/error.h>
#include <tvm/ffi/extra/c_env_api.h>
#include <tvm/ffi/function.h>

#include "check.hpp"
#include "gdn_kernel_amd.h"

namespace {

// q, k [T, Hq|Hk, 128] bf16 and v [T, Hv, 128] bf16 (packed tokens; a leading
// dim of 1 is accepted on q, k, v, a, b and output); state / new_state
// [N, Hv, 128, 128] fp32 (state may be a null tensor: zeros); A_log, dt_bias [Hv]
// fp32; a, b [T, Hv] bf16; cu_seqlens [N + 1] int64 (as the reference) or int32;
// output [T, Hv, 128] bf16.  Every tensor is checked (dtype, rank, extents,
// device, contiguity) first.
void GDNPrefillKernel(tvm::ffi::TensorView q, tvm::ffi::TensorView k, tvm::ffi::TensorView v,
                      tvm::ffi::TensorView state, tvm::ffi::TensorView A_log, tvm::ffi::TensorView a,
                      tvm::ffi::TensorView dt_bias, tvm::ffi::TensorView b, tvm::ffi::TensorView cu_seqlens,
                      double scale, tvm::ffi::TensorView output, tvm::ffi::TensorView new_state) {
  using gdn_tvm_ffi::check_tensor;
  using gdn_tvm_ffi::DType;
  const DLDevice dev = q.device();
  const int nd = static_cast<int>(q.ndim());
  if (nd != 3 && !(nd == 4 && q.size(0) == 1))
    TVM_FFI_THROW(ValueError) << "q must be [T, Hq, d] (optionally with a leading 1)";
  if (k.ndim() != nd || v.ndim() != nd) TVM_FFI_THROW(ValueError) << "q, k, v must have the same rank";
  // Shapes with the optional leading 1 of the token-major tensors.
  auto lead = [nd](std::vector<int64_t> s) {
    if (nd == 4) s.insert(s.begin(), 1);
    return s;
  };
  const int64_t T = q.size(nd - 3), Hq = q.size(nd - 2), Hk = k.size(nd - 2), Hv = v.size(nd - 2);
  const int64_t dk = q.size(nd - 1), dv = v.size(nd - 1);
  if (cu_seqlens.ndim() != 1 || cu_seqlens.size(0) < 1) TVM_FFI_THROW(ValueError) << "cu_seqlens must be [N + 1]";
  const int64_t N = cu_seqlens.size(0) - 1;
  check_tensor(q, "q", DType::kBF16, lead({T, Hq, dk}), dev);
  check_tensor(k, "k", DType::kBF16, lead({T, Hk, dk}), dev);
  check_tensor(v, "v", DType::kBF16, lead({T, Hv, dv}), dev);
  if (state.data_ptr() != nullptr) check_tensor(state, "state", DType::kF32, {N, Hv, dv, dk}, dev);
  check_tensor(A_log, "A_log", DType::kF32, {Hv}, dev);
  check_tensor(a, "a", DType::kBF16, lead({T, Hv}), dev);
  check_tensor(dt_bias, "dt_bias", DType::kF32, {Hv}, dev);
  check_tensor(b, "b", DType::kBF16, lead({T, Hv}), dev);
  check_tensor(cu_seqlens, "cu_seqlens", DType::kIndex, {N + 1}, dev);
  check_tensor(output, "output", DType::kBF16, lead({T, Hv, dv}), dev);
  check_tensor(new_state, "new_state", DType::kF32, {N, Hv, dv, dk}, dev);
  void* stream = TVMFFIEnvGetStream(dev.device_type, dev.device_id);  // the caller's hipStream_t
  const int32_t cu_dtype = cu_seqlens.dtype().bits == 64 ? GDN_INDEX_INT64 : GDN_INDEX_INT32;
  const int rc = gdn_prefill(
      static_cast<const gdn_bf16*>(q.data_ptr()), static_cast<const gdn_bf16*>(k.data_ptr()),
      static_cast<const gdn_bf16*>(v.data_ptr()), static_cast<const float*>(state.data_ptr()),
      static_cast<const float*>(A_log.data_ptr()), static_cast<const gdn_bf16*>(a.data_ptr()),
      static_cast<const float*>(dt_bias.data_ptr()), static_cast<const gdn_bf16*>(b.data_ptr()),
      cu_seqlens.data_ptr(), cu_dtype, N, T, scale, static_cast<gdn_bf16*>(output.data_ptr()),
      static_cast<float*>(new_state.data_ptr()), static_cast<int32_t>(Hq), static_cast<int32_t>(Hk),
      static_cast<int32_t>(Hv), static_cast<int32_t>(dk), static_cast<int32_t>(dv), stream);
  if (rc != GDN_OK) TVM_FFI_THROW(RuntimeError) << gdn_last_error();
}

}  // namespace

TVM_FFI_DLL_EXPORT_TYPED_FUNC(kernel, GDNPrefillKernel);
