// Runs one TVM-FFI shim (GDN_SHIM_DECODE: kernel.cpp, else kernel_prefill.cpp)
// against the stand-in tvm-ffi types of this directory, on host tensors, and prints
// one line per case: "<case>: ok" or "<case>: <ErrorKind>: <message>".  Every case
// either fails a check of the shim, fails the C ABI's argument validation (no device
// call), or is an empty batch (the C ABI returns before any device call), so no
// kernel is ever launched on these host pointers.
#include <cstdio>
#include <functional>

#ifdef GDN_SHIM_DECODE
#include "kernel.cpp"
#else
#include "kernel_prefill.cpp"
#endif

extern "C" void* TVMFFIEnvGetStream(int32_t, int32_t) { return nullptr; }

namespace {

using tvm::ffi::TensorView;
const DLDataType kBF = {kDLBfloat, 16, 1}, kF32 = {kDLFloat, 32, 1}, kI32 = {kDLInt, 32, 1},
                 kI64 = {kDLInt, 64, 1}, kI16 = {kDLInt, 16, 1};
const DLDevice kDev = {kDLROCM, 0}, kOther = {kDLROCM, 1};
alignas(16) char g_buf[64];  // a non-null host address; never dereferenced by any case
void* const P = g_buf;

TensorView T(DLDataType dt, std::vector<int64_t> shape, DLDevice dev = kDev, void* data = P,
             std::vector<int64_t> strides = {}) {
  return TensorView(data, dt, dev, std::move(shape), std::move(strides));
}

void run(const char* name, const std::function<void()>& f) {
  try {
    f();
    std::printf("%s: ok\n", name);
  } catch (const tvm_ffi_stub::Error& e) {
    std::printf("%s: %s: %s\n", name, e.kind.c_str(), e.what());
  }
}

}  // namespace

int main() {
#ifdef GDN_SHIM_DECODE
  // B, Hq, Hk, Hv, d -> the eleven decode arguments with one of them replaced.
  struct Args {
    int64_t B = 0, Hq = 16, Hk = 16, Hv = 32, d = 128;
  };
  auto call = [](Args s, int which = -1, TensorView* alt = nullptr) {
    TensorView t[10] = {T(kBF, {s.B, 1, s.Hq, s.d}),    T(kBF, {s.B, 1, s.Hk, s.d}),
                        T(kBF, {s.B, 1, s.Hv, s.d}),    T(kF32, {s.B, s.Hv, s.d, s.d}),
                        T(kF32, {s.Hv}),                T(kBF, {s.B, 1, s.Hv}),
                        T(kF32, {s.Hv}),                T(kBF, {s.B, 1, s.Hv}),
                        T(kBF, {s.B, 1, s.Hv, s.d}),    T(kF32, {s.B, s.Hv, s.d, s.d})};
    if (which >= 0) t[which] = *alt;
    GDNDecodeKernel(t[0], t[1], t[2], t[3], t[4], t[5], t[6], t[7], 0.0, t[8], t[9]);
  };
  Args ok;
  Args two;
  two.B = 2;
  run("valid_empty_batch", [&] { call(ok); });
  run("null_state", [&] { TensorView s = T(kF32, {0}, kDev, nullptr); call(ok, 3, &s); });
  run("q_dtype", [&] { TensorView x = T(kF32, {0, 1, 16, 128}); call(ok, 0, &x); });
  run("k_rank", [&] { TensorView x = T(kBF, {0, 16, 128}); call(ok, 1, &x); });
  run("output_extent", [&] { TensorView x = T(kBF, {0, 1, 32, 64}); call(ok, 8, &x); });
  run("state_device", [&] { TensorView x = T(kF32, {2, 32, 128, 128}, kOther); call(two, 3, &x); });
  run("state_strided", [&] {
    TensorView x = T(kF32, {2, 32, 128, 128}, kDev, P, {32 * 128 * 256, 128 * 256, 256, 1});
    call(two, 3, &x);
  });
  run("a_dtype", [&] { TensorView x = T(kF32, {0, 1, 32}); call(ok, 5, &x); });
  run("new_state_shape", [&] { TensorView x = T(kF32, {0, 32, 128, 64}); call(ok, 9, &x); });
  Args ratio = two;
  ratio.Hq = ratio.Hk = 3;
  ratio.Hv = 4;
  run("c_abi_head_ratio", [&] { call(ratio); });
  Args small = two;
  small.d = 64;
  run("c_abi_head_dim", [&] { call(small); });
#else
  // T, N, Hq, Hk, Hv, d, lead (a leading 1 on the token-major tensors)
  struct Args {
    int64_t T = 0, N = 0, Hq = 16, Hk = 16, Hv = 32, d = 128;
    bool lead = false;
    DLDataType cu = kI32;
  };
  auto call = [](Args s, int which = -1, TensorView* alt = nullptr) {
    auto L = [&](std::vector<int64_t> v) {
      if (s.lead) v.insert(v.begin(), 1);
      return v;
    };
    TensorView t[11] = {T(kBF, L({s.T, s.Hq, s.d})),        T(kBF, L({s.T, s.Hk, s.d})),
                        T(kBF, L({s.T, s.Hv, s.d})),        T(kF32, {s.N, s.Hv, s.d, s.d}),
                        T(kF32, {s.Hv}),                    T(kBF, L({s.T, s.Hv})),
                        T(kF32, {s.Hv}),                    T(kBF, L({s.T, s.Hv})),
                        T(s.cu, {s.N + 1}),                 T(kBF, L({s.T, s.Hv, s.d})),
                        T(kF32, {s.N, s.Hv, s.d, s.d})};
    if (which >= 0) t[which] = *alt;
    GDNPrefillKernel(t[0], t[1], t[2], t[3], t[4], t[5], t[6], t[7], t[8], 0.0, t[9], t[10]);
  };
  Args ok;
  ok.T = 5;  // no sequence: the C ABI returns before any device call
  run("valid_no_sequences", [&] { call(ok); });
  Args lead = ok;
  lead.lead = true;
  run("valid_leading_one", [&] { call(lead); });
  Args i64 = ok;
  i64.cu = kI64;
  run("valid_int64_offsets", [&] { call(i64); });
  run("cu_dtype", [&] { TensorView x = T(kI16, {1}); call(ok, 8, &x); });
  run("cu_rank", [&] { TensorView x = T(kI32, {1, 1}); call(ok, 8, &x); });
  run("rank_mismatch", [&] { TensorView x = T(kBF, {1, 5, 16, 128}); call(ok, 1, &x); });
  run("state_shape", [&] { TensorView x = T(kF32, {1, 32, 128, 128}); call(ok, 3, &x); });
  run("output_device", [&] { TensorView x = T(kBF, {5, 32, 128}, kOther); call(ok, 9, &x); });
  run("b_strided", [&] { TensorView x = T(kBF, {5, 32}, kDev, P, {64, 1}); call(ok, 7, &x); });
  Args ratio;
  ratio.T = 5;
  ratio.N = 1;
  ratio.Hq = ratio.Hk = 3;
  ratio.Hv = 4;
  run("c_abi_head_ratio", [&] { call(ratio); });
#endif
  return 0;
}
