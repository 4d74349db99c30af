// Test stand-in, not tvm-ffi: the export macro keeps a pointer to the function, so
// a shim compiles; the test driver includes the shim and calls the function itself.
#pragma once

#define TVM_FFI_DLL_EXPORT_TYPED_FUNC(name, fn) [[maybe_unused]] static auto* const tvm_ffi_stub_export_##name = &fn
