// Test stand-in, not tvm-ffi: TVM_FFI_THROW(Kind) << message throws a
// tvm_ffi_stub::Error carrying the kind's name when the statement ends.
#pragma once

#include <sstream>
#include <stdexcept>
#include <string>

namespace tvm_ffi_stub {

struct Error : std::runtime_error {
  std::string kind;
  Error(std::string k, const std::string& msg) : std::runtime_error(msg), kind(std::move(k)) {}
};

class Thrower {
 public:
  explicit Thrower(const char* kind) : kind_(kind) {}
  template <class T>
  Thrower& operator<<(const T& x) {
    os_ << x;
    return *this;
  }
  ~Thrower() noexcept(false) { throw Error(kind_, os_.str()); }

 private:
  std::string kind_;
  std::ostringstream os_;
};

}  // namespace tvm_ffi_stub

#define TVM_FFI_THROW(kind) ::tvm_ffi_stub::Thrower(#kind)
