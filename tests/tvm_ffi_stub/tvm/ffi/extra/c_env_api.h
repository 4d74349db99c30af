// Test stand-in, not tvm-ffi: the stream query the shims call (the test driver
// defines it).
#pragma once

#include <cstdint>

extern "C" void* TVMFFIEnvGetStream(int32_t device_type, int32_t device_id);
