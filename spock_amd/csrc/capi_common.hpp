// capi_common.hpp -- status codes and per-thread error text for the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/spock_hip.h"

namespace spk {

// Records a formatted message for spk_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Checks hipGetLastError() after a launch; returns SPK_OK or SPK_ERR_HIP.
int check_launch(const char* what);

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline hipStream_t to_hip(spk_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace spk
