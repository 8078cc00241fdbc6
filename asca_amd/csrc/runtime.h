// Host-side internals shared by the libasca_hip translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/asca_hip.h"

namespace asca {

// Record an error message for asca_last_error() and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Make sure the calling thread has the library's device current (HIP's current
// device is per thread).  Returns ASCA_OK or an error code.
int ensure_device();

// Called before every kernel launch: counts launches and applies the fault
// injection set by asca_fail_after() / ASCA_FAIL_LAUNCH.
int pre_launch(const char* kernel);

// Map the HIP status of the launch just made to an error code.
int post_launch(const char* kernel);

// Convert an opaque stream handle from the C ABI.
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Number of compute units of the active device (0 before init).
int cu_count();

}  // namespace asca
