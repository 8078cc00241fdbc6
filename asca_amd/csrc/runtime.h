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

// Device address of the static scratch of asca_gemm_noalloc on `device` (the
// current device), taken once at asca_init (gemm.hip).
int noalloc_scratch_init(int device);

// A caller-provided device workspace of `floats` floats.
struct Ws {
    float* p;
    size_t floats;
};

// Scratch for the entry points that take no workspace argument (as the
// reference's operators take none): get() allocates from the stream-ordered
// allocator on the call's stream (hipMallocAsync), release() returns it behind
// the work queued so far (hipFreeAsync).  Calls on different streams never
// share scratch and nothing waits for the device.
struct StreamScratch {
    Ws ws{nullptr, 0};
    int get(size_t floats, hipStream_t st);
    int release(hipStream_t st);
};

}  // namespace asca
