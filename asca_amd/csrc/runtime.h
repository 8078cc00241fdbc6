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

// Allow kernel `fn` `bytes` of dynamic LDS on the library's device.  Set once
// per (kernel, device) and remembered under a lock, so concurrent first calls
// from several host threads and a later asca_init on another device each set it.
int allow_lds(const void* fn, size_t bytes);

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
// reference's operators take none): each stream has one cached device buffer
// (from the library's stream-ordered pool, grown when a call needs more, the
// old one freed behind the work queued on that stream), so work on one stream
// uses it in stream order and calls on different streams never share it.
// get() holds a library lock until release() (or the destructor), so two host
// threads enqueueing on one stream do not interleave a grow with a launch.
struct StreamScratch {
    Ws ws{nullptr, 0};
    int get(size_t floats, hipStream_t st);
    int release(hipStream_t st);
    ~StreamScratch();

private:
    bool held_ = false;
};

// Drops the cached scratch of a stream that is about to be destroyed.
void stream_scratch_forget(hipStream_t st);

}  // namespace asca
