// Internal launchers of ops.hip shared with the composite operators
// (model.hip).  Not part of the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace asca {

// Stable counting sort of n tokens into E <= 256 buckets (hash_route(id) % E
// when `hash`, else the key itself); ws: asca_hash_route_ws_bytes bytes.
int bucket_launch(bool hash, const uint32_t* ids, int n, int E, int32_t* expert, int32_t* perm, int32_t* offsets,
                  void* ws, hipStream_t st);

// dx = res + rmsnorm_backward(x, dy) per row (res may be null).
int rmsnorm_bwd_launch(const float* x, const float* dy, const float* res, float* dx, long rows, int cols, float eps,
                       hipStream_t st);

}  // namespace asca
