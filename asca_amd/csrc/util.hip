// Plain streaming copy, used as the known-size reference kernel when HBM
// traffic counters (FETCH_SIZE / WRITE_SIZE) are calibrated.
#include "common.h"
#include "runtime.h"

namespace asca {

__global__ __launch_bounds__(256) void copy_f32_k(float4* __restrict__ dst, const float4* __restrict__ src,
                                                  long n4) {
    const long stride = (long)gridDim.x * blockDim.x;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) dst[i] = src[i];
}

}  // namespace asca

using namespace asca;

extern "C" int asca_copy_f32(float* dst, const float* src, size_t n, void* stream) {
    if (n == 0) return ASCA_OK;
    if (!dst || !src) return fail(ASCA_ERR_INVALID, "null pointer in asca_copy_f32");
    if (n % 4 || (reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15)
        return fail(ASCA_ERR_INVALID, "asca_copy_f32 needs 16-byte aligned buffers and n %% 4 == 0");
    int rc = pre_launch("copy_f32");
    if (rc) return rc;
    const long n4 = (long)(n / 4);
    const int cus = cu_count() > 0 ? cu_count() : 256;
    long blocks = (n4 + 255) / 256;
    if (blocks > (long)cus * 8) blocks = (long)cus * 8;
    hipLaunchKernelGGL(copy_f32_k, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                       reinterpret_cast<float4*>(dst), reinterpret_cast<const float4*>(src), n4);
    return post_launch("copy_f32");
}
