// In-bounds check of the wave-level primitives the kernels rely on: DPP
// quad_perm / row_half_mirror / row_mirror / row_ror:8 and the gfx950
// permlane16/32 swaps, the row_shr prefix product, and the operand/result lane layout of
// v_mfma_f32_16x16x4_f32 that the GEMM kernels assume.  One wave, lane-indexed
// input, results copied back.
#include "common.h"
#include "runtime.h"

namespace asca {

constexpr int SELFTEST_COLS = 16;

__global__ __launch_bounds__(64) void selftest_wave_k(float* __restrict__ out) {
    const int l = threadIdx.x;
    const float x = (float)l;
    const float y = (float)(100 + l);
    float r[SELFTEST_COLS];
    r[0] = dpp<DPP_QUAD_XOR1>(x);
    r[1] = dpp<DPP_QUAD_XOR2>(x);
    r[2] = dpp<DPP_HALF_MIRROR>(x);
    r[3] = dpp<DPP_ROW_MIRROR>(x);
    r[4] = dpp<DPP_ROW_ROR8>(x);
    {
        auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
        r[5] = __uint_as_float(p[0]);
        r[6] = __uint_as_float(p[1]);
    }
    {
        auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
        r[7] = __uint_as_float(p[0]);
        r[8] = __uint_as_float(p[1]);
    }
    r[9] = wave_sum(x);
    {
        // small integers: the product is exact whatever the summation order
        const float a = (float)((l * 7) % 13 - 6);
        const float b = (float)((l * 5) % 11 - 5);
        f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
        d = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, d, 0, 0, 0);
        r[10] = d[0];
        r[11] = d[1];
        r[12] = d[2];
        r[13] = d[3];
    }
    {
        // powers of two: the products are exact
        const float z = __int_as_float((127 + (l * 3) % 5 - 2) << 23);
        r[14] = prefix_prod<8>(z);
        r[15] = prefix_prod<2>(z);
    }
#pragma unroll
    for (int c = 0; c < SELFTEST_COLS; ++c) out[c * 64 + l] = r[c];
}

}  // namespace asca

using namespace asca;

extern "C" int asca_selftest_wave(float* host_out) {
    if (!host_out) return fail(ASCA_ERR_INVALID, "null output pointer");
    int rc = pre_launch("selftest_wave");
    if (rc) return rc;
    float* d = nullptr;
    const size_t bytes = SELFTEST_COLS * 64 * sizeof(float);
    hipError_t e = hipMalloc(&d, bytes);
    if (e != hipSuccess) return fail(ASCA_ERR_OOM, "hipMalloc: %s", hipGetErrorString(e));
    hipLaunchKernelGGL(selftest_wave_k, dim3(1), dim3(64), 0, nullptr, d);
    rc = post_launch("selftest_wave");
    if (!rc) {
        e = hipMemcpy(host_out, d, bytes, hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = fail(ASCA_ERR_HIP, "hipMemcpy: %s", hipGetErrorString(e));
    }
    hipFree(d);
    return rc;
}
