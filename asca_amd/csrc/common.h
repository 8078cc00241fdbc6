// Shared device helpers for the gfx950 (CDNA4) kernels of libasca_hip.
//
// Wave-level data movement uses DPP (quad_perm / row_half_mirror / row_mirror /
// row_ror) inside a 16-lane row and the gfx950 v_permlane16_swap /
// v_permlane32_swap instructions across rows, so reductions never touch LDS.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define ASCA_DEV __device__ __forceinline__

namespace asca {

// Accumulator type of the 16x16 MFMA instructions (four f32 per lane).
typedef float f32x4 __attribute__((ext_vector_type(4)));

// DPP control words (GCN3+/CDNA encodings).
constexpr int DPP_QUAD_XOR1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int DPP_ROW_MIRROR = 0x140; // lane i <- 15-i within a 16-lane row
constexpr int DPP_HALF_MIRROR = 0x141;// lane i <- 7-i within 8 lanes
constexpr int DPP_ROW_ROR8 = 0x128;   // lane i <- (i+8)&15: xor 8 inside a row

template <int CTRL>
ASCA_DEV float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// DPP move that leaves `old` in lanes whose source lane lies outside the row.
template <int CTRL>
ASCA_DEV float dpp_or(float old, float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Inclusive prefix product over the lanes of each 16-lane row, correct for the
// first N lanes of the row (N in 1, 2, 4, 8, 16): row_shr by 1, 2, 4, 8.
template <int N>
ASCA_DEV float prefix_prod(float x) {
    if constexpr (N > 1) x *= dpp_or<0x111>(1.0f, x);
    if constexpr (N > 2) x *= dpp_or<0x112>(1.0f, x);
    if constexpr (N > 4) x *= dpp_or<0x114>(1.0f, x);
    if constexpr (N > 8) x *= dpp_or<0x118>(1.0f, x);
    return x;
}

// x from lane (lane ^ 32) added to x: every lane receives the pair sum.
ASCA_DEV float add_xor32(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// x from lane (lane ^ 16) added to x.
ASCA_DEV float add_xor16(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Transposed pair reduction across lane^32: lanes < 32 return lo(own)+lo(partner),
// lanes >= 32 return hi(own)+hi(partner).  One swap, one add.
ASCA_DEV float tsum32(float lo, float hi) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Transposed pair reduction across lane^16: even 16-lane rows return lo sums,
// odd rows return hi sums.
ASCA_DEV float tsum16(float lo, float hi) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Butterfly sums over the low log2(N) lane bits (N in 1,2,4,8,16); the result is
// bitwise identical in every lane of the group.
template <int N>
ASCA_DEV float group_sum(float x) {
    if constexpr (N >= 2) x += dpp<DPP_QUAD_XOR1>(x);
    if constexpr (N >= 4) x += dpp<DPP_QUAD_XOR2>(x);
    if constexpr (N >= 8) x += dpp<DPP_HALF_MIRROR>(x);   // valid: quad-uniform
    if constexpr (N >= 16) x += dpp<DPP_ROW_MIRROR>(x);   // valid: 8-uniform
    return x;
}

// Sum over all 64 lanes, result in every lane.
ASCA_DEV float wave_sum(float x) {
    x = group_sum<16>(x);
    x = add_xor16(x);
    x = add_xor32(x);
    return x;
}

ASCA_DEV float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

// Raw buffer resource over `bytes` bytes at p: buffer stores whose offset is
// not below `bytes` are dropped by the hardware, so a store to a row past a
// sequence's end needs no exec-mask branch (which would split the scheduling
// region of the code around it).  Offsets are 32-bit byte offsets.
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr int RSRC_WORD3 = 0x00020000;   // raw 32-bit data, gfx9 (CDNA) encoding
ASCA_DEV Rsrc make_rsrc(const void* p, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, RSRC_WORD3);
}
ASCA_DEV void buf_store1(Rsrc r, unsigned off, float x, unsigned soff = 0) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), r, (int)off, (int)soff, 0);
}
// 16 bytes at byte offset off + soff (the whole store is dropped past the resource's size)
ASCA_DEV void buf_store4(Rsrc r, unsigned off, float4 x, unsigned soff = 0) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = {__float_as_uint(x.x), __float_as_uint(x.y), __float_as_uint(x.z), __float_as_uint(x.w)};
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, (int)soff, 0);
}
// Buffer loads at byte offset voff + soff (soff uniform: an SGPR, so a loop's
// per-lane offset is computed once and a block's offset costs no VALU); past
// the resource's size they return 0.
ASCA_DEV float buf_load1(Rsrc r, unsigned voff, unsigned soff) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}
ASCA_DEV float4 buf_load4(Rsrc r, unsigned voff, unsigned soff) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
    return make_float4(__uint_as_float(x[0]), __uint_as_float(x[1]), __uint_as_float(x[2]), __uint_as_float(x[3]));
}

// Workgroup barrier that orders LDS only.  __syncthreads() also waits for every
// outstanding global load and store of the wave (s_waitcnt vmcnt(0)), which
// turns a prefetch issued before it into a stall; kernels whose waves share
// nothing but LDS use this instead (s_waitcnt lgkmcnt(0); s_barrier).
ASCA_DEV void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace asca
