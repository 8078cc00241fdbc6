// Batched single-token decode of the gated delta rule: the state math of
// DeltaBlock::step (rust/src/delta.rs:356-407) for n_seq independent
// sequences, states resident in HBM.  The reference runs this on the CPU only
// and caps dh at 64 (delta.rs:361-362); here dh is any value up to 128.
//
// Per (sequence, head): q, k from the raw qkv row are L2-normalised by
// multiplying with 1/max(|x|, 1e-8) (as step does), alpha = sigmoid(g_h),
// beta = sigmoid(g_{H+h}); sk = S^T k; u = beta (v - alpha sk);
// S = alpha S + k u^T (row-wise scale_axpy); o = S^T q.
//
// HBM-bound: S (dh^2 floats) is read and written once per step, the I/O is
// 3dh + 2 floats in and dh out.  One block per (sequence, head), thread = (row
// group rg = tid / 32 of RPT rows, column quad cq = tid % 32), so each row of S
// is read and written by 32 consecutive threads with 16-byte accesses.  The
// aligned path uses RPT = 8 (512 threads, ~80 VGPRs, six waves per SIMD) and
// non-temporal loads and stores for S, which is touched once per step and is
// far larger than the caches (measured: 73.8% of HBM peak against 62.9% with
// 16 rows per thread and ordinary accesses).  S^T k and S^T q are reduced over
// the two row groups of a wave with one permlane32 swap, then over the waves
// through LDS.
#include "common.h"
#include "runtime.h"

namespace asca {

template <int RPT>
struct Dec {
    static constexpr int NT = 32 * (128 / RPT);  // threads: 32 column quads x row groups
    static constexpr int W = NT / 64;
};

// FULL: dh is exactly 128 (every row and column of the tile exists), so no
// load carries a condition and the loads of a thread are all in flight
// together (a load under a condition is waited for on its own).
template <bool VEC, int RPT, bool NTMP, bool FULL = false>
__global__ __launch_bounds__(Dec<RPT>::NT) void delta_decode_k(float* __restrict__ states,
                                                               const float* __restrict__ qkv,
                                                               const float* __restrict__ gate, float* __restrict__ o,
                                                               int H, int dh) {
    constexpr int W = Dec<RPT>::W;
    __shared__ float4 red[W][32];
    __shared__ float4 sk_s[32];
    const int unit = blockIdx.x;               // n * H + h
    const int n = unit / H, h = unit - n * H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int cq = tid & 31, rg = tid >> 5;    // column quad, row group
    const int c0 = cq * 4, r0 = rg * RPT;
    const long d = (long)H * dh;
    const float* row = qkv + (long)n * 3 * d;
    const float* qh = row + (long)h * dh;
    const float* kh = row + d + (long)h * dh;
    const float* vh = row + 2 * d + (long)h * dh;
    float* S = states + (long)unit * dh * dh;

    // state tile: rows r0..r0+RPT-1, columns c0..c0+3 (loads issued first)
    float4 s[RPT];
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
        const int a = r0 + j;
        if constexpr (VEC) {
            if (FULL || (a < dh && c0 < dh)) {
                const f32x4* src = reinterpret_cast<const f32x4*>(S + (long)a * dh + c0);
                const f32x4 x = NTMP ? __builtin_nontemporal_load(src) : *src;
                s[j] = make_float4(x[0], x[1], x[2], x[3]);
            } else {
                s[j] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        } else {
            float* e = reinterpret_cast<float*>(&s[j]);
#pragma unroll
            for (int x = 0; x < 4; ++x) e[x] = (a < dh && c0 + x < dh) ? S[(long)a * dh + c0 + x] : 0.0f;
        }
    }
    // norms of q and k over dh <= 128 elements, each wave on its own
    float qq = 0.0f, kk = 0.0f;
#pragma unroll
    for (int x = 0; x < 2; ++x) {
        const int i = lane + 64 * x;
        const float qv = FULL || i < dh ? qh[i] : 0.0f;
        const float kv = FULL || i < dh ? kh[i] : 0.0f;
        qq = fmaf(qv, qv, qq);
        kk = fmaf(kv, kv, kk);
    }
    qq = wave_sum(qq);
    kk = wave_sum(kk);
    const float qi = 1.0f / fmaxf(sqrtf(qq), 1e-8f);
    const float ki = 1.0f / fmaxf(sqrtf(kk), 1e-8f);
    const float al = sigmoid_f(gate[(long)n * 2 * H + h]);
    const float be = sigmoid_f(gate[(long)n * 2 * H + H + h]);
    float kr[RPT], qr[RPT];
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
        const int a = r0 + j;
        kr[j] = FULL || a < dh ? kh[a] * ki : 0.0f;
        qr[j] = FULL || a < dh ? qh[a] * qi : 0.0f;
    }
    float vv[4];
#pragma unroll
    for (int x = 0; x < 4; ++x) vv[x] = FULL || c0 + x < dh ? vh[c0 + x] : 0.0f;

    // sk = S^T k over this thread's rows, then the row groups
    float4 p = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
        p.x = fmaf(kr[j], s[j].x, p.x);
        p.y = fmaf(kr[j], s[j].y, p.y);
        p.z = fmaf(kr[j], s[j].z, p.z);
        p.w = fmaf(kr[j], s[j].w, p.w);
    }
    p.x = add_xor32(p.x);
    p.y = add_xor32(p.y);
    p.z = add_xor32(p.z);
    p.w = add_xor32(p.w);
    if (lane < 32) red[w][cq] = p;
    __syncthreads();
    if (tid < 32) {
        float4 t = red[0][tid];
#pragma unroll
        for (int ww = 1; ww < W; ++ww) {
            const float4 x = red[ww][tid];
            t.x += x.x; t.y += x.y; t.z += x.z; t.w += x.w;
        }
        sk_s[tid] = t;
    }
    __syncthreads();
    const float4 sk = sk_s[cq];
    const float u[4] = {be * (vv[0] - al * sk.x), be * (vv[1] - al * sk.y), be * (vv[2] - al * sk.z),
                        be * (vv[3] - al * sk.w)};

    // S = alpha S + k u^T (fma(k_a, u_i, alpha S), the order of simd::scale_axpy), o = S^T q
    float4 po = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
        s[j].x = fmaf(kr[j], u[0], al * s[j].x);
        s[j].y = fmaf(kr[j], u[1], al * s[j].y);
        s[j].z = fmaf(kr[j], u[2], al * s[j].z);
        s[j].w = fmaf(kr[j], u[3], al * s[j].w);
        po.x = fmaf(qr[j], s[j].x, po.x);
        po.y = fmaf(qr[j], s[j].y, po.y);
        po.z = fmaf(qr[j], s[j].z, po.z);
        po.w = fmaf(qr[j], s[j].w, po.w);
    }
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
        const int a = r0 + j;
        if constexpr (VEC) {
            if (FULL || (a < dh && c0 < dh)) {
                f32x4* dst = reinterpret_cast<f32x4*>(S + (long)a * dh + c0);
                const f32x4 x = {s[j].x, s[j].y, s[j].z, s[j].w};
                if (NTMP)
                    __builtin_nontemporal_store(x, dst);
                else
                    *dst = x;
            }
        } else {
            const float* e = reinterpret_cast<const float*>(&s[j]);
#pragma unroll
            for (int x = 0; x < 4; ++x)
                if (a < dh && c0 + x < dh) S[(long)a * dh + c0 + x] = e[x];
        }
    }
    po.x = add_xor32(po.x);
    po.y = add_xor32(po.y);
    po.z = add_xor32(po.z);
    po.w = add_xor32(po.w);
    __syncthreads();  // red reused
    if (lane < 32) red[w][cq] = po;
    __syncthreads();
    if (tid < 32) {
        float4 t = red[0][tid];
#pragma unroll
        for (int ww = 1; ww < W; ++ww) {
            const float4 x = red[ww][tid];
            t.x += x.x; t.y += x.y; t.z += x.z; t.w += x.w;
        }
        const int c = tid * 4;
        float* oh = o + (long)n * d + (long)h * dh;
        const float* e = reinterpret_cast<const float*>(&t);
#pragma unroll
        for (int x = 0; x < 4; ++x)
            if (FULL || c + x < dh) oh[c + x] = e[x];
    }
}

}  // namespace asca

using namespace asca;

extern "C" int asca_delta_decode_step(float* states, const float* qkv, const float* gate, float* o, int n_seq, int H,
                                      int dh, void* stream) {
    if (n_seq < 0 || H < 0) return fail(ASCA_ERR_INVALID, "negative shape n_seq=%d H=%d", n_seq, H);
    if (dh <= 0 || dh > 128) return fail(ASCA_ERR_UNSUPPORTED, "decode: dh=%d outside 1..128", dh);
    if ((long)n_seq * H == 0) return ASCA_OK;
    if (!states || !qkv || !gate || !o) return fail(ASCA_ERR_INVALID, "null pointer in asca_delta_decode_step");
    if ((long)n_seq * H > 0x7fffffffL) return fail(ASCA_ERR_INVALID, "n_seq*H too large");
    int rc = pre_launch("delta_decode");
    if (rc) return rc;
    const bool vec = dh % 4 == 0 && (reinterpret_cast<uintptr_t>(states) & 15) == 0;
    const hipStream_t st = as_stream(stream);
    if (vec && dh == 128)
        hipLaunchKernelGGL((delta_decode_k<true, 8, true, true>), dim3(n_seq * H), dim3(Dec<8>::NT), 0, st, states,
                           qkv, gate, o, H, dh);
    else if (vec)
        hipLaunchKernelGGL((delta_decode_k<true, 8, true>), dim3(n_seq * H), dim3(Dec<8>::NT), 0, st, states, qkv,
                           gate, o, H, dh);
    else
        hipLaunchKernelGGL((delta_decode_k<false, 16, false>), dim3(n_seq * H), dim3(Dec<16>::NT), 0, st, states,
                           qkv, gate, o, H, dh);
    return post_launch("delta_decode");
}
