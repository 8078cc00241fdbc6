// Gated delta rule, recurrent form, f32, dh = 64, one block per (sequence,
// head) unit.
//
// Same math, outputs and workspace as delta.hip (DeltaBlock::scan_cpu,
// rust/src/delta.rs:244-334, and bptt_cpu, :421-613).  When every unit has a
// CU of its own (B*H > 128 on the 256 CUs of an MI355X), a unit's 4096 state
// elements fill the CU's four SIMDs with one wave each (16 elements per lane,
// which halves the per-element share of the reductions, gate scalars and
// operand reads against 8), and a second wave on each SIMD does the block's
// matrix products, outputs and staging beside it, so that each fills the
// other's stalls.
//
//  * Forward: lane = 4c + p of a state wave holds rows 16p..16p+15 of value
//    column 16w + c, so S^T k is a two-level quad DPP sum; the k rows sit in
//    LDS with row quarter p at float 20p, so the four distinct 16-byte
//    addresses of a 16-lane read fall on four distinct bank groups.  The
//    outputs o = S_j^T q_j of a 16-step chunk come from the matrix waves a
//    chunk later, as 16-row products of the chunk's first state, its u rows
//    and the products k . q (16x16x4 f32 MFMA).
//  * Backward: lane (rg = lane & 7, cg = lane >> 3) holds the adjoint's rows
//    8rg..8rg+7 of columns 16w + 2cg, +1, and a 16-step segment runs only the
//    adjoint recurrence step by step: du = dS^T k is an 8-lane DPP sum and dS
//    takes two rank-1 updates, 48 FMAs per lane and step.  Everything else is
//    a product of 16-row matrices per segment, on the matrix cores (16x16x4 f32
//    MFMA): dq and dk from the segment's first checkpoint, the adjoint at its
//    top and the 16 x 16 step mixes u~ . dO~ and u~ . dsk~, dalpha from one
//    exact <dS, S> at the segment's bottom carried up by per-step dot products
//    (see bsegment_sc).  The block has eight waves: when every gate of the unit
//    lies in [2^-6, 2^6], four run the adjoint loop of one segment while the
//    other four, one per SIMD beside them, run the products and the epilogue
//    of the segment before it (a two-stage pipeline, see the pipelined
//    backward).  A unit with a gate outside that range (zero, tiny or huge
//    values) runs every segment on four waves instead, a segment with such a
//    gate in the plain recurrence, recomputing every state it needs from its
//    first checkpoint.
#include "common.h"
#include "delta.h"
#include "runtime.h"

namespace asca {
namespace d64 {

constexpr int DH = 64;
constexpr int W = 4;          // waves per unit
constexpr int NT = 64 * W;
constexpr int CK = D64_CK;    // checkpoint interval = forward chunk = backward segment
constexpr int DH2 = DH * DH;

__device__ float g_trash64[NT * 8];
ASCA_DEV float readlane_f(float x, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l)); }
ASCA_DEV float* trash(int i) { return g_trash64 + (i & (NT * 8 - 1)); }

// Loads of 4 / 2 floats: one vector access when the base is 16-byte aligned (AL),
// scalar accesses otherwise.
template <bool AL>
ASCA_DEV float4 ld4(const float* __restrict__ p) {
    if constexpr (AL) return *reinterpret_cast<const float4*>(p);
    else return make_float4(p[0], p[1], p[2], p[3]);
}

// D += A B on a 16x16x4 f32 MFMA: lane l gives A[l % 16][l / 16] and
// B[l / 16][l % 16] and holds D[4 (l / 16) + r][l % 16] in register r.
ASCA_DEV f32x4 mfma4(float a, float b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

// ================================================================== forward

constexpr int SW = 8;                        // state waves of the forward
constexpr int FNT = 64 * (SW + W);           // forward block: SW state waves, then W matrix waves
// Pitch of every 64-float row in the forward's LDS (k, q, the state's S^T rows,
// u): 68 = 4 mod 32, so the 16-byte reads of eight consecutive rows at one
// offset, or of one row at eight consecutive offsets, fall on distinct banks.
constexpr int FP = 68;
// Chunk staging buffer (floats): k rows [CK][FP], q rows [CK][FP], the rows
// beta_j v_j (divided by G_{j+1} in a scaled chunk) [CK][DH] for the state
// waves, one gate table per matrix wave [W][CK][8], the chunk's flag and a sink
// for the writes of lanes without a table row.
constexpr int F_K = 0;
constexpr int F_Q = CK * FP;
constexpr int F_V = 2 * CK * FP;
constexpr int F_G = F_V + DH * CK;
constexpr int F_FLAG = F_G + W * CK * 8;
constexpr int F_SINK = F_FLAG + 4;
constexpr int F_BUF = F_SINK + 8;
static_assert(F_BUF % 4 == 0 && F_V % 4 == 0, "float4 buffers");
// The forward's LDS (floats): three staging buffers (chunk c in buffer c mod
// 3), then per chunk parity the state before the chunk as S^T rows, the
// chunk's u rows (u / G_{j+1} in a scaled chunk) and its rows S^T k (over G_j
// in a scaled chunk), and per chunk mod 3 the matrix waves' partial products
// k . q.
constexpr int F_ST = 3 * F_BUF;                  // [2][DH][FP]
constexpr int F_U = F_ST + 2 * DH * FP;          // [2][CK][FP]
constexpr int F_X = F_U + 2 * CK * FP;           // [2][CK][FP]
constexpr int F_GP = F_X + 2 * CK * FP;          // [3][W][64] float4
constexpr int F_END = F_GP + 3 * W * 64 * 4;
constexpr size_t F_LDS = (size_t)F_END * 4;
static_assert(F_LDS <= 160 * 1024 && F_ST % 4 == 0 && F_GP % 4 == 0, "forward LDS");

struct FStage {
    float4 kq[2]; // two float4 of the chunk's k or q rows
    float4 v;     // one float4 of the chunk's v rows
    float a, b;   // lane j (mod CK): alpha, beta of step t0 + j (as loaded)
};

// Global -> registers for chunk c by the staging thread tx (0..NT-1) of matrix
// wave w = tx / 64, which stages the k and q columns 16 w .. 16 w + 15 of every
// step (the ones its own products fgram read); every lane loads (clamped
// addresses), so no load sits under a lane condition.
template <bool AL>
ASCA_DEV void fstage_load(FStage& st, int c, const float* __restrict__ q, const float* __restrict__ k,
                          const float* __restrict__ v, const float* __restrict__ alpha,
                          const float* __restrict__ beta, long ubase, long gbase, long d, int T, int H, int tx,
                          int lane) {
    const int t0 = c * CK;
    {
        const int j = lane >> 2, c4 = 4 * (tx >> 6) + (lane & 3);
        const long t = min(t0 + j, T - 1);
        st.kq[0] = ld4<AL>(k + ubase + t * d + 4 * c4);
        st.kq[1] = ld4<AL>(q + ubase + t * d + 4 * c4);
    }
    {
        const int j = tx >> 4, c4 = tx & 15;
        const long t = min(t0 + j, T - 1);
        st.v = ld4<AL>(v + ubase + t * d + 4 * c4);
    }
    {
        // raw values: fstage_store applies the padding past T, so that no
        // arithmetic on the loads waits for them here
        const long tc = min(t0 + (lane & (CK - 1)), T - 1);
        st.a = alpha[gbase + tc * H];
        st.b = beta[gbase + tc * H];
    }
}

// Registers -> the chunk buffer by staging thread tx of matrix wave w; wave w
// builds gate table w, row j = {beta_j, 1/G_{j+1}, alpha_j, alpha_j beta_j,
// G_{j+1}, G_j, 0, 0}, and wave 0 the flag: whether every alpha of the chunk
// lies in [2^-6, 2^6], the range in which the scaled state of a 16-step chunk
// stays within 2^+-96 of the true one.  The state waves' v rows carry beta_j
// (and 1/G_{j+1} when the chunk is scaled) already.
ASCA_DEV void fstage_store(const FStage& st, int c, int T, float* __restrict__ buf, int tx, int w, int lane) {
    {
        const int j = lane >> 2, c4 = 4 * w + (lane & 3);
        *reinterpret_cast<float4*>(buf + F_K + j * FP + 4 * c4) = st.kq[0];
        *reinterpret_cast<float4*>(buf + F_Q + j * FP + 4 * c4) = st.kq[1];
    }
    float sa = st.a, sb = st.b;
    asm volatile("" : "+v"(sa), "+v"(sb));   // keeps the gate arithmetic here, after the loads' wait
    // steps past T: alpha = 1, beta = 0 leave the state unchanged
    if (c * CK + (lane & (CK - 1)) >= T) {
        sa = 1.0f;
        sb = 0.0f;
    }
    const bool gl = lane < CK;
    const float pr = prefix_prod<CK>(gl ? sa : 1.0f);   // G_{j+1} in lane j
    const float pv = dpp_or<0x111>(1.0f, pr);            // G_j (row_shr 1; lane 0 keeps 1)
    const float rp = __builtin_amdgcn_rcpf(pr);
    float* const row = gl ? buf + F_G + (w * CK + lane) * 8 : buf + F_SINK;
    *reinterpret_cast<float4*>(row) = make_float4(sb, rp, sa, sa * sb);
    *reinterpret_cast<float2*>(row + 4) = make_float2(pr, pv);
    const bool bad = gl && !(sa >= 0x1p-6f && sa <= 0x1p6f);
    const bool scal = __ballot(bad) == 0;
    *(w == 0 && lane == 0 ? buf + F_FLAG : buf + F_SINK + 3) = scal ? 1.0f : 0.0f;
    {
        // row j of v times beta_j (over G_{j+1} when scaled), the factor taken
        // from lane j of this wave
        const int j = tx >> 4, c4 = tx & 15;
        const float fj = __shfl(scal ? sb * rp : sb, j);
        *reinterpret_cast<float4*>(buf + F_V + j * DH + 4 * c4) =
            make_float4(st.v.x * fj, st.v.y * fj, st.v.z * fj, st.v.w * fj);
    }
}

ASCA_DEV void st4(float* __restrict__ dst, float a, float b, float c, float e) {
    *reinterpret_cast<float4*>(dst) = make_float4(a, b, c, e);
}

// State wave w (0..SW-1), lane = 8 c + g: column 8 w + c, rows 4 g .. 4 g + 3
// (s[0..3]) and 32 + 4 g .. 32 + 4 g + 3 (s[4..7]), so the 8 lanes of a column
// hold its 64 rows, S^T k is three DPP levels inside them, and the two 16-byte
// k reads of a step cover 32 consecutive floats across the 8 lanes (distinct
// banks).  The CK steps of a chunk (rust/src/delta.rs:289-314 per step,
// without the output o).  Step j
// writes its column's u (u / G_{j+1} when scaled) and x = S^T k (over G_j when
// scaled) to row j of the chunk's u and x rows; the matrix waves take them from
// there (the outputs, the stored S^T k).  The gates arrive lane-distributed
// (lane j: step j) and are read out with v_readlane.  No barrier inside the
// chunk: the matrix waves never write what the state waves read in it.
//   SC = false: s is the state; u = beta v - alpha beta x, S <- alpha S + k u^T.
//   SC = true:  s = S / G_j; x = s^T k, u / G_{j+1} = beta v / G_{j+1} - beta x and
//     s <- s + k (u / G_{j+1})^T (one FMA per element).
template <bool SC>
ASCA_DEV void fsteps(float (&s)[8], const float* __restrict__ ks, const float (&vb)[CK], float gb, float ga,
                     float gab, float* __restrict__ ub, float* __restrict__ xb) {
    float4 kk[2][2];
    kk[0][0] = *reinterpret_cast<const float4*>(ks);
    kk[0][1] = *reinterpret_cast<const float4*>(ks + 32);
#pragma unroll
    for (int j = 0; j < CK; ++j) {
        const int cs = j & 1;
        if (j + 1 < CK) {
            kk[cs ^ 1][0] = *reinterpret_cast<const float4*>(ks + (j + 1) * FP);
            kk[cs ^ 1][1] = *reinterpret_cast<const float4*>(ks + (j + 1) * FP + 32);
        }
        // the reads of step j + 1 stay at the top of step j, a whole step ahead
        // of their use
        __builtin_amdgcn_sched_barrier(0);
        const float kv[8] = {kk[cs][0].x, kk[cs][0].y, kk[cs][0].z, kk[cs][0].w,
                             kk[cs][1].x, kk[cs][1].y, kk[cs][1].z, kk[cs][1].w};
        float a = s[0] * kv[0];
#pragma unroll
        for (int m = 1; m < 8; ++m) a = fmaf(s[m], kv[m], a);
        const float x = group_sum<8>(a);
        float u0;
        if constexpr (SC) {
            u0 = fmaf(-readlane_f(gb, j), x, vb[j]);
#pragma unroll
            for (int m = 0; m < 8; ++m) s[m] = fmaf(kv[m], u0, s[m]);
        } else {
            u0 = fmaf(-readlane_f(gab, j), x, vb[j]);
            const float al = readlane_f(ga, j);
#pragma unroll
            for (int m = 0; m < 8; ++m) s[m] = fmaf(al, s[m], kv[m] * u0);
        }
        // the 8 lanes of a column store the same values
        ub[j * FP] = u0;
        xb[j * FP] = x;
    }
}

// Matrix wave mw: the outputs o of one chunk for the columns 16 mw .. 16 mw +
// 15 of every step, rows j:
//   scaled chunk: o = G_{j+1} (S^T q_j + sum_{l <= j} u~_l (k_l . q_j))
//   plain chunk:  o = G_{j+1} S^T q_j + sum_{l <= j} Gamma_{jl} u_l (k_l . q_j)
// with S the state before the chunk, G_{j+1} the product of the chunk's alpha
// up to step j and Gamma_{jl} that from step l + 1 to j (both formed by
// multiplication only).  S^T q runs on the matrix cores (16x16x4 f32 MFMA) from
// the q rows and the state's rows, as two accumulation chains; the 16 x 16
// products k_l . q_j arrive as per-wave partials (fgram, a chunk earlier) in
// exactly the lane layout the step mix takes as its operand (l = 4 gq + r).
// The wave also stores the chunk's checkpoint rows 16 mw .. 16 mw + 15 (S^T,
// read here for S^T q) and the S^T k of its columns (times G_j in a scaled
// chunk) from the state waves' x rows.
ASCA_DEV void fprod(const float* __restrict__ buf, const float* __restrict__ st, const float* __restrict__ ub,
                    const float* __restrict__ xb, const float4* __restrict__ gpart, int mw, int lane,
                    float* __restrict__ od, float* __restrict__ skd, float* __restrict__ ckd, long d, int nvalid,
                    float* __restrict__ tr) {
    const int jr = lane & 15, gq = lane >> 4;
    const bool sc = buf[F_FLAG] == 1.0f;
    const float* const gt = buf + F_G;   // gate table 0
    // k_l . q_jr for l = 4 gq + r, masked to l <= jr (plain: times Gamma)
    float4 gm = gpart[lane];
#pragma unroll
    for (int v4 = 1; v4 < W; ++v4) {
        const float4 y = gpart[v4 * 64 + lane];
        gm.x += y.x; gm.y += y.y; gm.z += y.z; gm.w += y.w;
    }
    float am[4] = {gm.x, gm.y, gm.z, gm.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int l = 4 * gq + r;
        if (!sc) {
            float x = 1.0f;
#pragma unroll
            for (int m = 1; m < CK; ++m) x *= (m > l && m <= jr) ? gt[m * 8 + 2] : 1.0f;
            am[r] *= x;
        }
        am[r] = l <= jr ? am[r] : 0.0f;
    }
    f32x4 a1[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}}, a2 = a1[0];
    // S^T q: k index a = 16 m + 4 gq + e (e = 0..3), both operands as 16-byte vectors
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const float4 x = *reinterpret_cast<const float4*>(buf + F_Q + jr * FP + 16 * m + 4 * gq);
        const float4 y = *reinterpret_cast<const float4*>(st + (16 * mw + jr) * FP + 16 * m + 4 * gq);
        f32x4& acc = a1[m & 1];
        acc = mfma4(x.x, y.x, acc);
        acc = mfma4(x.y, y.y, acc);
        acc = mfma4(x.z, y.z, acc);
        acc = mfma4(x.w, y.w, acc);
        *reinterpret_cast<float4*>(ckd + (16 * mw + jr) * DH + 16 * m + 4 * gq) = y;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) a2 = mfma4(am[r], ub[(4 * gq + r) * FP + 16 * mw + jr], a2);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int j = 4 * gq + r;
        const float xv = xb[j * FP + 16 * mw + jr];
        *(j < nvalid ? skd + j * d + 16 * mw + jr : tr + 4 + r) = sc ? xv * gt[j * 8 + 5] : xv;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int j = 4 * gq + r;
        const float g1 = gt[j * 8 + 4];
        const float sq = a1[0][r] + a1[1][r];
        const float ov = sc ? g1 * (sq + a2[r]) : fmaf(g1, sq, a2[r]);
        *(j < nvalid ? od + j * d + 16 * mw + jr : tr + r) = ov;
    }
}

// Matrix wave mw: its partial of the products k_l . q_j of a chunk over the
// rows a = 16 mw .. 16 mw + 15, as D = K Q^T (MFMA e takes a = 16 mw + 4 gq + e
// from lane group gq, so each lane reads its operands as one 16-byte vector),
// so that lane (gq, jr) register r holds k_{4gq+r} . q_jr.  It reads only what
// the wave's own lanes staged (fstage_store), right after staging them.
ASCA_DEV void fgram(const float* __restrict__ buf, float4* __restrict__ gpart, int mw, int lane) {
    const int jr = lane & 15, gq = lane >> 4;
    // the wave reads back what its own lanes wrote
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float4 x = *reinterpret_cast<const float4*>(buf + F_K + jr * FP + 16 * mw + 4 * gq);
    const float4 y = *reinterpret_cast<const float4*>(buf + F_Q + jr * FP + 16 * mw + 4 * gq);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    acc = mfma4(x.x, y.x, acc);
    acc = mfma4(x.y, y.y, acc);
    acc = mfma4(x.z, y.z, acc);
    acc = mfma4(x.w, y.w, acc);
    gpart[mw * 64 + lane] = make_float4(acc[0], acc[1], acc[2], acc[3]);
}

// One block per unit = h*B + b (the reference's s_pre order,
// rust/src/delta.rs:54-56), as a two-stage pipeline over chunks: in period c
// the state waves (0..SW-1, two per SIMD) run chunk c while the matrix waves
// (SW..SW+W-1, one per SIMD) form the outputs of chunk c - 1, then stage chunk
// c + 1 and its partial products k . q.  One block barrier per period, at its
// start: with three staging buffers the buffer being restaged (that of chunk
// c - 2) is one that no wave reads any more in the period.
template <bool AL>
__global__ __launch_bounds__(FNT) void delta_fwd64_k(const float* __restrict__ q, const float* __restrict__ k,
                                                     const float* __restrict__ v, const float* __restrict__ alpha,
                                                     const float* __restrict__ beta, float* __restrict__ o,
                                                     float* __restrict__ sk_out, float* __restrict__ ckpt, int B,
                                                     int T, int H, int nslots) {
    extern __shared__ float4 lds4[];
    float* const lds = reinterpret_cast<float*>(lds4);
    const int unit = blockIdx.x;
    const int h = unit / B, b = unit - h * B;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const long d = (long)H * DH;
    const long ubase = (long)b * T * d + (long)h * DH;
    const long gbase = (long)b * T * H + h;
    const int nchunk = (T + CK - 1) / CK;
    float* const tr = trash((threadIdx.x & (NT - 1)) * 8);

    if (w < SW) {
        // state waves
        const int g = lane & 7, col = 8 * w + (lane >> 3);
        float s[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) s[m] = 0.0f;
        lds_barrier();   // chunk 0 staged
        for (int ci = 0, b3 = 0; ci < nchunk; ++ci, b3 = b3 == 2 ? 0 : b3 + 1) {
            lds_barrier();   // P0
            const float* const buf = lds + b3 * F_BUF;
            const float* const gt = buf + F_G + (w & (W - 1)) * CK * 8;
            const bool sc = __builtin_amdgcn_readfirstlane(__float_as_int(buf[F_FLAG])) == __float_as_int(1.0f);
            float vb[CK];
#pragma unroll
            for (int j = 0; j < CK; ++j) vb[j] = buf[F_V + j * DH + col];
            // lane j (< CK): step j's gate row
            const float4 g4 = *reinterpret_cast<const float4*>(gt + (lane & (CK - 1)) * 8);
            // the state before the chunk (the checkpoint) as S^T rows
            float* const stb = lds + F_ST + (ci & 1) * DH * FP + col * FP + 4 * g;
            st4(stb, s[0], s[1], s[2], s[3]);
            st4(stb + 32, s[4], s[5], s[6], s[7]);
            float* const ub = lds + F_U + (ci & 1) * CK * FP + col;
            float* const xb = lds + F_X + (ci & 1) * CK * FP + col;
            if (sc) {
                fsteps<true>(s, buf + F_K + 4 * g, vb, g4.x, g4.z, g4.w, ub, xb);
                const float ge = gt[(CK - 1) * 8 + 4];
#pragma unroll
                for (int m = 0; m < 8; ++m) s[m] *= ge;
            } else {
                fsteps<false>(s, buf + F_K + 4 * g, vb, g4.x, g4.z, g4.w, ub, xb);
            }
        }
        lds_barrier();   // P0 of the period in which the matrix waves finish the last chunk
        // the state after step T-1
        float* const ckl = ckpt + ((long)unit * nslots + nchunk) * DH2 + col * DH + 4 * g;
        st4(ckl, s[0], s[1], s[2], s[3]);
        st4(ckl + 32, s[4], s[5], s[6], s[7]);
    } else {
        // matrix waves
        const int mw = w - SW, tx = threadIdx.x - 64 * SW;
        FStage stg;
        float4* const gp = reinterpret_cast<float4*>(lds + F_GP);
        fstage_load<AL>(stg, 0, q, k, v, alpha, beta, ubase, gbase, d, T, H, tx, lane);
        fstage_store(stg, 0, T, lds, tx, mw, lane);
        fgram(lds, gp, mw, lane);
        // the loads of chunk ci + 2 are issued in period ci, right after the
        // store of chunk ci + 1, a whole period ahead of their own store
        if (nchunk > 1) fstage_load<AL>(stg, 1, q, k, v, alpha, beta, ubase, gbase, d, T, H, tx, lane);
        lds_barrier();   // chunk 0 staged
        for (int ci = 0, b3 = 0; ci <= nchunk; ++ci, b3 = b3 == 2 ? 0 : b3 + 1) {
            lds_barrier();   // P0
            if (ci > 0) {
                const int cp = ci - 1, bp = b3 == 0 ? 2 : b3 - 1;
                fprod(lds + bp * F_BUF, lds + F_ST + (cp & 1) * DH * FP, lds + F_U + (cp & 1) * CK * FP,
                      lds + F_X + (cp & 1) * CK * FP, gp + bp * W * 64, mw, lane,
                      o + ubase + (long)cp * CK * d, sk_out + ubase + (long)cp * CK * d,
                      ckpt + ((long)unit * nslots + cp) * DH2, d, T - cp * CK, tr);
            }
            if (ci + 1 < nchunk) {
                const int bn = b3 == 2 ? 0 : b3 + 1;
                fstage_store(stg, ci + 1, T, lds + bn * F_BUF, tx, mw, lane);
                if (ci + 2 < nchunk)
                    fstage_load<AL>(stg, ci + 2, q, k, v, alpha, beta, ubase, gbase, d, T, H, tx, lane);
                fgram(lds + bn * F_BUF, gp + bn * W * 64, mw, lane);
            }
        }
    }
}
// ================================================================= backward

constexpr int BM = 8;       // adjoint rows per lane (two columns each)
constexpr int P = 68;       // LDS pitch of every 64-float row
// Position of element r in a padded row (4 floats after the first 32): the
// 16-byte reads of rows 8 rg .. 8 rg + 7 by the eight row groups of the adjoint
// loop then fall on distinct banks.
ASCA_DEV int rpad(int r) { return r + 4 * (r >> 5); }

// k-order of a 64-float row for the 16x16x4 f32 MFMA: position 16 g + kb
// holds column kcol(g, kb) = 16 (kb >> 2) + 4 g + (kb & 3).  Lane group g of an
// MFMA then reads the 16 values it feeds as four 16-byte vectors, the strided
// reads of a 64-row matrix by the four lane groups fall on disjoint banks, and
// the columns 2c, 2c + 1 of the adjoint loop stay adjacent (one 8-byte access).
ASCA_DEV int kpos(int i) { return 16 * ((i >> 2) & 3) + 4 * (i >> 4) + (i & 3); }
ASCA_DEV int kcol(int g, int kb) { return 16 * (kb >> 2) + 4 * g + (kb & 3); }


// Segment staging buffer (floats), written while the previous segment runs:
constexpr int S_Q = 0;                   // [CK][P] q rows, element a at rpad(a)
constexpr int S_K = S_Q + CK * P;        // [CK][P] k rows, element a at rpad(a)
constexpr int S_DO = S_K + CK * P;       // [CK][P] dO, k-order (scaled segment: G_{j+1} dO_j)
constexpr int S_U = S_DO + CK * P;       // [CK][P] u = beta (v - alpha sk), k-order (scaled: u_j / G_{j+1})
constexpr int S_SK = S_U + CK * P;       // [CK][P] sk, k-order
constexpr int S_WV = S_SK + CK * P;      // [CK][P] v - alpha sk, k-order
constexpr int S_M = S_WV + CK * P;       // [DH][P] the state before the segment as S^T (row i = column i of S)
constexpr int S_G = S_M + DH * P;        // [CK][8] gate table; the scaled-segment flag at S_G + 8 CK
constexpr int S_SINK = S_G + 8 * CK + 4;
constexpr int S_BUF = S_SINK + 12;
// Work area after the two staging buffers.  A scaled segment uses:
constexpr int W_XT = 0;                      // [DH][P] adjoint at the segment's top (scaled), row i = column i
constexpr int W_DSK = W_XT + DH * P;         // [CK][P] G_j dsk_j, k-order
constexpr int W_PP = W_DSK + CK * P;         // [W][CK][17] partial products u~ . dO~ over each wave's columns
constexpr int W_RP = W_PP + W * CK * 17;     // [W][CK][17] partial products u~ . dsk~
constexpr int W_DQ = W_RP + W * CK * 17;     // [CK][P] dq rows
// a plain segment, over the same space: per-wave dq and dk row partials
constexpr int W_RQ = 0;                      // [CK][W][P]
constexpr int W_RK = CK * W * P;             // [CK][W][P]
constexpr int W_DK = W_DQ + CK * P;          // [CK][P] dk rows
constexpr int W_DU = W_DK + CK * P;          // [CK][P] du, k-order
constexpr int W_AB = W_DU + CK * P;          // [CK][W][2] per-wave step sums (see the segment bodies)
constexpr int W_QDQ = W_AB + CK * W * 2;     // [W][CK] per-wave partial q . dq
constexpr int W_KDK = W_QDQ + W * CK;        // [W][CK] per-wave partial k . dk
constexpr int W_BR = W_KDK + W * CK;         // [W] per-wave partial <dS, S> at the segment's bottom
constexpr int W_END = W_BR + 8;
static_assert(W_RK + CK * W * P == W_DK, "plain partials fill the scaled segment's space");
static_assert(S_BUF % 4 == 0 && S_G % 4 == 0 && W_DQ % 4 == 0 && W_DU % 4 == 0, "16-byte rows");
constexpr size_t B_LDS = (2 * (size_t)S_BUF + W_END) * 4;
static_assert(B_LDS <= 160 * 1024, "backward LDS");

// Gate rows (S_G + 8 j): alpha, beta, G_{j+1}, 1/G_{j+1}, 1/alpha, |q|, |k|.
// Global -> registers for segment g; every lane loads (clamped addresses).
// (vectors first: a scalar member ahead of the float4 array kept the compiler
// from promoting the whole struct to registers)
struct BStage {
    float4 rq[2];    // two float4 of the segment's q or k rows
    float4 rw[3];    // row j = tid / 16, floats 4 (tid % 16) .. + 3 of dO, v, sk
    float4 rm[4];    // the state before the segment: S^T rows 16 e + tid / 16
    float rab;       // lane j < CK: alpha of step j; CK <= j < 2CK: beta (as loaded)
    float rqk;       // the same lanes: |q|, |k| (fused backward)
};

template <bool FUSED, bool AL>
ASCA_DEV void bstage_load(BStage& st, int g, const float* __restrict__ q, const float* __restrict__ k,
                          const float* __restrict__ v, const float* __restrict__ d_o,
                          const float* __restrict__ skv, const float* __restrict__ alpha,
                          const float* __restrict__ beta, const float* __restrict__ qnorm,
                          const float* __restrict__ knorm, const float* __restrict__ ckb, long ubase, long gbase,
                          long d, int T, int H, int tx, int lane) {
    const int t0 = g * CK;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int f = tx + NT * i;
        const int tsr = f >> 8, j = (f >> 4) & (CK - 1), c4 = f & 15;
        const long t = min(t0 + j, T - 1);
        st.rq[i] = ld4<AL>((tsr ? k : q) + ubase + t * d + 4 * c4);
    }
    {
        const int j = tx >> 4, c4 = tx & 15;
        const long o = ubase + (long)min(t0 + j, T - 1) * d + 4 * c4;
        st.rw[0] = ld4<AL>(d_o + o);
        st.rw[1] = ld4<AL>(v + o);
        st.rw[2] = ld4<true>(skv + o);   // the workspace's, always aligned
    }
    {
        const int gl = lane & (2 * CK - 1);
        const long tc = min(t0 + (gl & (CK - 1)), T - 1);
        // raw values: bstage_store applies the padding past T, so these loads
        // never turn into loads under a lane condition
        st.rab = (gl < CK ? alpha : beta)[gbase + tc * H];
        st.rqk = FUSED ? (gl < CK ? qnorm : knorm)[gbase + tc * H] : 0.0f;
    }
    const float* const cs = ckb + (long)g * DH2;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        st.rm[e] = *reinterpret_cast<const float4*>(cs + (long)(16 * e + (tx >> 4)) * DH + 4 * (tx & 15));
}

// Registers -> the staging buffer nb of segment g.  Every wave derives the
// gates, G_{j+1} and the segment's flag from its own copy of the gate loads.
// Steps past T get alpha = 1, beta = 0 and dO = 0, which leave the adjoint
// and every sum unchanged.
// tx: the thread's index among the NT staging threads, w: their wave.
ASCA_DEV void bstage_store(const BStage& st, int g, int T, float* __restrict__ nb, int tx, int w, int lane) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int f = tx + NT * i;
        const int tsr = f >> 8, j = (f >> 4) & (CK - 1), c4 = f & 15;
        *reinterpret_cast<float4*>(nb + (tsr ? S_K : S_Q) + j * P + rpad(4 * c4)) = st.rq[i];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
        *reinterpret_cast<float4*>(nb + S_M + (16 * e + (tx >> 4)) * P + 4 * (tx & 15)) = st.rm[e];
    // Both segment bodies store here; without this opaque copy the compiler
    // hoists the identical gate arithmetic of the two into the segment's
    // start, right behind the loads it waits for.
    float rab = st.rab, rqk = st.rqk;
    asm volatile("" : "+v"(rab), "+v"(rqk));
    const bool ga = lane < CK;
    const bool gb = lane >= CK && lane < 2 * CK;
    if (g * CK + (lane & (CK - 1)) >= T) rab = ga ? 1.0f : 0.0f;
    const float pr = prefix_prod<CK>(ga ? rab : 1.0f);   // lane j < CK: G_{j+1}
    // A segment is scaled when every alpha lies in [2^-6, 2^6]: G and 1/G stay
    // within 2^+-96, and nothing divides by a gate but dalpha's final 1/alpha.
    const bool bad = ga && !(rab >= 0x1p-6f && rab <= 0x1p6f);
    const bool sc = __ballot(bad) == 0;
    {
        const int j = tx >> 4, c4 = tx & 15;
        const float aj = __shfl(rab, j), bj = __shfl(rab, CK + j), gj = __shfl(pr, j);
        const float go = sc ? gj : 1.0f;
        const float gu = sc ? __builtin_amdgcn_rcpf(gj) : 1.0f;
        float4 x = st.rw[0];
        const float s0 = g * CK + j < T ? go : 0.0f;
        x = make_float4(x.x * s0, x.y * s0, x.z * s0, x.w * s0);
        const float4 vv = st.rw[1], sk = st.rw[2];
        const float4 wv = make_float4(fmaf(-aj, sk.x, vv.x), fmaf(-aj, sk.y, vv.y), fmaf(-aj, sk.z, vv.z),
                                      fmaf(-aj, sk.w, vv.w));
        const float bu = bj * gu;
        const int o = j * P + kpos(4 * c4);
        *reinterpret_cast<float4*>(nb + S_DO + o) = x;
        *reinterpret_cast<float4*>(nb + S_U + o) = make_float4(bu * wv.x, bu * wv.y, bu * wv.z, bu * wv.w);
        *reinterpret_cast<float4*>(nb + S_SK + o) = sk;
        *reinterpret_cast<float4*>(nb + S_WV + o) = wv;
    }
    // gate table: wave 0, lane j < CK writes alpha_j, G_{j+1}, 1/G_{j+1},
    // 1/alpha_j, |q_j| into row j; lane CK + j writes beta_j, |k_j|
    float* const sink = nb + S_SINK;
    const bool w0 = w == 0;
    float* const row = (w0 && (ga || gb)) ? nb + S_G + (lane & (CK - 1)) * 8 : sink;
    float* const rowa = (w0 && ga) ? row : sink;
    row[ga ? 0 : 1] = rab;
    row[ga ? 5 : 6] = rqk;
    rowa[2] = pr;
    rowa[3] = __builtin_amdgcn_rcpf(pr);
    rowa[4] = __builtin_amdgcn_rcpf(rab);
    *(w0 && lane == 0 ? nb + S_G + 8 * CK : sink + 3) = sc ? 1.0f : 0.0f;
}

// Operands of one step of the adjoint loop for this lane: rows rowb .. rowb + 7
// of q and k, and the lane's column pair (in k-order at kc) of dO, sk, v - alpha sk.
struct BOps {
    float q[BM], k[BM];
    float2 dO, sk, wv;
    float4 gt;   // alpha, beta, G_{j+1}, 1/G_{j+1}
};

ASCA_DEV void bops_read(BOps& o, const float* __restrict__ buf, int j, int rowb, int kc) {
    const float* const qr = buf + S_Q + j * P + rpad(rowb);
    const float* const kr = buf + S_K + j * P + rpad(rowb);
#pragma unroll
    for (int e = 0; e < BM; e += 4) {
        const float4 x = *reinterpret_cast<const float4*>(qr + e);
        const float4 y = *reinterpret_cast<const float4*>(kr + e);
        o.q[e] = x.x; o.q[e + 1] = x.y; o.q[e + 2] = x.z; o.q[e + 3] = x.w;
        o.k[e] = y.x; o.k[e + 1] = y.y; o.k[e + 2] = y.z; o.k[e + 3] = y.w;
    }
    o.dO = *reinterpret_cast<const float2*>(buf + S_DO + j * P + kc);
    o.sk = *reinterpret_cast<const float2*>(buf + S_SK + j * P + kc);
    o.wv = *reinterpret_cast<const float2*>(buf + S_WV + j * P + kc);
    o.gt = *reinterpret_cast<const float4*>(buf + S_G + 8 * j);
}

// Column sums over the eight column groups of a wave (lane bits 3..5) of the
// eight row partials p[m] (row rowb + m), transposed so that lane l ends with
// the whole sum of row 8 (l & 7) + (l >> 3).
ASCA_DEV float colsum8(const float (&p)[BM], int lane) {
    const float y0 = tsum32(p[0], p[4]), y1 = tsum32(p[1], p[5]);
    const float y2 = tsum32(p[2], p[6]), y3 = tsum32(p[3], p[7]);
    const float z0 = tsum16(y0, y2), z1 = tsum16(y1, y3);
    const bool b3 = (lane & 8) != 0;
    const float keep = b3 ? z1 : z0, send = b3 ? z0 : z1;
    return keep + dpp<DPP_ROW_ROR8>(send);
}

// du of a step for the lane's column pair: every lane of a column group holds
// the same du and G_j dsk, so every lane writes, the even row groups du and
// (with DSK) the odd ones G_j dsk; duplicates store identical values, and no
// lane mask is set up around the store.
template <bool DSK>
ASCA_DEV void put_du(float* __restrict__ dub, float* __restrict__ dskb, int j, int kc, int rg, float du0, float du1,
                     float sh0, float sh1) {
    const bool odd = DSK && (rg & 1);
    *reinterpret_cast<float2*>((odd ? dskb : dub) + j * P + kc) = odd ? make_float2(sh0, sh1) : make_float2(du0, du1);
}

// One step of the scaled adjoint loop (rust/src/delta.rs:508-563 for the
// adjoint only).  ds = G_{j+1} dS_j with dS_j excluding q_j dO_j^T on entry:
//   ds += q_j (G_{j+1} dO_j)^T;  t = ds^T k_j = G_{j+1} du_j;
//   G_j dsk_j = -beta_j t;        ds += k_j (G_j dsk_j)^T  (= G_j dS_{j-1} part).
// AB: returns the lane's transposed (ea, eb) pair of the step: ea = -beta
// du.sk, eb = du.(v - alpha sk) over the lane's columns (row group 0 only),
// and every lane stores du (even row groups) or G_j dsk (odd ones).  Without
// AB (the pipelined backward, whose matrix waves form these step sums from the
// du rows), nothing is returned and every lane stores both rows.
template <bool AB>
ASCA_DEV float bstep_sc(const BOps& in, float (&ds)[BM][2], float* __restrict__ dub, float* __restrict__ dskb, int j,
                        int kc, int rg) {
#pragma unroll
    for (int m = 0; m < BM; ++m) {
        ds[m][0] = fmaf(in.q[m], in.dO.x, ds[m][0]);
        ds[m][1] = fmaf(in.q[m], in.dO.y, ds[m][1]);
    }
    float c0 = 0.0f, c1 = 0.0f;
#pragma unroll
    for (int m = 0; m < BM; ++m) {
        c0 = fmaf(ds[m][0], in.k[m], c0);
        c1 = fmaf(ds[m][1], in.k[m], c1);
    }
    const float t0 = group_sum<8>(c0), t1 = group_sum<8>(c1);
    const float du0 = t0 * in.gt.w, du1 = t1 * in.gt.w;
    const float sh0 = -in.gt.y * t0, sh1 = -in.gt.y * t1;
    if constexpr (AB) {
        put_du<true>(dub, dskb, j, kc, rg, du0, du1, sh0, sh1);
    } else {
        *reinterpret_cast<float2*>(dub + j * P + kc) = make_float2(du0, du1);
        *reinterpret_cast<float2*>(dskb + j * P + kc) = make_float2(sh0, sh1);
    }
#pragma unroll
    for (int m = 0; m < BM; ++m) {
        ds[m][0] = fmaf(in.k[m], sh0, ds[m][0]);
        ds[m][1] = fmaf(in.k[m], sh1, ds[m][1]);
    }
    if constexpr (AB) {
        const float ea = rg == 0 ? -in.gt.y * fmaf(du1, in.sk.y, du0 * in.sk.x) : 0.0f;
        const float eb = rg == 0 ? fmaf(du1, in.wv.y, du0 * in.wv.x) : 0.0f;
        return tsum32(ea, eb);
    } else {
        return 0.0f;
    }
}

// One scaled segment (every alpha in [2^-6, 2^6]).  With G_j the product of the
// segment's alpha before step j, S the state before the segment, u~_j = u_j /
// G_{j+1}, dO~_j = G_{j+1} dO_j, dsk~_j = G_j dsk_j and X~ the scaled adjoint
// entering at the top, every output of the segment is a sum of 16-row matrix
// products (rows j):
//   dq = dO~ S^T + (M_le o P^T) K
//   dk = dsk~ S^T + U~ X~^T + (M_ge o P) Q + (lower(R^T) + upper(R)) K
// with P = U~ dO~^T and R = U~ dsk~^T (strict lower / upper parts), and
//   dalpha_j = br_j / alpha_j - beta_j du_j.sk_j,
//   br_j = <dS_out, S> - dsk_0.sk_0 + sum_{l<j} (u_l.du_l - q_l.dq_l - dsk_{l+1}.sk_{l+1}),
// the scaled <dS_j, S_{j-1}> carried from the exact product at the bottom.  Only
// the adjoint recurrence runs step by step (on the VALU); the products run on
// the matrix cores after it.  Wave w computes the dq / dk columns 16 w .. 16 w
// + 15 of every step; the products over the columns (P, R) are summed from
// per-wave partials.
ASCA_DEV void bsegment_sc(float (&ds)[BM][2], const BStage& stg, int g, int T, const float* __restrict__ buf,
                          float* __restrict__ nb, float* __restrict__ wk, int w, int lane, int rg, int cg,
                          int rowb, int kc) {
    const int jr = lane & 15, gq = lane >> 4;
    float pab[CK];
    BOps op[2];
    bops_read(op[(CK - 1) & 1], buf, CK - 1, rowb, kc);
#pragma unroll
    for (int jj = CK - 1; jj >= 0; --jj) {
        // the operand reads of the next step are issued a whole step ahead
        if (jj > 0) bops_read(op[(jj - 1) & 1], buf, jj - 1, rowb, kc);
        pab[jj] = bstep_sc<true>(op[jj & 1], ds, wk + W_DU, wk + W_DSK, jj, kc, rg);
        if (jj == CK / 2) {
            // the staged operands of the next segment (loads issued at this
            // segment's start) go to its buffer; the fence keeps the scheduler
            // from hoisting the stores, and their wait, to the segment's start
            __builtin_amdgcn_sched_barrier(0);
            bstage_store(stg, g > 0 ? g - 1 : 0, T, nb, threadIdx.x, w, lane);
        }
    }
    // products of inputs alone: dO~ S^T, U~ X~^T and the partial P
    f32x4 adq = {0.f, 0.f, 0.f, 0.f}, adk = adq, ap = adq;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float4 x = *reinterpret_cast<const float4*>(buf + S_DO + jr * P + 16 * gq + 4 * e);
        const float4 y = *reinterpret_cast<const float4*>(buf + S_U + jr * P + 16 * gq + 4 * e);
        const float xs[4] = {x.x, x.y, x.z, x.w}, ys[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            adq = mfma4(xs[i], buf[S_M + kcol(gq, 4 * e + i) * P + 16 * w + jr], adq);
            adk = mfma4(ys[i], wk[W_XT + kcol(gq, 4 * e + i) * P + 16 * w + jr], adk);
        }
    }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
        ap = mfma4(buf[S_U + jr * P + 16 * kb + 4 * w + gq], buf[S_DO + jr * P + 16 * kb + 4 * w + gq], ap);
    // ds = dS_{-1} without q_{-1} dO_{-1}^T (G_0 = 1): its product with S
    {
        float x = 0.0f;
#pragma unroll
        for (int n = 0; n < 2; ++n)
#pragma unroll
            for (int e = 0; e < BM; e += 4) {
                const float4 s = *reinterpret_cast<const float4*>(buf + S_M + (16 * w + 2 * cg + n) * P + rowb + e);
                x = fmaf(ds[e][n], s.x, x);
                x = fmaf(ds[e + 1][n], s.y, x);
                x = fmaf(ds[e + 2][n], s.z, x);
                x = fmaf(ds[e + 3][n], s.w, x);
            }
        x = wave_sum(x);
        if (lane == 0) wk[W_BR + w] = x;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) wk[W_PP + (w * CK + 4 * gq + r) * 17 + jr] = ap[r];
    cross_step_sum<CK, W>(pab, wk + W_AB, w, lane);
    lds_barrier();   // dsk~, du, the partial P and the step sums of every wave

    // products with dsk~: dsk~ S^T and the partial R
    {
        float r_u[4], r_d[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            r_u[kb] = buf[S_U + jr * P + 16 * kb + 4 * w + gq];
            r_d[kb] = wk[W_DSK + jr * P + 16 * kb + 4 * w + gq];
        }
        f32x4 ar = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) ar = mfma4(r_u[kb], r_d[kb], ar);
#pragma unroll
        for (int r = 0; r < 4; ++r) wk[W_RP + (w * CK + 4 * gq + r) * 17 + jr] = ar[r];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float4 x = *reinterpret_cast<const float4*>(wk + W_DSK + jr * P + 16 * gq + 4 * e);
            adk = mfma4(x.x, buf[S_M + kcol(gq, 4 * e) * P + 16 * w + jr], adk);
            adk = mfma4(x.y, buf[S_M + kcol(gq, 4 * e + 1) * P + 16 * w + jr], adk);
            adk = mfma4(x.z, buf[S_M + kcol(gq, 4 * e + 2) * P + 16 * w + jr], adk);
            adk = mfma4(x.w, buf[S_M + kcol(gq, 4 * e + 3) * P + 16 * w + jr], adk);
        }
    }
    lds_barrier();   // every wave's partial R

    // the 16 x 16 step mixes: k = 4 kb + gq, row j = jr
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        const int kk = 4 * kb + gq;
        float pkj = 0.0f, pjk = 0.0f, rkj = 0.0f, rjk = 0.0f;
#pragma unroll
        for (int u4 = 0; u4 < W; ++u4) {
            pkj += wk[W_PP + (u4 * CK + kk) * 17 + jr];
            pjk += wk[W_PP + (u4 * CK + jr) * 17 + kk];
            rkj += wk[W_RP + (u4 * CK + kk) * 17 + jr];
            rjk += wk[W_RP + (u4 * CK + jr) * 17 + kk];
        }
        const float bk = buf[S_K + kk * P + rpad(16 * w + jr)];
        const float bq = buf[S_Q + kk * P + rpad(16 * w + jr)];
        adq = mfma4(kk <= jr ? pkj : 0.0f, bk, adq);
        adk = mfma4(kk >= jr ? pjk : 0.0f, bq, adk);
        adk = mfma4(kk < jr ? rkj : (kk > jr ? rjk : 0.0f), bk, adk);
    }
    // dq, dk rows and the partial q . dq, k . dk of the wave's columns
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int j = 4 * gq + r;
        wk[W_DQ + j * P + 16 * w + jr] = adq[r];
        wk[W_DK + j * P + 16 * w + jr] = adk[r];
        const float x = group_sum<16>(adq[r] * buf[S_Q + j * P + rpad(16 * w + jr)]);
        const float y = group_sum<16>(adk[r] * buf[S_K + j * P + rpad(16 * w + jr)]);
        if (jr == 0) {
            wk[W_QDQ + w * CK + j] = x;
            wk[W_KDK + w * CK + j] = y;
        }
    }
}

// Plain forms for a segment with some gate outside [2^-6, 2^6] (zeros, tiny or
// huge values): every state the steps need is recomputed forwards from the
// segment's first checkpoint, so no gate is ever divided by.
ASCA_DEV void fwd_update(float (&x)[BM][2], const float* __restrict__ buf, int j, int rowb, int kc) {
    const float* const kr = buf + S_K + j * P + rpad(rowb);
    const float2 u = *reinterpret_cast<const float2*>(buf + S_U + j * P + kc);
    const float a = buf[S_G + 8 * j];
#pragma unroll
    for (int e = 0; e < BM; e += 4) {
        const float4 kk = *reinterpret_cast<const float4*>(kr + e);
        const float km[4] = {kk.x, kk.y, kk.z, kk.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[e + i][0] = a * x[e + i][0] + km[i] * u.x;
            x[e + i][1] = a * x[e + i][1] + km[i] * u.y;
        }
    }
}

// One plain reverse step for this lane's 8 x 2 tile (rust/src/delta.rs:485-572
// per element); s = S_j, sm = S_{j-1}, ds = dS_j without q_j dO_j^T on entry.
// Writes the wave's dq / dk row partials and du; returns the lane's transposed
// (dalpha, dbeta) pair partial.
ASCA_DEV float bstep_plain(const BOps& in, const float (&s)[BM][2], const float (&sm)[BM][2], float (&ds)[BM][2],
                           const float2 u, float* __restrict__ wk, int j, int w, int lane, int rg, int kc) {
    const float a = in.gt.x, b = in.gt.y;
    float pq[BM], pk[BM];
#pragma unroll
    for (int m = 0; m < BM; ++m) {
        pq[m] = fmaf(s[m][1], in.dO.y, s[m][0] * in.dO.x);
        ds[m][0] = fmaf(in.q[m], in.dO.x, ds[m][0]);
        ds[m][1] = fmaf(in.q[m], in.dO.y, ds[m][1]);
    }
    float c0 = 0.0f, c1 = 0.0f;
#pragma unroll
    for (int m = 0; m < BM; ++m) {
        c0 = fmaf(ds[m][0], in.k[m], c0);
        c1 = fmaf(ds[m][1], in.k[m], c1);
    }
    const float du0 = group_sum<8>(c0), du1 = group_sum<8>(c1);
    const float dk0 = -a * b * du0, dk1 = -a * b * du1;
    put_du<false>(wk + W_DU, wk + W_DSK, j, kc, rg, du0, du1, 0.0f, 0.0f);
    float pa0 = 0.0f, pa1 = 0.0f;
#pragma unroll
    for (int m = 0; m < BM; ++m) {
        float x = u.x * ds[m][0];
        x = fmaf(u.y, ds[m][1], x);
        x = fmaf(dk0, sm[m][0], x);
        pk[m] = fmaf(dk1, sm[m][1], x);
        pa0 = fmaf(ds[m][0], sm[m][0], pa0);
        pa1 = fmaf(ds[m][1], sm[m][1], pa1);
        ds[m][0] = a * ds[m][0] + in.k[m] * dk0;
        ds[m][1] = a * ds[m][1] + in.k[m] * dk1;
    }
    const float ea = -b * fmaf(du1, in.sk.y, du0 * in.sk.x);
    const float eb = fmaf(du1, in.wv.y, du0 * in.wv.x);
    const int r = rpad(8 * (lane & 7) + (lane >> 3));
    wk[W_RQ + (j * W + w) * P + r] = colsum8(pq, lane);
    wk[W_RK + (j * W + w) * P + r] = colsum8(pk, lane);
    return tsum32(pa0 + pa1 + (rg == 0 ? ea : 0.0f), rg == 0 ? eb : 0.0f);
}

// A plain segment in reverse: a rolled loop, since these segments are rare and
// their registers must not raise the kernel's budget.
ASCA_DEV void bsegment_plain(float (&ds)[BM][2], const BStage& stg, int g, int T, const float* __restrict__ buf,
                             float* __restrict__ nb, float* __restrict__ wk, int w, int lane, int rg, int cg,
                             int rowb, int kc) {
    float st0[BM][2];
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int e = 0; e < BM; e += 4) {
            const float4 x = *reinterpret_cast<const float4*>(buf + S_M + (16 * w + 2 * cg + n) * P + rowb + e);
            st0[e][n] = x.x; st0[e + 1][n] = x.y; st0[e + 2][n] = x.z; st0[e + 3][n] = x.w;
        }
#pragma nounroll
    for (int jj = CK - 1; jj >= 0; --jj) {
        float sm[BM][2], s[BM][2];
#pragma unroll
        for (int m = 0; m < BM; ++m) {
            sm[m][0] = st0[m][0];
            sm[m][1] = st0[m][1];
        }
#pragma nounroll
        for (int i = 0; i < jj; ++i) fwd_update(sm, buf, i, rowb, kc);
#pragma unroll
        for (int m = 0; m < BM; ++m) {
            s[m][0] = sm[m][0];
            s[m][1] = sm[m][1];
        }
        fwd_update(s, buf, jj, rowb, kc);
        BOps op;
        bops_read(op, buf, jj, rowb, kc);
        const float2 u = *reinterpret_cast<const float2*>(buf + S_U + jj * P + kc);
        const float pab = bstep_plain(op, s, sm, ds, u, wk, jj, w, lane, rg, kc);
        // lanes < 32 hold dalpha pair sums, lanes >= 32 dbeta ones
        const float tot = add_xor16(group_sum<16>(pab));
        if ((lane & 31) == 0) wk[W_AB + (jj * W + w) * 2 + (lane >> 5)] = tot;
    }
    // after the loop, not inside it under a condition: every path then provably
    // waits for the staged loads here, and no later reuse of their registers does
    bstage_store(stg, g > 0 ? g - 1 : 0, T, nb, threadIdx.x, w, lane);
}

// Arguments shared by the backward's paths.
struct BArgs {
    const float* q; const float* k; const float* v; const float* alpha; const float* beta; const float* d_o;
    const float* skv; const float* qnorm; const float* knorm;
    float* gq; float* gk; float* gv; float* ga; float* gb;
    const float* ckb;
    long ldx, ldg, d, ubase, gbase, hoff;
    int b, h, T, H, nseg;
};

// The serial path, on waves 0..3: each segment's products, sums and
// epilogue follow its adjoint loop on the same waves.  Taken by every unit
// that has a plain segment; waves 4..7 meanwhile only mirror its barriers
// (bwd_mirror).
template <bool FUSED, bool AL>
ASCA_DEV void bwd_serial(const BArgs& A, float* __restrict__ lds, int w, int lane) {
    const float *q = A.q, *k = A.k, *v = A.v, *alpha = A.alpha, *beta = A.beta, *d_o = A.d_o, *skv = A.skv;
    const float *qnorm = A.qnorm, *knorm = A.knorm, *ckb = A.ckb;
    float *gq = A.gq, *gk = A.gk, *gv = A.gv, *ga = A.ga, *gb = A.gb;
    const long ldx = A.ldx, ldg = A.ldg, d = A.d, ubase = A.ubase, gbase = A.gbase, hoff = A.hoff;
    const int b = A.b, h = A.h, T = A.T, H = A.H, nseg = A.nseg;
    float* const wk = lds + 2 * S_BUF;
    const int rg = lane & 7, cg = lane >> 3;
    const int rowb = BM * rg;
    const int kc = kpos(16 * w + 2 * cg);

    float ds[BM][2];
#pragma unroll
    for (int m = 0; m < BM; ++m) ds[m][0] = ds[m][1] = 0.0f;

    BStage stg;
    bstage_load<FUSED, AL>(stg, nseg - 1, q, k, v, d_o, skv, alpha, beta, qnorm, knorm, ckb, ubase, gbase, d, T, H,
                           threadIdx.x, lane);
    bstage_store(stg, nseg - 1, T, lds + ((nseg - 1) & 1) * S_BUF, threadIdx.x, w, lane);
    lds_barrier();

    for (int g = nseg - 1; g >= 0; --g) {
        const int t0 = g * CK;
        float* const buf = lds + (g & 1) * S_BUF;
        float* const nb = lds + ((g + 1) & 1) * S_BUF;   // the next segment's (g - 1)
        const bool sc = __builtin_amdgcn_readfirstlane(__float_as_int(buf[S_G + 8 * CK])) == __float_as_int(1.0f);
        if (sc) {
            // the adjoint entering the segment, scaled by its G_CK, as X~^T
            const float gend = buf[S_G + 8 * (CK - 1) + 2];
#pragma unroll
            for (int n = 0; n < 2; ++n) {
#pragma unroll
                for (int m = 0; m < BM; ++m) ds[m][n] *= gend;
#pragma unroll
                for (int e = 0; e < BM; e += 4)
                    *reinterpret_cast<float4*>(wk + W_XT + (16 * w + 2 * cg + n) * P + rowb + e) =
                        make_float4(ds[e][n], ds[e + 1][n], ds[e + 2][n], ds[e + 3][n]);
            }
        }
        bstage_load<FUSED, AL>(stg, g > 0 ? g - 1 : 0, q, k, v, d_o, skv, alpha, beta, qnorm, knorm, ckb, ubase,
                               gbase, d, T, H, threadIdx.x, lane);
        lds_barrier();   // X~^T of every wave

        if (sc)
            bsegment_sc(ds, stg, g, T, buf, nb, wk, w, lane, rg, cg, rowb, kc);
        else
            bsegment_plain(ds, stg, g, T, buf, nb, wk, w, lane, rg, cg, rowb, kc);
        lds_barrier();   // dq, dk rows, the step sums

        // Per-step scalars, lane l of every 16-lane row carrying step l: the
        // totals of the per-wave step sums (scaled segment: ea = -beta du.sk,
        // eb = du.(v - alpha sk), q.dq, k.dk; plain: dalpha, dbeta) and, for a
        // scaled segment, dalpha's bracket br_l (an exclusive prefix over the
        // per-step dot products).  Each wave then reads its steps' values by
        // readlane instead of from LDS.
        const int l = lane & (CK - 1);
        float ea = 0.0f, eb = 0.0f, qdq = 0.0f, kdk = 0.0f;
#pragma unroll
        for (int u4 = 0; u4 < W; ++u4) {
            ea += wk[W_AB + (l * W + u4) * 2];
            eb += wk[W_AB + (l * W + u4) * 2 + 1];
        }
        const float4 gl0 = *reinterpret_cast<const float4*>(buf + S_G + 8 * l);       // alpha, beta, G, 1/G
        const float4 gl1 = *reinterpret_cast<const float4*>(buf + S_G + 8 * l + 4);   // 1/alpha, |q|, |k|, -
        float dal = ea;
        if (sc) {
            float bsum = 0.0f;
#pragma unroll
            for (int u4 = 0; u4 < W; ++u4) {
                qdq += wk[W_QDQ + u4 * CK + l];
                kdk += wk[W_KDK + u4 * CK + l];
                bsum += wk[W_BR + u4];
            }
            const float ea1 = dpp_or<0x101>(0.0f, ea);       // row_shl 1: step l + 1
            const float al1 = dpp_or<0x101>(1.0f, gl0.x);
            const float term = l + 1 < CK ? gl0.y * eb - qdq - al1 * ea1 : 0.0f;
            float x = term;   // inclusive prefix sum over the 16 lanes of each row
            x += dpp_or<0x111>(0.0f, x);
            x += dpp_or<0x112>(0.0f, x);
            x += dpp_or<0x114>(0.0f, x);
            x += dpp_or<0x118>(0.0f, x);
            const float br = bsum - readlane_f(gl0.x, 0) * readlane_f(ea, 0) + (x - term);
            dal = fmaf(br, gl1.x, ea);   // dalpha_l = br_l / alpha_l - beta_l du_l.sk_l
        }

        // fused norm / sigmoid backward and stores: wave w takes steps w + W i,
        // lane = row.  Every LDS read of the wave's steps is issued before the
        // arithmetic and the stores (steps past T only skip their stores).
        constexpr int NS = CK / W;
        const int a = lane;
        const int ws = __builtin_amdgcn_readfirstlane(w);
        float dq[NS], dk[NS], du[NS], qa[NS], ka[NS];
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            const int jj = ws + W * i;
            if (sc) {
                dq[i] = wk[W_DQ + jj * P + a];
                dk[i] = wk[W_DK + jj * P + a];
            } else {
                const float* const rq = wk + W_RQ + jj * W * P + rpad(a);
                const float* const rk = wk + W_RK + jj * W * P + rpad(a);
                dq[i] = (rq[0] + rq[P]) + (rq[2 * P] + rq[3 * P]);
                dk[i] = (rk[0] + rk[P]) + (rk[2 * P] + rk[3 * P]);
            }
            du[i] = wk[W_DU + jj * P + kpos(a)];
            qa[i] = buf[S_Q + jj * P + rpad(a)];
            ka[i] = buf[S_K + jj * P + rpad(a)];
        }
        static_assert(W == 4, "the step sums above add four waves");
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            const int jj = ws + W * i;
            if (t0 + jj >= T) continue;   // wave-uniform
            const float dA = readlane_f(dal, jj), dB = readlane_f(eb, jj);
            const float al = readlane_f(gl0.x, jj), be = readlane_f(gl0.y, jj);
            const long r = (long)b * T + t0 + jj;
            gv[r * ldx + hoff + a] = be * du[i];
            if constexpr (FUSED) {
                const float dotq = sc ? readlane_f(qdq, jj) : wave_sum(qa[i] * dq[i]);
                const float dotk = sc ? readlane_f(kdk, jj) : wave_sum(ka[i] * dk[i]);
                // 1/|q|, 1/|k| by the hardware reciprocal (within 1 ulp)
                const float rq = __builtin_amdgcn_rcpf(readlane_f(gl1.y, jj));
                const float rk = __builtin_amdgcn_rcpf(readlane_f(gl1.z, jj));
                gq[r * ldx + hoff + a] = (dq[i] - qa[i] * dotq) * rq;
                gk[r * ldx + hoff + a] = (dk[i] - ka[i] * dotk) * rk;
                if (lane == 0) {
                    ga[r * ldg + h] = dA * al * (1.0f - al);
                    gb[r * ldg + h] = dB * be * (1.0f - be);
                }
            } else {
                gq[r * ldx + hoff + a] = dq[i];
                gk[r * ldx + hoff + a] = dk[i];
                if (lane == 0) {
                    ga[r * ldg + h] = dA;
                    gb[r * ldg + h] = dB;
                }
            }
        }
        // a plain segment's row partials share space with the next segment's X~^T
        if (!sc) lds_barrier();
    }
}


// Barriers of bwd_serial, for the waves that take no part in it.
ASCA_DEV void bwd_mirror(const float* __restrict__ lds, int nseg) {
    lds_barrier();
    for (int g = nseg - 1; g >= 0; --g) {
        lds_barrier();   // segment start
        const float* const buf = lds + (g & 1) * S_BUF;
        const bool sc = __builtin_amdgcn_readfirstlane(__float_as_int(buf[S_G + 8 * CK])) == __float_as_int(1.0f);
        if (sc) {
            lds_barrier();   // the scaled segment's two
            lds_barrier();
        }
        lds_barrier();   // rows and sums
        if (!sc) lds_barrier();
    }
}

// ------------------------------------------------- pipelined backward
// A unit whose segments are all scaled runs on eight waves as a two-stage
// pipeline: in period p, the adjoint waves (0..3) run the adjoint loop of
// segment g = nseg - 1 - p while the matrix waves (4..7) run the products and
// the epilogue of segment g + 1, whose loop ended in period p - 1, and stage
// segment g - 1.  One adjoint wave and one matrix wave share each SIMD, so
// the matrix waves' MFMA and LDS latencies fill the adjoint loop's stalls.
// Two block barriers per period: P0 at its start, P1 halfway through the
// loop, which the matrix waves reach once they no longer read the staging
// buffer of g + 1, so that they may restage it with g - 1.  Data the stages
// hand over (the top adjoint X~, du, dsk~, step sums) alternate between two
// slots by segment parity.
constexpr int Q_STG = 0;                          // [2][S_BUF] staging
constexpr int Q_XT = 2 * S_BUF;                   // [2][DH][P] X~^T
constexpr int Q_DU = Q_XT + 2 * DH * P;           // [2][CK][P] du, k-order
constexpr int Q_DSK = Q_DU + 2 * CK * P;          // [2][CK][P] G_j dsk_j, k-order
constexpr int Q_DQ = Q_DSK + 2 * CK * P;          // [CK][P] dq rows
constexpr int Q_DK = Q_DQ + CK * P;               // [CK][P] dk rows
constexpr int Q_PR = Q_DK + CK * P;               // [W][2][CK][17] each matrix wave's P and R
constexpr int Q_AB = Q_PR + W * 2 * CK * 17;      // [2][CK][W][2] step sums
constexpr int Q_QDQ = Q_AB + 2 * CK * W * 2;      // [W][CK] per-wave partial q . dq
constexpr int Q_KDK = Q_QDQ + W * CK;             // [W][CK] per-wave partial k . dk
constexpr int Q_BR = Q_KDK + W * CK;              // [2][8] per-wave partial <dS, S>
constexpr int Q_D0 = Q_BR + 16;                   // [CK][DH] dO~ S^T from the adjoint waves
constexpr int Q_END = Q_D0 + CK * DH;
static_assert(Q_DU % 4 == 0 && Q_DQ % 4 == 0 && Q_AB % 4 == 0, "16-byte rows");
constexpr size_t B_LDS_ALL = (size_t)(Q_END > 2 * S_BUF + W_END ? Q_END : 2 * S_BUF + W_END) * 4;
static_assert(B_LDS_ALL <= 160 * 1024, "backward LDS");

// Adjoint waves: the loop of one scaled segment (as in bsegment_sc, without
// the products and the step sums), with P1 between steps CK/2 and CK/2 - 1;
// then the anchor <dS_out, S>.
ASCA_DEV void aloop(float (&ds)[BM][2], const float* __restrict__ buf, float* __restrict__ dub,
                    float* __restrict__ dskb, float* __restrict__ brb, int w, int lane, int rg, int cg, int rowb,
                    int kc) {
    BOps op[2];
    bops_read(op[(CK - 1) & 1], buf, CK - 1, rowb, kc);
#pragma unroll
    for (int jj = CK - 1; jj >= 0; --jj) {
        if (jj > 0) bops_read(op[(jj - 1) & 1], buf, jj - 1, rowb, kc);
        bstep_sc<false>(op[jj & 1], ds, dub, dskb, jj, kc, rg);
        if (jj == CK / 2) lds_barrier();   // P1
    }
    float x = 0.0f;
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int e = 0; e < BM; e += 4) {
            const float4 s = *reinterpret_cast<const float4*>(buf + S_M + (16 * w + 2 * cg + n) * P + rowb + e);
            x = fmaf(ds[e][n], s.x, x);
            x = fmaf(ds[e + 1][n], s.y, x);
            x = fmaf(ds[e + 2][n], s.z, x);
            x = fmaf(ds[e + 3][n], s.w, x);
        }
    x = wave_sum(x);
    if (lane == 0) brb[w] = x;
}

// Adjoint wave w, after the loop of a segment: the part dO~ S^T of its dq
// columns 16 w .. 16 w + 15 (a product of staged inputs only), computed as
// mprod would, into d0, where matrix wave w starts its dq sums from it a
// period later; the adjoint waves have this time to spare before the next
// period while the matrix waves run the epilogue.
ASCA_DEV void adj_dq(const float* __restrict__ buf, float* __restrict__ d0, int w, int lane) {
    const int jr = lane & 15, gq = lane >> 4;
    float a_do[16], b_s[16];
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
        const float4 x = *reinterpret_cast<const float4*>(buf + S_DO + jr * P + 16 * gq + 4 * e4);
        a_do[4 * e4] = x.x; a_do[4 * e4 + 1] = x.y; a_do[4 * e4 + 2] = x.z; a_do[4 * e4 + 3] = x.w;
    }
#pragma unroll
    for (int kb = 0; kb < 16; ++kb) b_s[kb] = buf[S_M + kcol(gq, kb) * P + 16 * w + jr];
    f32x4 adq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 16; ++kb) adq = mfma4(a_do[kb], b_s[kb], adq);
#pragma unroll
    for (int r = 0; r < 4; ++r) d0[(4 * gq + r) * DH + 16 * w + jr] = adq[r];
}

// What a matrix wave keeps of a segment's staging buffer for its epilogue.
struct MEpi {
    float qa[CK / W], ka[CK / W];   // q, k of the wave's steps, lane = row
    float4 gl0, gl1;                // lane l < CK: step l's gate row
};

// Matrix wave mw: the products of one segment (bsegment_sc's formulas) for the
// dq / dk columns 16 mw .. 16 mw + 15 of every step, with P and R in full
// (each wave its own, through a private LDS area), the rows and the partial
// q . dq, k . dk; then what the epilogue needs from the staging buffer.
ASCA_DEV void mprod(const float* __restrict__ buf, const float* __restrict__ xt, const float* __restrict__ dsk,
                    const float* __restrict__ dub, float* __restrict__ abb, float* __restrict__ lds, int mw,
                    int lane, MEpi& e) {
    // dq starts from dO~ S^T (adj_dq, the adjoint waves' product)
    const int jr = lane & 15, gq = lane >> 4;
    float a_do[16], a_u[16], a_dk[16], b_s[16], b_x[16];
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
        const float4 x = *reinterpret_cast<const float4*>(buf + S_DO + jr * P + 16 * gq + 4 * e4);
        const float4 y = *reinterpret_cast<const float4*>(buf + S_U + jr * P + 16 * gq + 4 * e4);
        const float4 z = *reinterpret_cast<const float4*>(dsk + jr * P + 16 * gq + 4 * e4);
        a_do[4 * e4] = x.x; a_do[4 * e4 + 1] = x.y; a_do[4 * e4 + 2] = x.z; a_do[4 * e4 + 3] = x.w;
        a_u[4 * e4] = y.x; a_u[4 * e4 + 1] = y.y; a_u[4 * e4 + 2] = y.z; a_u[4 * e4 + 3] = y.w;
        a_dk[4 * e4] = z.x; a_dk[4 * e4 + 1] = z.y; a_dk[4 * e4 + 2] = z.z; a_dk[4 * e4 + 3] = z.w;
    }
#pragma unroll
    for (int kb = 0; kb < 16; ++kb) {
        b_s[kb] = buf[S_M + kcol(gq, kb) * P + 16 * mw + jr];
        b_x[kb] = xt[kcol(gq, kb) * P + 16 * mw + jr];
    }
    f32x4 adk = {0.f, 0.f, 0.f, 0.f}, ap = adk, ar = adk, adq;
#pragma unroll
    for (int r = 0; r < 4; ++r) adq[r] = lds[Q_D0 + (4 * gq + r) * DH + 16 * mw + jr];
#pragma unroll
    for (int kb = 0; kb < 16; ++kb) {
        adk = mfma4(a_u[kb], b_x[kb], adk);
        adk = mfma4(a_dk[kb], b_s[kb], adk);
        ap = mfma4(a_u[kb], a_do[kb], ap);
        ar = mfma4(a_u[kb], a_dk[kb], ar);
    }
    float* const prv = lds + Q_PR + mw * 2 * CK * 17;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        prv[(4 * gq + r) * 17 + jr] = ap[r];
        prv[CK * 17 + (4 * gq + r) * 17 + jr] = ar[r];
    }
    // the wave reads back what its own lanes wrote
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        const int kk = 4 * kb + gq;
        const float pkj = prv[kk * 17 + jr], pjk = prv[jr * 17 + kk];
        const float rkj = prv[CK * 17 + kk * 17 + jr], rjk = prv[CK * 17 + jr * 17 + kk];
        const float bk = buf[S_K + kk * P + rpad(16 * mw + jr)];
        const float bq = buf[S_Q + kk * P + rpad(16 * mw + jr)];
        adq = mfma4(kk <= jr ? pkj : 0.0f, bk, adq);
        adk = mfma4(kk >= jr ? pjk : 0.0f, bq, adk);
        adk = mfma4(kk < jr ? rkj : (kk > jr ? rjk : 0.0f), bk, adk);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int j = 4 * gq + r;
        lds[Q_DQ + j * P + 16 * mw + jr] = adq[r];
        lds[Q_DK + j * P + 16 * mw + jr] = adk[r];
        const float x = group_sum<16>(adq[r] * buf[S_Q + j * P + rpad(16 * mw + jr)]);
        const float y = group_sum<16>(adk[r] * buf[S_K + j * P + rpad(16 * mw + jr)]);
        if (jr == 0) {
            lds[Q_QDQ + mw * CK + j] = x;
            lds[Q_KDK + mw * CK + j] = y;
        }
    }
#pragma unroll
    for (int i = 0; i < CK / W; ++i) {
        e.qa[i] = buf[S_Q + (mw + W * i) * P + rpad(lane)];
        e.ka[i] = buf[S_K + (mw + W * i) * P + rpad(lane)];
    }
    e.gl0 = *reinterpret_cast<const float4*>(buf + S_G + 8 * (lane & (CK - 1)));
    e.gl1 = *reinterpret_cast<const float4*>(buf + S_G + 8 * (lane & (CK - 1)) + 4);
    {
        // the step sums of dalpha / dbeta over the k-order positions 16 mw ..
        // 16 mw + 15 (lane: step jr, positions 16 mw + 4 gq .. + 3):
        // ea_j = -beta_j du_j . sk_j, eb_j = du_j . (v_j - alpha_j sk_j)
        const int c0 = 16 * mw + 4 * gq;
        const float4 u = *reinterpret_cast<const float4*>(dub + jr * P + c0);
        const float4 a = *reinterpret_cast<const float4*>(buf + S_SK + jr * P + c0);
        const float4 b = *reinterpret_cast<const float4*>(buf + S_WV + jr * P + c0);
        float ea = u.x * a.x, eb = u.x * b.x;
        ea = fmaf(u.y, a.y, ea);
        eb = fmaf(u.y, b.y, eb);
        ea = fmaf(u.z, a.z, ea);
        eb = fmaf(u.z, b.z, eb);
        ea = fmaf(u.w, a.w, ea);
        eb = fmaf(u.w, b.w, eb);
        ea = add_xor32(add_xor16(ea));
        eb = add_xor32(add_xor16(eb));
        if (gq == 0) *reinterpret_cast<float2*>(abb + (jr * W + mw) * 2) = make_float2(-buf[S_G + 8 * jr + 1] * ea, eb);
    }
}

// Matrix wave mw: dalpha's bracket and the epilogue of segment gp (as in
// bwd_serial's), steps mw + W i.
template <bool FUSED>
ASCA_DEV void mepi(const BArgs& A, const MEpi& e, float* __restrict__ lds, const float* __restrict__ abb,
                   const float* __restrict__ brb, const float* __restrict__ dub, int gp, int mw, int lane) {
    const int l = lane & (CK - 1);
    float ea = 0.0f, eb = 0.0f, qdq = 0.0f, kdk = 0.0f, bsum = 0.0f;
#pragma unroll
    for (int u4 = 0; u4 < W; ++u4) {
        ea += abb[(l * W + u4) * 2];
        eb += abb[(l * W + u4) * 2 + 1];
        qdq += lds[Q_QDQ + u4 * CK + l];
        kdk += lds[Q_KDK + u4 * CK + l];
        bsum += brb[u4];
    }
    const float ea1 = dpp_or<0x101>(0.0f, ea);       // row_shl 1: step l + 1
    const float al1 = dpp_or<0x101>(1.0f, e.gl0.x);
    const float term = l + 1 < CK ? e.gl0.y * eb - qdq - al1 * ea1 : 0.0f;
    float x = term;   // inclusive prefix sum over the 16 lanes of each row
    x += dpp_or<0x111>(0.0f, x);
    x += dpp_or<0x112>(0.0f, x);
    x += dpp_or<0x114>(0.0f, x);
    x += dpp_or<0x118>(0.0f, x);
    const float br = bsum - readlane_f(e.gl0.x, 0) * readlane_f(ea, 0) + (x - term);
    const float dal = fmaf(br, e.gl1.x, ea);
    const int t0 = gp * CK;
    const int ws = __builtin_amdgcn_readfirstlane(mw);
    // the per-step factors of the row stores (lane l: step l) go through the
    // wave's own product scratch (free until the next period's products) and
    // come back as broadcast 16-byte reads: no v_readlane per stored row
    float* const fac = lds + Q_PR + mw * 2 * CK * 17;   // [CK][8]
    if (lane < CK) {
        if constexpr (FUSED)
            *reinterpret_cast<float4*>(fac + 8 * lane) =
                make_float4(e.gl0.y, qdq, __builtin_amdgcn_rcpf(e.gl1.y), kdk);
        else
            *reinterpret_cast<float4*>(fac + 8 * lane) = make_float4(e.gl0.y, 0.0f, 1.0f, 0.0f);
        fac[8 * lane + 4] = FUSED ? __builtin_amdgcn_rcpf(e.gl1.z) : 1.0f;
    }
    // dalpha and dbeta of every step of the segment from wave 0, lane l = step l
    if (ws == 0 && lane < CK && t0 + lane < A.T) {
        const long r = (long)A.b * A.T + t0 + lane;
        const float al = e.gl0.x, be = e.gl0.y;
        A.ga[r * A.ldg + A.h] = FUSED ? dal * al * (1.0f - al) : dal;
        A.gb[r * A.ldg + A.h] = FUSED ? eb * be * (1.0f - be) : eb;
    }
    float dq[CK / W], dk[CK / W], du[CK / W];
#pragma unroll
    for (int i = 0; i < CK / W; ++i) {
        const int jj = ws + W * i;
        dq[i] = lds[Q_DQ + jj * P + lane];
        dk[i] = lds[Q_DK + jj * P + lane];
        du[i] = dub[jj * P + kpos(lane)];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float4 c[CK / W];
    float rk[CK / W];
#pragma unroll
    for (int i = 0; i < CK / W; ++i) {
        const int jj = ws + W * i;
        c[i] = *reinterpret_cast<const float4*>(fac + 8 * jj);
        rk[i] = fac[8 * jj + 4];
    }
#pragma unroll
    for (int i = 0; i < CK / W; ++i) {
        const int jj = ws + W * i;
        if (t0 + jj >= A.T) continue;   // wave-uniform
        const long r = (long)A.b * A.T + t0 + jj;
        const long o = r * A.ldx + A.hoff + lane;
        A.gv[o] = c[i].x * du[i];
        if constexpr (FUSED) {
            A.gq[o] = (dq[i] - e.qa[i] * c[i].y) * c[i].z;
            A.gk[o] = (dk[i] - e.ka[i] * c[i].w) * rk[i];
        } else {
            A.gq[o] = dq[i];
            A.gk[o] = dk[i];
        }
    }
}

template <bool FUSED, bool AL>
__global__ __launch_bounds__(2 * NT) void delta_bwd64_k(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ alpha, const float* __restrict__ beta, const float* __restrict__ d_o,
    const float* __restrict__ skv, const float* __restrict__ ckpt, const float* __restrict__ qnorm,
    const float* __restrict__ knorm, float* __restrict__ gq, float* __restrict__ gk, float* __restrict__ gv,
    long ldx, float* __restrict__ ga, float* __restrict__ gb, long ldg, int B, int T, int H, int nslots) {
    extern __shared__ float4 lds4[];
    float* const lds = reinterpret_cast<float*>(lds4);

    const int unit = blockIdx.x;
    BArgs A;
    A.q = q; A.k = k; A.v = v; A.alpha = alpha; A.beta = beta; A.d_o = d_o; A.skv = skv;
    A.qnorm = qnorm; A.knorm = knorm; A.gq = gq; A.gk = gk; A.gv = gv; A.ga = ga; A.gb = gb;
    A.h = unit / B;
    A.b = unit - A.h * B;
    A.T = T; A.H = H;
    A.ldx = ldx; A.ldg = ldg;
    A.d = (long)H * DH;
    A.ubase = (long)A.b * T * A.d + (long)A.h * DH;
    A.gbase = (long)A.b * T * H + A.h;
    A.hoff = (long)A.h * DH;
    A.ckb = ckpt + (long)unit * nslots * DH2;
    A.nseg = (T + CK - 1) / CK;
    const int nseg = A.nseg;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;

    // every gate of the unit in the scaled range?  (the steps past T are padded in range)
    int bad = 0;
    for (int t = threadIdx.x; t < T; t += 2 * NT) {
        const float a = alpha[A.gbase + (long)t * H];
        bad |= !(a >= 0x1p-6f && a <= 0x1p6f);
    }
    if (__syncthreads_or(bad)) {
        if (w < W) bwd_serial<FUSED, AL>(A, lds, w, lane);
        else bwd_mirror(lds, nseg);
        return;
    }

    const int rg = lane & 7, cg = lane >> 3;
    const int rowb = BM * rg;
    if (w < W) {
        // adjoint waves
        const int kc = kpos(16 * w + 2 * cg);
        float ds[BM][2];
#pragma unroll
        for (int m = 0; m < BM; ++m) ds[m][0] = ds[m][1] = 0.0f;
        lds_barrier();   // the first segment staged
        for (int p = 0; p <= nseg; ++p) {
            const int g = nseg - 1 - p;
            lds_barrier();   // P0
            if (g >= 0) {
                const float* const buf = lds + Q_STG + (g & 1) * S_BUF;
                const float gend = buf[S_G + 8 * (CK - 1) + 2];
                float* const xt = lds + Q_XT + (g & 1) * DH * P;
#pragma unroll
                for (int n = 0; n < 2; ++n) {
#pragma unroll
                    for (int m = 0; m < BM; ++m) ds[m][n] *= gend;
#pragma unroll
                    for (int e = 0; e < BM; e += 4)
                        *reinterpret_cast<float4*>(xt + (16 * w + 2 * cg + n) * P + rowb + e) =
                            make_float4(ds[e][n], ds[e + 1][n], ds[e + 2][n], ds[e + 3][n]);
                }
                aloop(ds, buf, lds + Q_DU + (g & 1) * CK * P, lds + Q_DSK + (g & 1) * CK * P,
                      lds + Q_BR + (g & 1) * 8, w, lane, rg, cg, rowb, kc);
                adj_dq(buf, lds + Q_D0, w, lane);
            } else {
                lds_barrier();   // P1
            }
        }
    } else {
        // matrix waves
        const int mw = w - W, tx = threadIdx.x - NT;
        BStage stg;
        bstage_load<FUSED, AL>(stg, nseg - 1, q, k, v, d_o, skv, alpha, beta, qnorm, knorm, A.ckb, A.ubase, A.gbase,
                               A.d, T, H, tx, lane);
        bstage_store(stg, nseg - 1, T, lds + Q_STG + ((nseg - 1) & 1) * S_BUF, tx, mw, lane);
        // the loads of segment g - 1 are issued right after P1 of the period
        // before (of segment g + 1), a whole period ahead of their store, and
        // ahead of that period's epilogue stores
        if (nseg > 1)
            bstage_load<FUSED, AL>(stg, nseg - 2, q, k, v, d_o, skv, alpha, beta, qnorm, knorm, A.ckb, A.ubase,
                                   A.gbase, A.d, T, H, tx, lane);
        lds_barrier();   // the first segment staged
        for (int p = 0; p <= nseg; ++p) {
            const int g = nseg - 1 - p, gp = g + 1;
            lds_barrier();   // P0
            MEpi e;
            if (gp < nseg)
                mprod(lds + Q_STG + (gp & 1) * S_BUF, lds + Q_XT + (gp & 1) * DH * P, lds + Q_DSK + (gp & 1) * CK * P,
                      lds + Q_DU + (gp & 1) * CK * P, lds + Q_AB + (gp & 1) * CK * W * 2, lds, mw, lane, e);
            lds_barrier();   // P1
            if (g >= 1) bstage_store(stg, g - 1, T, lds + Q_STG + ((g - 1) & 1) * S_BUF, tx, mw, lane);
            if (g >= 2)
                bstage_load<FUSED, AL>(stg, g - 2, q, k, v, d_o, skv, alpha, beta, qnorm, knorm, A.ckb, A.ubase,
                                       A.gbase, A.d, T, H, tx, lane);
            if (gp < nseg)
                mepi<FUSED>(A, e, lds, lds + Q_AB + (gp & 1) * CK * W * 2, lds + Q_BR + (gp & 1) * 8,
                            lds + Q_DU + (gp & 1) * CK * P, gp, mw, lane);
        }
    }
}

}  // namespace d64

template <bool AL>
static int launch_fwd64_t(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                          float* o, const DeltaWs& ws, int B, int T, int H, hipStream_t st) {
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&d64::delta_fwd64_k<AL>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)d64::F_LDS);
        if (e != hipSuccess)
            return fail(ASCA_ERR_HIP, "hipFuncSetAttribute(LDS %zu): %s", d64::F_LDS, hipGetErrorString(e));
        attr = true;
    }
    int rc = pre_launch("delta_fwd64");
    if (rc) return rc;
    hipLaunchKernelGGL(d64::delta_fwd64_k<AL>, dim3(B * H), dim3(d64::FNT), d64::F_LDS, st, q, k, v, alpha, beta, o,
                       ws.sk, ws.ckpt, B, T, H, ws.nslots);
    return post_launch("delta_fwd64");
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int launch_fwd64(const float* q, const float* k, const float* v, const float* alpha, const float* beta, float* o,
                 const DeltaWs& ws, int B, int T, int H, hipStream_t st) {
    if (ws.ck != d64::CK || ws.cs != 1) return fail(ASCA_ERR_INVALID, "delta_fwd64: workspace layout mismatch");
    return aligned16(q) && aligned16(k) && aligned16(v)
               ? launch_fwd64_t<true>(q, k, v, alpha, beta, o, ws, B, T, H, st)
               : launch_fwd64_t<false>(q, k, v, alpha, beta, o, ws, B, T, H, st);
}

template <bool FUSED, bool AL>
static int launch_bwd64_t(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                          const float* d_o, const DeltaWs& ws, const float* qn, const float* kn, float* gq,
                          float* gk, float* gv, long ldx, float* ga, float* gb, long ldg, int B, int T, int H,
                          hipStream_t st) {
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&d64::delta_bwd64_k<FUSED, AL>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)d64::B_LDS_ALL);
        if (e != hipSuccess)
            return fail(ASCA_ERR_HIP, "hipFuncSetAttribute(LDS %zu): %s", d64::B_LDS_ALL, hipGetErrorString(e));
        attr = true;
    }
    int rc = pre_launch("delta_bwd64");
    if (rc) return rc;
    hipLaunchKernelGGL((d64::delta_bwd64_k<FUSED, AL>), dim3(B * H), dim3(2 * d64::NT), d64::B_LDS_ALL, st, q, k, v,
                       alpha, beta, d_o, ws.sk, ws.ckpt, qn, kn, gq, gk, gv, ldx, ga, gb, ldg, B, T, H, ws.nslots);
    return post_launch("delta_bwd64");
}

int launch_bwd64(bool fused, const float* q, const float* k, const float* v, const float* alpha,
                 const float* beta, const float* d_o, const DeltaWs& ws, const float* qn, const float* kn,
                 float* gq, float* gk, float* gv, long ldx, float* ga, float* gb, long ldg, int B, int T, int H,
                 hipStream_t st) {
    if (ws.ck != d64::CK || ws.cs != 1) return fail(ASCA_ERR_INVALID, "delta_bwd64: workspace layout mismatch");
    const bool al = aligned16(q) && aligned16(k) && aligned16(v) && aligned16(d_o);
#define ASCA_B64(F, A) \
    return launch_bwd64_t<F, A>(q, k, v, alpha, beta, d_o, ws, qn, kn, gq, gk, gv, ldx, ga, gb, ldg, B, T, H, st)
    if (fused) {
        if (al) ASCA_B64(true, true);
        ASCA_B64(true, false);
    }
    if (al) ASCA_B64(false, true);
    ASCA_B64(false, false);
#undef ASCA_B64
}

}  // namespace asca
