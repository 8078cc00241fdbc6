// Gated delta rule at dh = 64, f32: the recurrence advanced 16 steps at a time
// on the matrix cores, with the state resident in registers.
//
// Same math, outputs and tolerances as DeltaBlock::scan_cpu / bptt_cpu
// (rust/src/delta.rs:244-334, :421-613).  Over a block of C = 16 steps the
// recurrence S_t = alpha_t S_{t-1} + k_t u_t^T, u_t = beta_t (v_t - alpha_t
// S_{t-1}^T k_t) unrolls into the UT (WY) form of docs/SPEC_V2.md:50-69: with
// gamma_t = prod_{s<=t} alpha_s and Gamma[t][m] = prod_{m<s<=t} alpha_s (running
// products inside the block, never a division, so alpha = 0 is exact),
//
//     L  = strict_tril(diag(beta) (Gamma o K K^T)),   T = (I + L)^-1
//     U  = T diag(beta) (V - diag(gamma) K S)           (the 16 u_t rows)
//     O  = diag(gamma) Q S + tril(Gamma o Q K^T) U       (the 16 o_t rows)
//     S' = gamma_15 S + K^T diag(Gamma[15][:]) U.
//
// One block per (sequence, head) unit, in the reference's h*B + b order; four
// waves, one per SIMD, each owning value columns 16w .. 16w + 15 of S.  Column i
// of S meets only k, q, the gates and its own v_i, so a wave advances its 64 x 16
// slab of S alone: four 16x16 accumulator tiles of the 16x16x4 f32 MFMA (lane l
// holds S[16r + 4(l/16) + j][16w + l%16] in register j of tile r).  Because the
// accumulator's row index is the MFMA's contraction index (with the k order
// permuted inside each 4-row group), the state feeds the products K S and
// Q S directly and the block update lands in the same registers: the state
// never leaves them.  Per block and wave that is 16 + 16 + 4 + 4 + 16 = 56 MFMAs
// (K S, Q S, T R, M U, the update).
//
// The state-independent per-block matrices (T, M, gamma, beta, Gamma[15][:])
// are formed one group of four blocks ahead, one block per wave (the Gram
// products K K^T and Q K^T on the MFMA, T by back substitution one row per lane),
// and handed over in LDS with one barrier per group.
#include "common.h"
#include "delta.h"
#include "runtime.h"

namespace asca {
namespace ut64 {

constexpr int DH = 64;
constexpr int C = 16;          // steps per block (= checkpoint interval)
constexpr int NW = 4;          // waves per unit
constexpr int NT = 64 * NW;
constexpr int DH2 = DH * DH;

// D += A B on a 16x16x4 f32 MFMA: lane l gives A[l % 16][l / 16] and
// B[l / 16][l % 16] and holds D[4 (l / 16) + r][l % 16] in register r.
ASCA_DEV f32x4 mfma4(float a, float b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }
ASCA_DEV float readlane_f(float x, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l)); }
ASCA_DEV float el(const float4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

template <bool AL>
ASCA_DEV float4 ld4(const float* __restrict__ p) {
    if constexpr (AL) return *reinterpret_cast<const float4*>(p);
    else return make_float4(p[0], p[1], p[2], p[3]);
}

// One block's state-independent matrices in LDS (floats).
constexpr int P_T = 0;      // T = (I + L)^-1, row-major [16][16]
constexpr int P_M = 256;    // M = tril(Gamma o Q K^T), row-major [16][16]
constexpr int P_GAM = 512;  // gamma_t
constexpr int P_BET = 528;  // beta_t (0 past the sequence end)
constexpr int P_GC = 544;   // Gamma[15][m] = prod_{m<s<=15} alpha_s
constexpr int P_SZ = 576;
constexpr int NSLOT = 8;    // two groups of four blocks
constexpr int F_SCR = NSLOT * P_SZ;      // per wave: L^T scratch [16][16]
constexpr int F_FLOATS = F_SCR + NW * 256;

struct PrepIn {
    float4 kr[4], qr[4];  // K, Q rows n = lane % 16: columns 16r + 4(lane/16) .. +3
    float a, b;           // alpha, beta of step n (as loaded)
};

// Forms block p's matrices from its loads into the slot `ps`.  Steps past the
// sequence end get alpha = 1, beta = 0: they leave the state, T and the
// products of the live steps unchanged.  `scr` is the wave's own scratch.
ASCA_DEV void prep_compute(const PrepIn& pi, int p, int T, float* __restrict__ ps, float* __restrict__ scr,
                           int lane) {
    const int n = lane & 15, g = lane >> 4;
    const bool live = p * C + n < T;
    const float a = live ? pi.a : 1.0f;
    const float b = live ? pi.b : 0.0f;
    // Gram products: A[t][m] = k_t . k_m, Bq[t][m] = q_t . k_m (lane: t = 4g + i, m = n)
    f32x4 A = {0.f, 0.f, 0.f, 0.f}, Bq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            A = mfma4(el(pi.kr[r], i), el(pi.kr[r], i), A);
            Bq = mfma4(el(pi.qr[r], i), el(pi.kr[r], i), Bq);
        }
    const float gam = prefix_prod<16>(a);  // lane n: gamma_n
    // G[i] = Gamma[4g + i][n] for 4g + i >= n; pr ends as Gamma[15][n]
    float G[4] = {1.f, 1.f, 1.f, 1.f};
    float pr = 1.0f;
#pragma unroll
    for (int s = 0; s < C; ++s) {
        const float as = readlane_f(a, s);
        pr = s > n ? pr * as : pr;
        if ((s >> 2) == g) G[s & 3] = pr;
    }
    if (g == 0) {
        ps[P_GAM + n] = gam;
        ps[P_BET + n] = b;
        ps[P_GC + n] = pr;
    }
    const float4 bt = *reinterpret_cast<const float4*>(ps + P_BET + 4 * g);
    float Lv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = 4 * g + i;
        Lv[i] = n < t ? el(bt, i) * G[i] * A[i] : 0.f;
        ps[P_M + t * 16 + n] = n <= t ? G[i] * Bq[i] : 0.f;
    }
    // scr holds L^T row-major: scr[j*16 + m] = L[m][j]
    *reinterpret_cast<float4*>(scr + n * 16 + 4 * g) = make_float4(Lv[0], Lv[1], Lv[2], Lv[3]);
    // row n of T = (I + L)^-1 from x^T (I + L) = e_n^T, columns from the last:
    // x_j = [j == n] - sum_{m > j} x_m L[m][j]
    float x[C];
#pragma unroll
    for (int j = C - 1; j >= 0; --j) {
        float acc = n == j ? 1.f : 0.f;
#pragma unroll
        for (int m = j + 1; m < C; ++m) acc -= x[m] * scr[j * 16 + m];
        x[j] = acc;
    }
    if (g == 0) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
            *reinterpret_cast<float4*>(ps + P_T + n * 16 + 4 * q4) =
                make_float4(x[4 * q4], x[4 * q4 + 1], x[4 * q4 + 2], x[4 * q4 + 3]);
    }
}

// Staging of a group's k, q, v rows in LDS: buffer of 4 blocks x 16 rows, row
// pitch 68 floats (68 = 4 mod 32: the 16-byte reads of 16 rows at one offset
// spread over the banks).  Two buffers, alternating by group.
constexpr int RP = 68;
constexpr int G_ROWS = NW * C;               // rows of one group
constexpr int S_MAT = G_ROWS * RP;           // one matrix of a group
constexpr int S_BUF = 3 * S_MAT;             // k, q, v
constexpr int F_STG = F_FLOATS;              // [2][S_BUF]
constexpr int F_OT = F_STG + 2 * S_BUF;      // per wave: the o and u tiles [2][16][20] on their way out
constexpr int OTP = 20;
constexpr int F_ALL = F_OT + NW * 2 * C * OTP;
constexpr size_t F_LDS = (size_t)F_ALL * 4;
static_assert(F_LDS <= 160 * 1024, "forward LDS");

// Wave w stages block c0 + w of the group: 16 rows of k, q, v, four 16-byte
// loads per matrix and lane (a row per 16 lanes).  Rows past the sequence end
// repeat its last row (their gates make them inert).
struct Stage {
    float4 x[3][4];
};

template <bool AL>
ASCA_DEV void stage_load(Stage& st, int c, const float* __restrict__ q, const float* __restrict__ k,
                         const float* __restrict__ v, long ubase, long d, int T, int lane) {
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
        const long t = min(c * C + (lane >> 4) + 4 * s4, T - 1);
        const long off = ubase + t * d + 4 * (lane & 15);
        st.x[0][s4] = ld4<AL>(k + off);
        st.x[1][s4] = ld4<AL>(q + off);
        st.x[2][s4] = ld4<AL>(v + off);
    }
}

ASCA_DEV void stage_store(const Stage& st, float* __restrict__ buf, int w, int lane) {
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
        const int row = 16 * w + (lane >> 4) + 4 * s4;
#pragma unroll
        for (int m = 0; m < 3; ++m)
            *reinterpret_cast<float4*>(buf + m * S_MAT + row * RP + 4 * (lane & 15)) = st.x[m][s4];
    }
}

// Checkpoint slot layout (4096 floats): the accumulator tiles as the forward's
// waves hold them, 16 bytes per lane: float4 index (w*4 + r)*64 + lane holds
// S[16r + 4(lane/16) + j][16w + lane%16], j = 0..3.
ASCA_DEV void ck_store(float* __restrict__ slot, const f32x4 (&S)[4], int w, int lane) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
        *reinterpret_cast<float4*>(slot + ((w * 4 + r) * 64 + lane) * 4) = make_float4(S[r][0], S[r][1], S[r][2], S[r][3]);
}

// One block of 16 steps for the wave's 64 x 16 slab of S: outputs o, the u rows
// (for the backward), the checkpoint (state before the block) and the block
// update.  `kb` points at the block's first staged k row
// (q and v rows follow at S_MAT and 2 S_MAT).
template <bool FULL, bool AL>
ASCA_DEV void chain_step(f32x4 (&S)[4], const float* __restrict__ kb, const float* __restrict__ ps,
                         float* __restrict__ ot, int c, float* __restrict__ o, float* __restrict__ ws_u,
                         float* __restrict__ ckb, long ubase, long d, int T, int w, int lane) {
    const int n = lane & 15, g = lane >> 4;
    const float* qb = kb + S_MAT;
    const float* vb = kb + 2 * S_MAT;
    float4 kc[4], qc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        kc[r] = *reinterpret_cast<const float4*>(kb + n * RP + 16 * r + 4 * g);
        qc[r] = *reinterpret_cast<const float4*>(qb + n * RP + 16 * r + 4 * g);
    }
    const float4 gm = *reinterpret_cast<const float4*>(ps + P_GAM + 4 * g);
    const float4 bt = *reinterpret_cast<const float4*>(ps + P_BET + 4 * g);
    const float4 gc = *reinterpret_cast<const float4*>(ps + P_GC + 4 * g);
    const float4 tr = *reinterpret_cast<const float4*>(ps + P_T + n * 16 + 4 * g);
    const float4 mr = *reinterpret_cast<const float4*>(ps + P_M + n * 16 + 4 * g);
    const float g15 = ps[P_GAM + 15];
    float vv[4], kt[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        vv[i] = vb[(4 * g + i) * RP + 16 * w + n];
#pragma unroll
        for (int r = 0; r < 4; ++r) kt[r][i] = kb[(4 * g + i) * RP + 16 * r + n];
    }
    f32x4 ka = {0.f, 0.f, 0.f, 0.f}, kb2 = ka, qa = ka, qb2 = ka;
#pragma unroll
    for (int r = 0; r < 4; r += 2)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ka = mfma4(el(kc[r], i), S[r][i], ka);
            qa = mfma4(el(qc[r], i), S[r][i], qa);
            kb2 = mfma4(el(kc[r + 1], i), S[r + 1][i], kb2);
            qb2 = mfma4(el(qc[r + 1], i), S[r + 1][i], qb2);
        }
    float R[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) R[i] = el(bt, i) * (vv[i] - el(gm, i) * (ka[i] + kb2[i]));
    f32x4 U = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) U = mfma4(el(tr, i), R[i], U);
    f32x4 O;
#pragma unroll
    for (int i = 0; i < 4; ++i) O[i] = el(gm, i) * (qa[i] + qb2[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) O = mfma4(el(mr, i), U[i], O);
    ck_store(ckb + (long)c * DH2, S, w, lane);
    // o and u rows leave as 16-byte stores: the 16 x 16 tiles go through the
    // wave's LDS scratch (lane: row lane / 4, columns 4 (lane % 4) .. +3)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        ot[(4 * g + i) * OTP + n] = O[i];
        ot[C * OTP + (4 * g + i) * OTP + n] = U[i];
    }
    {
        const int rr = lane >> 2, cc = 4 * (lane & 3);
        const float4 o4 = *reinterpret_cast<const float4*>(ot + rr * OTP + cc);
        const float4 u4 = *reinterpret_cast<const float4*>(ot + C * OTP + rr * OTP + cc);
        const long t = (long)c * C + rr;
        if (FULL || t < T) {
            float* po = o + ubase + t * d + 16 * w + cc;
            if constexpr (AL) *reinterpret_cast<float4*>(po) = o4;
            else { po[0] = o4.x; po[1] = o4.y; po[2] = o4.z; po[3] = o4.w; }
            *reinterpret_cast<float4*>(ws_u + ubase + t * d + 16 * w + cc) = u4;
        }
    }
    float Ut[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) Ut[i] = el(gc, i) * U[i];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        S[r] *= g15;
#pragma unroll
        for (int i = 0; i < 4; ++i) S[r] = mfma4(kt[r][i], Ut[i], S[r]);
    }
}

// A helper wave's gate loads: lane l holds alpha, beta of step 16 c + (l % 16).
ASCA_DEV void gate_load(float& a, float& b, int c, const float* __restrict__ alpha, const float* __restrict__ beta,
                        long gbase, int T, int H, int lane) {
    const long t = min(c * C + (lane & 15), T - 1);
    a = alpha[gbase + t * H];
    b = beta[gbase + t * H];
}

// The helper wave's prep of block p from its staged rows (rows 16 hw .. of `buf`).
ASCA_DEV void helper_prep(int p, const float* __restrict__ buf, float a, float b, float* __restrict__ ps,
                          float* __restrict__ scr, int T, int hw, int lane) {
    const int n = lane & 15, g = lane >> 4;
    PrepIn pi;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        pi.kr[r] = *reinterpret_cast<const float4*>(buf + (C * hw + n) * RP + 16 * r + 4 * g);
        pi.qr[r] = *reinterpret_cast<const float4*>(buf + S_MAT + (C * hw + n) * RP + 16 * r + 4 * g);
    }
    pi.a = a;
    pi.b = b;
    prep_compute(pi, p, T, ps, scr, lane);
}

// Block of 2 NW waves.  Waves 0 .. NW-1 (one per SIMD) run the chain: wave w owns
// value columns 16w .. 16w + 15 and advances the state block by block from the
// staged rows and the prepared matrices.  Waves NW .. 2NW-1 (one per SIMD beside
// them) are helpers: during group g the helper hw stages block 4(g+1) + hw's
// k, q, v rows into the other buffer and forms that block's matrices, so the
// chain waves' matrix cores share their SIMD with the helpers' products and the
// helpers' VALU and LDS work fills the chain's dependency stalls.  One barrier
// per group of four blocks.
template <bool AL>
__global__ __launch_bounds__(2 * NT) void ut_fwd64_k(const float* __restrict__ q, const float* __restrict__ k,
                                                     const float* __restrict__ v, const float* __restrict__ alpha,
                                                     const float* __restrict__ beta, float* __restrict__ o,
                                                     float* __restrict__ ws_u, float* __restrict__ ckpt, int B,
                                                     int T, int H, int nslots) {
    extern __shared__ float lds[];
    const int unit = blockIdx.x;  // h*B + b
    const int h = unit / B, b = unit - h * B;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const long d = (long)H * DH;
    const long ubase = (long)b * T * d + (long)h * DH;
    const int NC = (T + C - 1) / C;

    if (w >= NW) {
        const int hw = w - NW;
        const long gbase = (long)b * T * H + h;
        float* scr = lds + F_SCR + hw * 256;
        Stage stg;
        float ga, gb;
        stage_load<AL>(stg, min(hw, NC - 1), q, k, v, ubase, d, T, lane);
        gate_load(ga, gb, min(hw, NC - 1), alpha, beta, gbase, T, H, lane);
        stage_store(stg, lds + F_STG, hw, lane);
        if (hw < NC) helper_prep(hw, lds + F_STG, ga, gb, lds + hw * P_SZ, scr, T, hw, lane);
        stage_load<AL>(stg, min(NW + hw, NC - 1), q, k, v, ubase, d, T, lane);
        gate_load(ga, gb, min(NW + hw, NC - 1), alpha, beta, gbase, T, H, lane);
        lds_barrier();
        for (int c0 = 0; c0 < NC; c0 += NW) {
            const int pn = c0 + NW + hw;
            float* nbuf = lds + F_STG + (((c0 / NW) + 1) & 1) * S_BUF;
            stage_store(stg, nbuf, hw, lane);
            const float a = ga, bb = gb;
            stage_load<AL>(stg, min(pn + NW, NC - 1), q, k, v, ubase, d, T, lane);
            gate_load(ga, gb, min(pn + NW, NC - 1), alpha, beta, gbase, T, H, lane);
            if (pn < NC) helper_prep(pn, nbuf, a, bb, lds + (pn % NSLOT) * P_SZ, scr, T, hw, lane);
            lds_barrier();
        }
        return;
    }

    float* ot = lds + F_OT + w * 2 * C * OTP;
    float* ckb = ckpt + (long)unit * nslots * DH2;
    f32x4 S[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) S[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    lds_barrier();
    const int NCF = T / C;
    for (int c0 = 0; c0 < NC; c0 += NW) {
        const float* buf = lds + F_STG + ((c0 / NW) & 1) * S_BUF;
        if (c0 + NW <= NCF) {
#pragma unroll
            for (int j = 0; j < NW; ++j)
                chain_step<true, AL>(S, buf + j * C * RP, lds + ((c0 + j) % NSLOT) * P_SZ, ot, c0 + j, o, ws_u, ckb,
                                     ubase, d, T, w, lane);
        } else {
            for (int j = 0; j < NW && c0 + j < NC; ++j)
                chain_step<false, AL>(S, buf + j * C * RP, lds + ((c0 + j) % NSLOT) * P_SZ, ot, c0 + j, o, ws_u,
                                      ckb, ubase, d, T, w, lane);
        }
        lds_barrier();
    }
    ck_store(ckb + (long)NC * DH2, S, w, lane);
}

}  // namespace ut64

static bool ut_aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <bool AL>
static int launch_ut_fwd64_t(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                             float* o, const DeltaWs& ws, int B, int T, int H, hipStream_t st) {
    const int units = B * H;
    const size_t lds = ut64::F_LDS;
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&ut64::ut_fwd64_k<AL>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)ut64::F_LDS);
        if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipFuncSetAttribute: %s", hipGetErrorString(e));
        attr = true;
    }
    int rc = pre_launch("ut_fwd64");
    if (rc) return rc;
    hipLaunchKernelGGL(ut64::ut_fwd64_k<AL>, dim3(units), dim3(2 * ut64::NT), lds, st, q, k, v, alpha, beta, o, ws.sk,
                       ws.ckpt, B, T, H, ws.nslots);
    return post_launch("ut_fwd64");
}

int launch_ut_fwd64(const float* q, const float* k, const float* v, const float* alpha, const float* beta, float* o,
                    const DeltaWs& ws, int B, int T, int H, hipStream_t st) {
    if (ws.ck != ut64::C || ws.cs != 1) return fail(ASCA_ERR_INVALID, "ut_fwd64: workspace layout mismatch");
    return ut_aligned16(q) && ut_aligned16(k) && ut_aligned16(v) && ut_aligned16(o)
               ? launch_ut_fwd64_t<true>(q, k, v, alpha, beta, o, ws, B, T, H, st)
               : launch_ut_fwd64_t<false>(q, k, v, alpha, beta, o, ws, B, T, H, st);
}

}  // namespace asca
