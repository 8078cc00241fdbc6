// Kernels of the gated delta rule at dh = 64, f32: the recurrence advanced 16 steps at a time
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
//
// The kernel templates and their launch templates live in this header, included
// by delta_ut64.hip (the forward and the fused, 16-byte-aligned backward: the
// hot path, compiled with its own scheduler setting) and by delta_ut64_b.hip
// (the other backward variants, compiled with the default one).
#pragma once
#include "common.h"
#include "delta.h"
#include "runtime.h"

namespace asca {
namespace ut64 {

constexpr int DH = 64;
constexpr int C = 16;          // steps per block; a checkpoint every 2 C steps
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

// Buffer resources over the unit's part of every array the forward reads or
// writes, made once per kernel: a load's or store's lane offset is then
// loop-invariant and the block's offset a uniform register.  Rows past the
// sequence end lie outside the row resources: they load as 0 (their gates make
// such steps inert) and their stores are dropped.
struct FRes {
    Rsrc q, k, v, o, al, be, u, ck, rec;
};

struct PrepIn {
    float4 kr[4], qr[4];  // K, Q rows n = lane % 16: columns 16r + 4(lane/16) .. +3
    float a, b;           // alpha, beta of step n (as loaded)
};

// Forms block p's matrices from its loads into the slot `ps`.  Steps past the
// sequence end get alpha = 1, beta = 0: they leave the state, T and the
// products of the live steps unchanged.  `scr` is the wave's own scratch.
// Record of a block for the backward (1344 floats): K K^T, Q K^T, T, M and
// Gamma (zero above the diagonal) in the accumulator layout, 16 bytes per lane (float4 index 64 m + lane holds
// matrix m's elements [4 (lane/16) + j][lane % 16], j = 0..3), then the per-step gate
// vectors gamma_t, beta_t gamma_t, Gamma[15][t], beta_t (16 floats each; steps past the
// sequence end as alpha = 1, beta = 0), so that no wave of the backward forms them again.
constexpr int R_A = 0, R_BQ = 256, R_T = 512, R_M = 768, R_G = 1024, R_V = 1280, R_SZ = 1344;
// U_TILE: the u rows for the backward, per unit and block (U_BLK floats): the
// four chain waves' 16 x 16 tiles (value columns 16w ..) one after another,
// each row-major, so a wave writes its block's u as one contiguous 1 KB.
constexpr int U_BLK = 4 * 256;
static_assert(U_BLK == D64_BLK * DH, "a block's u rows");
constexpr int RV_GAM = R_V, RV_BG = R_V + 16, RV_GC = R_V + 32, RV_BET = R_V + 48;
static_assert(R_SZ == D64_REC, "record size");
static_assert(C == D64_BLK && D64_CK == 2 * C, "a checkpoint before every other block");

ASCA_DEV void prep_compute(const PrepIn& pi, int p, int T, float* __restrict__ ps, float* __restrict__ scr,
                           Rsrc rrec, int lane) {
    const unsigned srec = 4u * (unsigned)(p * R_SZ);   // the block's record
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
    buf_store1(rrec, 4u * (R_V + lane), g == 0 ? gam : g == 1 ? b * gam : g == 2 ? pr : b, srec);
    const float4 bt = *reinterpret_cast<const float4*>(ps + P_BET + 4 * g);
    float Lv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = 4 * g + i;
        Lv[i] = n < t ? el(bt, i) * G[i] * A[i] : 0.f;
        ps[P_M + t * 16 + n] = n <= t ? G[i] * Bq[i] : 0.f;
    }
    // scr holds L row-major: scr[m*16 + j] = L[m][j]
#pragma unroll
    for (int i = 0; i < 4; ++i) scr[(4 * g + i) * 16 + n] = Lv[i];
    // row n of T = (I + L)^-1 from x^T (I + L) = e_n^T, columns from the last:
    // x_j = [j == n] - sum_{m > j} x_m L[m][j]
    // Right-looking: once x_m is final it is taken out of every x_j, j < m (the
    // terms of each x_j in descending m), so x_j is one FMA behind x_{j+1}
    // instead of at the end of a chain of 15 - j, with 16 live partial sums.
    float x[C];
#pragma unroll
    for (int j = 0; j < C; ++j) x[j] = n == j ? 1.f : 0.f;
    float4 rw[2][4];
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) rw[C & 1][q4] = *reinterpret_cast<const float4*>(scr + (C - 1) * 16 + 4 * q4);
#pragma unroll
    for (int m = C - 1; m >= 1; --m) {
        // row m - 1 read one step ahead (broadcast: every lane the same address)
        if (m > 1) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4)
                if (4 * q4 < m - 1) rw[m & 1][q4] = *reinterpret_cast<const float4*>(scr + (m - 1) * 16 + 4 * q4);
        }
#pragma unroll
        for (int j = 0; j < m; ++j) x[j] -= x[m] * el(rw[(m + 1) & 1][j >> 2], j & 3);
        __builtin_amdgcn_sched_barrier(0);   // keep the solve's steps in order (bounds the live registers)
    }
    if (g == 0) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
            *reinterpret_cast<float4*>(ps + P_T + n * 16 + 4 * q4) =
                make_float4(x[4 * q4], x[4 * q4 + 1], x[4 * q4 + 2], x[4 * q4 + 3]);
    }
    buf_store4(rrec, 16u * ((R_A >> 2) + lane), make_float4(A[0], A[1], A[2], A[3]), srec);
    buf_store4(rrec, 16u * ((R_BQ >> 2) + lane), make_float4(Bq[0], Bq[1], Bq[2], Bq[3]), srec);
    const float* tp = ps + P_T + 64 * g + n;
    buf_store4(rrec, 16u * ((R_T >> 2) + lane), make_float4(tp[0], tp[16], tp[32], tp[48]), srec);
    const float* mp = ps + P_M + 64 * g + n;
    buf_store4(rrec, 16u * ((R_M >> 2) + lane), make_float4(mp[0], mp[16], mp[32], mp[48]), srec);
    buf_store4(rrec, 16u * ((R_G >> 2) + lane),
               make_float4(n <= 4 * g ? G[0] : 0.f, n <= 4 * g + 1 ? G[1] : 0.f, n <= 4 * g + 2 ? G[2] : 0.f,
                           n <= 4 * g + 3 ? G[3] : 0.f),
               srec);
}

// Staging of a group's k, q, v rows in LDS: buffer of 4 blocks x 16 rows, row
// pitch 68 floats (68 = 4 mod 32: the 16-byte reads of 16 rows at one offset
// spread over the banks).  Two buffers, alternating by group.
constexpr int RP = 68;
constexpr int G_ROWS = NW * C;               // rows of one group
constexpr int S_MAT = G_ROWS * RP;           // one matrix of a group
constexpr int S_BUF = 3 * S_MAT;             // k, q, v
constexpr int F_STG = F_FLOATS;              // [2][S_BUF]
constexpr int F_OT = F_STG + 2 * S_BUF;      // per wave: the o and u tiles and a state tile [3][16][20] on their way out
constexpr int OTP = 20;
constexpr int F_ALL = F_OT + NW * 3 * C * OTP;
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
                         const float* __restrict__ v, const FRes& R, long ubase, long d, int T, int lane) {
    if constexpr (AL) {
        const unsigned so = 4u * (unsigned)(c * C * d);
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
            const unsigned vo = 4u * (unsigned)(((lane >> 4) + 4 * s4) * d + 4 * (lane & 15));
            st.x[0][s4] = buf_load4(R.k, vo, so);
            st.x[1][s4] = buf_load4(R.q, vo, so);
            st.x[2][s4] = buf_load4(R.v, vo, so);
        }
        return;
    }
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

// Checkpoint slot layout (4096 floats), the state before a block as the
// backward's key-slab waves read it, 16 bytes per lane: float4 index
// (r*4 + c)*64 + lane holds S[16r + lane%16][16c + 4(lane/16) + j], j = 0..3
// (key tile r, value tile c).  The forward's wave w holds value tile c = w with
// keys and values swapped within each 16 x 16 tile, so every tile is transposed
// through the wave's LDS scratch `st` on its way out.
ASCA_DEV void ck_store(const FRes& R, int slot, const f32x4 (&S)[4], float* __restrict__ st, int w, int lane) {
    const int n = lane & 15, g = lane >> 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int i = 0; i < 4; ++i) st[(4 * g + i) * OTP + n] = S[r][i];
        const float4 t4 = *reinterpret_cast<const float4*>(st + n * OTP + 4 * g);
        buf_store4(R.ck, 16u * ((r * 4 + w) * 64 + lane), t4, 4u * (unsigned)(slot * DH2));
    }
}

// One block of 16 steps for the wave's 64 x 16 slab of S: outputs o, the u rows
// (for the backward), the checkpoint (state before the block, even blocks) and the block
// update.  `kb` points at the block's first staged k row
// (q and v rows follow at S_MAT and 2 S_MAT).
template <bool FULL, bool AL>
ASCA_DEV void chain_step(f32x4 (&S)[4], const float* __restrict__ kb, const float* __restrict__ ps,
                         float* __restrict__ ot, int c, float* __restrict__ o, const FRes& res, bool ckw, long ubase,
                         long d, int T, int w, int lane) {
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
    if (ckw) ck_store(res, c >> 1, S, ot + 2 * C * OTP, w, lane);
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
        if constexpr (AL) {
            // rows past the sequence end fall outside the resource: dropped
            buf_store4(res.o, 4u * (unsigned)(rr * d + 16 * w + cc), o4, 4u * (unsigned)(c * C * d));
        } else {
            const long t = (long)c * C + rr;
            if (FULL || t < T) {
                float* po = o + ubase + t * d + 16 * w + cc;
                po[0] = o4.x; po[1] = o4.y; po[2] = o4.z; po[3] = o4.w;
            }
        }
        // u tile: 1 KB contiguous per wave and block (layout at U_TILE)
        buf_store4(res.u, 4u * (unsigned)(w * 256 + rr * 16 + cc), u4, 4u * (unsigned)(c * U_BLK));
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
// Steps past the sequence end load 0 (prep_compute makes them alpha = 1, beta = 0).
ASCA_DEV void gate_load(float& a, float& b, int c, const FRes& R, int H, int lane) {
    const unsigned vo = 4u * (unsigned)((lane & 15) * H), so = 4u * (unsigned)(c * C * H);
    a = buf_load1(R.al, vo, so);
    b = buf_load1(R.be, vo, so);
}

// The helper wave's prep of block p from its staged rows (rows 16 hw .. of `buf`).
ASCA_DEV void helper_prep(int p, const float* __restrict__ buf, float a, float b, float* __restrict__ ps,
                          float* __restrict__ scr, Rsrc rrec, int T, int hw, int lane) {
    const int n = lane & 15, g = lane >> 4;
    PrepIn pi;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        pi.kr[r] = *reinterpret_cast<const float4*>(buf + (C * hw + n) * RP + 16 * r + 4 * g);
        pi.qr[r] = *reinterpret_cast<const float4*>(buf + S_MAT + (C * hw + n) * RP + 16 * r + 4 * g);
    }
    pi.a = a;
    pi.b = b;
    prep_compute(pi, p, T, ps, scr, rrec, lane);
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
                                                     float* __restrict__ ws_u, float* __restrict__ ckpt,
                                                     float* __restrict__ rec, int B, int T, int H, int nslots) {
    extern __shared__ float lds[];
    const int unit = blockIdx.x;  // h*B + b
    const int h = unit / B, b = unit - h * B;
    // the wave index, uniform in a scalar register (so are the block indices and
    // buffer offsets derived from it)
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const long d = (long)H * DH;
    const long ubase = (long)b * T * d + (long)h * DH;
    const int NC = (T + C - 1) / C;
    FRes R;
    {
        const unsigned rows = 4u * (unsigned)((T - 1) * d + DH);   // the unit's columns of rows t < T
        R.q = make_rsrc(q + ubase, rows);
        R.k = make_rsrc(k + ubase, rows);
        R.v = make_rsrc(v + ubase, rows);
        R.o = make_rsrc(o + ubase, rows);
        const long gbase = (long)b * T * H + h;
        const unsigned grow = 4u * (unsigned)((T - 1) * H + 1);
        R.al = make_rsrc(alpha + gbase, grow);
        R.be = make_rsrc(beta + gbase, grow);
        R.u = make_rsrc(ws_u + (long)unit * NC * U_BLK, 4u * (unsigned)(NC * U_BLK));
        R.ck = make_rsrc(ckpt + (long)unit * nslots * DH2, 4u * (unsigned)(nslots * DH2));
        R.rec = make_rsrc(rec + (long)unit * NC * R_SZ, 4u * (unsigned)(NC * R_SZ));
    }

    if (w >= NW) {
        const int hw = w - NW;
        float* scr = lds + F_SCR + hw * 256;
        Stage stg;
        float ga, gb;
        stage_load<AL>(stg, min(hw, NC - 1), q, k, v, R, ubase, d, T, lane);
        gate_load(ga, gb, min(hw, NC - 1), R, H, lane);
        stage_store(stg, lds + F_STG, hw, lane);
        if (hw < NC) helper_prep(hw, lds + F_STG, ga, gb, lds + hw * P_SZ, scr, R.rec, T, hw, lane);
        stage_load<AL>(stg, min(NW + hw, NC - 1), q, k, v, R, ubase, d, T, lane);
        gate_load(ga, gb, min(NW + hw, NC - 1), R, H, lane);
        lds_barrier();
        for (int c0 = 0; c0 < NC; c0 += NW) {
            const int pn = c0 + NW + hw;
            float* nbuf = lds + F_STG + (((c0 / NW) + 1) & 1) * S_BUF;
            stage_store(stg, nbuf, hw, lane);
            const float a = ga, bb = gb;
            stage_load<AL>(stg, min(pn + NW, NC - 1), q, k, v, R, ubase, d, T, lane);
            gate_load(ga, gb, min(pn + NW, NC - 1), R, H, lane);
            if (pn < NC) helper_prep(pn, nbuf, a, bb, lds + (pn % NSLOT) * P_SZ, scr, R.rec, T, hw, lane);
            lds_barrier();
        }
        return;
    }

    float* ot = lds + F_OT + w * 3 * C * OTP;
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
                chain_step<true, AL>(S, buf + j * C * RP, lds + ((c0 + j) % NSLOT) * P_SZ, ot, c0 + j, o, R,
                                     (j & 1) == 0, ubase, d, T, w, lane);
        } else {
            for (int j = 0; j < NW && c0 + j < NC; ++j)
                chain_step<false, AL>(S, buf + j * C * RP, lds + ((c0 + j) % NSLOT) * P_SZ, ot, c0 + j, o, R,
                                      ((c0 + j) & 1) == 0, ubase, d, T, w, lane);
        }
        lds_barrier();
    }
    ck_store(R, (NC + 1) >> 1, S, ot + 2 * C * OTP, w, lane);
}

// ================================================================= backward
//
// Reverse over the blocks, with X = dL/dS' the gradient of the state after the
// block (zero after the last step, as bptt_cpu starts, delta.rs:475-587), the
// block's gradients follow from the UT form (the oracle's chunked restatement):
//
//     dU = M^T dO + diag(Gamma[15][:]) K X,      Y = T^T dU,     dv = diag(beta) Y
//     X_prev = gamma_15 X + (diag(gamma) Q)^T dO - K^T diag(beta gamma) Y
//     dM = tril(dO U^T),   dL = -strict_tril(Y U^T),   dA = dL o beta_row o Gamma
//     dq = diag(gamma) dO S^T + (Gamma o dM) K
//     dk = -diag(beta gamma) Y S^T + diag(Gamma[15][:]) U X^T + (Gamma o dM)^T Q + (dA + dA^T) K
//     dbeta, dgamma, dGamma from row sums, dalpha from running products (no division).
//
// Eight waves per unit.  The four chain waves own value columns 16w .. 16w + 15
// of X (accumulator tiles, like the forward's state) and run only the X
// recurrence (K X, M^T dO, T^T dU, the update: 56 MFMAs per block) plus dv and
// their share of dO U^T and Y U^T.  They hand X (before its update) and Y over
// in LDS, and stage the k, q, dO, u rows of the block after theirs.  The four
// helper waves own key columns 16hw .. 16hw + 15 of dq and dk:
// one block behind the chain they form dO S^T, Y S^T, U X^T over all value
// columns (S from the forward's checkpoint, advanced by one block for odd
// blocks), dq and dk and their row
// sums; one more block behind, the L2-norm backward of dq, dk (from the row dots
// of all four helpers) and the stores.  One barrier per block.  The gate gradients
// need sums over all four helpers and all value columns: the helpers leave
// theirs in the workspace's backward scratch, and after the block loop all
// eight waves form dalpha, dbeta of every block from them.
constexpr int SB_MAT = C * RP;
constexpr int SB_K = 0, SB_Q = SB_MAT, SB_DO = 2 * SB_MAT, SB_U = 3 * SB_MAT;
constexpr int SB_BUF = 4 * SB_MAT;
constexpr int NSB = 3;                       // stage buffers: block c in buffer c % 3
constexpr int HO_DS = 0;                     // X tiles, checkpoint layout [r][c][lane][4]
constexpr int HO_Y = 4096;                   // Y tiles: [c][lane] float4 = Y[n][16c + 4g ..]
constexpr int HO_DM = 5120;                  // per chain wave dO_w U_w^T (accumulator layout)
constexpr int HO_DL = 6144;                  // per chain wave Y_w U_w^T
constexpr int HO_YV = 7168;                  // per chain wave row sums of Y_w o V_w [w][16]
constexpr int HO_SZ = 7232;
// a helper's five row sums over its keys: q.dq, k.dk (to the epilogue, in LDS
// [hw][2][16]) and q.F, k.Zt, k.D (to the gate gradients, in the backward scratch)
constexpr int EP_RQ = 0, EP_RK = 1, EP_QF = 2, EP_ZK = 3, EP_KD = 4;
constexpr int EP_SZ = NW * 2 * 16;
// per unit and block in the backward's scratch (GS_SZ floats): what the gate
// gradients need, written by the helpers with the block's products, read after
// the block loop
constexpr int GS_ROW = 0;                    // [hw][3][16]: q.F, k.Zt, k.D row sums per helper
constexpr int GS_DSS = 192;                  // [hw]: <X, S> per helper
constexpr int GS_YV = 196;                   // [16]: row sums of Y o V
constexpr int GS_DM = 256;                   // dM, accumulator layout [lane][4]
constexpr int GS_DL = 512;                   // dL
constexpr int GS_SZ = 768;
constexpr int WSCR = 2 * C * OTP + 128;      // per wave: two transpose tiles and a vector area
constexpr int SVO = 2 * C * OTP;             // the vector area's offset
constexpr int B_STG = 0;
constexpr int B_HO = B_STG + NSB * SB_BUF;
constexpr int B_EP = B_HO + 2 * HO_SZ;
constexpr int B_SCR = B_EP + 2 * EP_SZ;
constexpr int B_END = B_SCR + 2 * NW * WSCR;
constexpr size_t B_LDS = (size_t)B_END * 4;
static_assert(2 * NW * 4 * WSCR <= B_END, "the gate tail's scratch fits in the loop's LDS");
static_assert(B_LDS <= 160 * 1024 && B_HO % 4 == 0 && B_EP % 4 == 0 && B_SCR % 4 == 0, "backward LDS");

// Orders the wave's own LDS writes before its reads of other lanes' values.  The
// LDS executes one wave's instructions in issue order, so only the compiler has
// to keep them in program order: a compiler barrier, no wait.
ASCA_DEV void wave_sync() { asm volatile("" ::: "memory"); }

// 16x16 tile in the accumulator layout (lane (g, n) holds X[4g + j][n]) ->
// lane (g, n) receives X[n][4g .. 4g + 3].
ASCA_DEV float4 tile_t(const f32x4& x, float* __restrict__ st, int lane) {
    const int n = lane & 15, g = lane >> 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) st[(4 * g + j) * OTP + n] = x[j];
    wave_sync();
    const float4 r = *reinterpret_cast<const float4*>(st + n * OTP + 4 * g);
    wave_sync();
    return r;
}

// Values held by lane t of each 16-lane row (the same in every row) -> lane
// (g, n) receives those of lanes 4g .. 4g + 3.
ASCA_DEV float4 rows4(float x, float* __restrict__ sv, int lane) {
    if (lane < 16) sv[lane] = x;
    wave_sync();
    const float4 r = *reinterpret_cast<const float4*>(sv + 4 * (lane >> 4));
    wave_sync();
    return r;
}

// rows4 for several values at once (one LDS round trip).
template <int NQ>
ASCA_DEV void rows4x(const float (&x)[NQ], float4 (&out)[NQ], float* __restrict__ sv, int lane) {
    if (lane < 16) {
#pragma unroll
        for (int e = 0; e < NQ; ++e) sv[16 * e + lane] = x[e];
    }
    wave_sync();
#pragma unroll
    for (int e = 0; e < NQ; ++e) out[e] = *reinterpret_cast<const float4*>(sv + 16 * e + 4 * (lane >> 4));
    wave_sync();
}

// Two 16x16 accumulator tiles transposed at once (see tile_t).
ASCA_DEV void tile_t2(const f32x4& x, const f32x4& y, float4& xt, float4& yt, float* __restrict__ st, int lane) {
    const int n = lane & 15, g = lane >> 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        st[(4 * g + j) * OTP + n] = x[j];
        st[C * OTP + (4 * g + j) * OTP + n] = y[j];
    }
    wave_sync();
    xt = *reinterpret_cast<const float4*>(st + n * OTP + 4 * g);
    yt = *reinterpret_cast<const float4*>(st + C * OTP + n * OTP + 4 * g);
    wave_sync();
}

// Exclusive suffix product over each 16-lane row: lane m gets prod_{m<s<16} x_s.
ASCA_DEV float suffix_excl_prod(float x) {
    x *= dpp_or<0x101>(1.0f, x);
    x *= dpp_or<0x102>(1.0f, x);
    x *= dpp_or<0x104>(1.0f, x);
    x *= dpp_or<0x108>(1.0f, x);
    return dpp_or<0x101>(1.0f, x);
}

template <bool AL>
ASCA_DEV void store4(float* __restrict__ p, float4 x) {
    if constexpr (AL) *reinterpret_cast<float4*>(p) = x;
    else { p[0] = x.x; p[1] = x.y; p[2] = x.z; p[3] = x.w; }
}

ASCA_DEV float4 f4scale(float s, float4 x) { return make_float4(s * x.x, s * x.y, s * x.z, s * x.w); }
ASCA_DEV float4 f4add(float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }

struct BArgs {
    const float *q, *k, *v, *alpha, *beta, *d_o, *u, *ckpt, *rec, *qn, *kn;
    float *gq, *gk, *gv, *ga, *gb;
    float* gsc;   // scratch of this call: per block the sums of the gate gradients (GS_SZ floats)
    long ldx, ldg, d, ubase, gbase, rowbase;
    int B, T, H, h, nslots, NC, unit;
    int di, ldxi, ldgi;   // d, ldx, ldg as 32-bit strides (the launcher checks they fit)
};

// Buffer resources over the unit's part of every array the block loops read,
// made once per kernel (after the unit rebase): a load's lane offset is then
// loop-invariant and the block's offset a uniform register.  Rows past the
// sequence end lie outside the row resources and load as 0.
struct BRes {
    Rsrc ck, rec, nq, nk, v, k, q, dO, u;
};

ASCA_DEV BRes bres_make(const BArgs& A) {
    BRes r;
    r.ck = make_rsrc(A.ckpt, 4u * (unsigned)(A.nslots * DH2));
    r.rec = make_rsrc(A.rec, 4u * (unsigned)(A.NC * R_SZ));
    const unsigned rows = 4u * (unsigned)((A.T - 1) * A.di + DH);   // the unit's columns of rows t < T
    r.v = make_rsrc(A.v, rows);
    r.k = make_rsrc(A.k, rows);
    r.q = make_rsrc(A.q, rows);
    r.dO = make_rsrc(A.d_o, rows);
    r.u = make_rsrc(A.u, 4u * (unsigned)(A.NC * U_BLK));
    const unsigned nrm = 4u * (unsigned)((A.T - 1) * A.H + 1);
    r.nq = make_rsrc(A.qn ? A.qn : A.rec, A.qn ? nrm : 0u);
    r.nk = make_rsrc(A.kn ? A.kn : A.rec, A.kn ? nrm : 0u);
    return r;
}

struct BChainIn {
    float4 v;         // V[16c + n][16w + 4g ..]
    float4 tr, mr;    // T and M of the block (accumulator layout)
    float4 gm, bg, gc;  // gamma, beta gamma, Gamma[15][.] of steps 4g .. 4g + 3
    float g15, bn;    // gamma_15; beta of step n
};

template <bool AL>
ASCA_DEV void bchain_load(BChainIn& ci, int c, const BArgs& A, const BRes& R, int w, int lane) {
    const int n = lane & 15, g = lane >> 4;
    if constexpr (AL) {
        // v of rows past the sequence end: 0 (outside the resource; their dv is not stored)
        ci.v = buf_load4(R.v, 4u * (unsigned)(n * A.di + 16 * w + 4 * g), 4u * (unsigned)(c * C * A.di));
    } else {
        const int t = min(c * C + n, A.T - 1);
        ci.v = ld4<AL>(A.v + (unsigned)(t * A.di + 16 * w + 4 * g));
    }
    const unsigned sb = 4u * (unsigned)(c * R_SZ);
    ci.tr = buf_load4(R.rec, 16u * ((R_T >> 2) + lane), sb);
    ci.mr = buf_load4(R.rec, 16u * ((R_M >> 2) + lane), sb);
    ci.gm = buf_load4(R.rec, 16u * ((RV_GAM >> 2) + g), sb);
    ci.bg = buf_load4(R.rec, 16u * ((RV_BG >> 2) + g), sb);
    ci.gc = buf_load4(R.rec, 16u * ((RV_GC >> 2) + g), sb);
    ci.g15 = buf_load1(R.rec, 4u * (RV_GAM + 15), sb);
    ci.bn = buf_load1(R.rec, 4u * (RV_BET + n), sb);
}

template <bool AL>
ASCA_DEV void bchain_step(f32x4 (&X)[4], const BChainIn& ci, const float* __restrict__ sb, float* __restrict__ ho,
                          float* __restrict__ scr, int c, const BArgs& A, int w, int lane) {
    const int n = lane & 15, g = lane >> 4;
    const bool live = c * C + n < A.T;
    const float bt = ci.bn;
    const float g15 = ci.g15;
    const float4 gm = ci.gm, bg = ci.bg, gc = ci.gc;
    float4 kc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) kc[r] = *reinterpret_cast<const float4*>(sb + SB_K + n * RP + 16 * r + 4 * g);
    float dO[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) dO[j] = sb[SB_DO + (4 * g + j) * RP + 16 * w + n];
    f32x4 kx = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) kx = mfma4(el(kc[r], j), X[r][j], kx);
    f32x4 dU;
#pragma unroll
    for (int j = 0; j < 4; ++j) dU[j] = el(gc, j) * kx[j];
#pragma unroll
    for (int j = 0; j < 4; ++j) dU = mfma4(el(ci.mr, j), dO[j], dU);
    f32x4 Y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) Y = mfma4(el(ci.tr, j), dU[j], Y);
    // hand X (the gradient after this block) and Y over to the helpers
#pragma unroll
    for (int r = 0; r < 4; ++r)
        *reinterpret_cast<float4*>(ho + HO_DS + ((r * 4 + w) * 64 + lane) * 4) = tile_t(X[r], scr, lane);
    const float4 y4 = tile_t(Y, scr, lane);  // Y[n][16w + 4g ..]
    *reinterpret_cast<float4*>(ho + HO_Y + (w * 64 + lane) * 4) = y4;
    if (live) store4<AL>(A.gv + (unsigned)((c * C + n) * A.ldxi + 16 * w + 4 * g), f4scale(bt, y4));
    // the wave's shares of dO U^T and Y U^T, and of the row sums of Y o V
    const float4 do4 = *reinterpret_cast<const float4*>(sb + SB_DO + n * RP + 16 * w + 4 * g);
    const float4 u4 = *reinterpret_cast<const float4*>(sb + SB_U + n * RP + 16 * w + 4 * g);
    f32x4 pm = {0.f, 0.f, 0.f, 0.f}, pl = pm;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        pm = mfma4(el(do4, j), el(u4, j), pm);
        pl = mfma4(el(y4, j), el(u4, j), pl);
    }
    *reinterpret_cast<float4*>(ho + HO_DM + (w * 64 + lane) * 4) = make_float4(pm[0], pm[1], pm[2], pm[3]);
    *reinterpret_cast<float4*>(ho + HO_DL + (w * 64 + lane) * 4) = make_float4(pl[0], pl[1], pl[2], pl[3]);
    const float4 vv = live ? ci.v : make_float4(0.f, 0.f, 0.f, 0.f);
    float yv = y4.x * vv.x + y4.y * vv.y + y4.z * vv.z + y4.w * vv.w;
    yv = add_xor32(add_xor16(yv));
    if (lane < 16) ho[HO_YV + w * 16 + lane] = yv;
    // X <- gamma_15 X + Q^T (diag(gamma) dO) - K^T (diag(beta gamma) Y)
    float dOg[4], Yb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        dOg[j] = el(gm, j) * dO[j];
        Yb[j] = -el(bg, j) * Y[j];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        X[r] *= g15;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float qv = sb[SB_Q + (4 * g + j) * RP + 16 * r + n];
            const float kv = sb[SB_K + (4 * g + j) * RP + 16 * r + n];
            X[r] = mfma4(qv, dOg[j], X[r]);
            X[r] = mfma4(kv, Yb[j], X[r]);
        }
    }
}

struct BHelpIn {
    float4 sk[4];        // checkpoint before block c & ~1: S[16hw + n][16c + 4g ..], value tile c
    float gam, gcn, bt;  // gamma, Gamma[15][.], beta of step 16c + n
    float4 bb;           // beta of steps 4g .. 4g + 3
    float4 gq;           // block c - 1 (odd c): Gamma'[15][4i + g], i = 0..3
    float g15p;          // block c - 1: gamma'_15
    float qn, kn;        // norms of row 16c + n (1 for the raw gradients)
    float4 gr;           // Gamma of the block (accumulator layout)
};

template <bool FUSED>
ASCA_DEV void bhelp_load(BHelpIn& hi, int c, const BArgs& A, const BRes& R, int hw, int lane) {
    const int n = lane & 15, g = lane >> 4;
    const unsigned sc = 4u * (unsigned)((c >> 1) * DH2);
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) hi.sk[cc] = buf_load4(R.ck, 16u * ((hw * 4 + cc) * 64 + lane), sc);
    const unsigned sb = 4u * (unsigned)(c * R_SZ);
    hi.gam = buf_load1(R.rec, 4u * (RV_GAM + n), sb);
    hi.gcn = buf_load1(R.rec, 4u * (RV_GC + n), sb);
    hi.bt = buf_load1(R.rec, 4u * (RV_BET + n), sb);
    hi.bb = buf_load4(R.rec, 16u * ((RV_BET >> 2) + g), sb);
    const unsigned sp = 4u * (unsigned)(max(c - 1, 0) * R_SZ);  // block c - 1 is whole for odd c
    hi.gq = make_float4(buf_load1(R.rec, 4u * (RV_GC + g), sp), buf_load1(R.rec, 4u * (RV_GC + 4 + g), sp),
                        buf_load1(R.rec, 4u * (RV_GC + 8 + g), sp), buf_load1(R.rec, 4u * (RV_GC + 12 + g), sp));
    hi.g15p = buf_load1(R.rec, 4u * (RV_GAM + 15), sp);
    if constexpr (FUSED) {
        // rows past the sequence end read row T - 1 (their norms must stay finite)
        const unsigned t = (unsigned)min(c * C + n, A.T - 1);
        hi.qn = buf_load1(R.nq, 4u * t * (unsigned)A.H, 0u);
        hi.kn = buf_load1(R.nk, 4u * t * (unsigned)A.H, 0u);
    } else {
        hi.qn = 1.0f;
        hi.kn = 1.0f;
    }
    hi.gr = buf_load4(R.rec, 16u * ((R_G >> 2) + lane), sb);
}

ASCA_DEV float rowsum16(float x) { return group_sum<16>(x); }

// What a helper carries from the products of a block to its epilogue: dq, dk as
// row pieces (lane (g, n): row n, keys 16hw + 4g .. + 3), ready to store.
struct BCarry {
    f32x4 dq, dk;   // raw dq, dk
    float4 qr, kr;  // qhat, khat at the same places
    float rq, rk;   // 1 / |q|, 1 / |k| of row n
};

// The products of block c for the helper's keys 16hw .. 16hw + 15, computed
// transposed (keys as accumulator rows): lane (g, n) holds row n (step) and keys
// 16hw + 4g + r, so the per-step gate factors are the lane's own, the row sums
// over keys are in-register sums plus two lane swaps, and dq, dk leave without a
// transpose.
ASCA_DEV void bhelp_products(BCarry& cy, const BHelpIn& hi, const float* __restrict__ sb,
                             const float* __restrict__ sbp, const float* __restrict__ ho, float* __restrict__ ep,
                             float* __restrict__ scr, int c, const BArgs& A, int hw, int lane) {
    const int n = lane & 15, g = lane >> 4;
    const float bt = hi.bt, gam = hi.gam, gcn = hi.gcn;
    const float4 bb = hi.bb;                    // beta of rows 4g .. 4g + 3
    const float G[4] = {hi.gr.x, hi.gr.y, hi.gr.z, hi.gr.w};
    // The forward stores the state before every other block.  An odd block's
    // state follows from the block before (staged in `sbp`, always whole):
    // S = gamma'_15 S' + K'^T diag(Gamma'[15][:]) U', here for the helper's 16
    // keys (rows) as the transposed tiles of the checkpoint layout.
    float4 sk[4] = {hi.sk[0], hi.sk[1], hi.sk[2], hi.sk[3]};
    if (c & 1) {
        const float g15 = hi.g15p;
        const float4 gq = hi.gq;  // Gamma'[15][4i + g], i = 0..3
        float kg[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) kg[i] = el(gq, i) * sbp[SB_K + (4 * i + g) * RP + 16 * hw + n];
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            f32x4 t4 = {g15 * sk[cc].x, g15 * sk[cc].y, g15 * sk[cc].z, g15 * sk[cc].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) t4 = mfma4(sbp[SB_U + (4 * i + g) * RP + 16 * cc + n], kg[i], t4);
            sk[cc] = make_float4(t4[0], t4[1], t4[2], t4[3]);
        }
    }
    // (dO S^T)^T, (Y S^T)^T, (U X^T)^T: keys x steps, over all value columns
    f32x4 F = {0.f, 0.f, 0.f, 0.f}, Zt = F, D = F;
    float dss = 0.0f;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
        const float4 dO4 = *reinterpret_cast<const float4*>(sb + SB_DO + n * RP + 16 * cc + 4 * g);
        const float4 u4 = *reinterpret_cast<const float4*>(sb + SB_U + n * RP + 16 * cc + 4 * g);
        const float4 y4 = *reinterpret_cast<const float4*>(ho + HO_Y + (cc * 64 + lane) * 4);
        const float4 x4 = *reinterpret_cast<const float4*>(ho + HO_DS + ((hw * 4 + cc) * 64 + lane) * 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            F = mfma4(el(sk[cc], j), el(dO4, j), F);
            Zt = mfma4(el(sk[cc], j), el(y4, j), Zt);
            D = mfma4(el(x4, j), el(u4, j), D);
            dss += el(x4, j) * el(sk[cc], j);
        }
    }
    // dM = tril(dO U^T), dL = -strict_tril(Y U^T) from the chain waves' shares
    float4 pm = *reinterpret_cast<const float4*>(ho + HO_DM + lane * 4);
    float4 pl = *reinterpret_cast<const float4*>(ho + HO_DL + lane * 4);
#pragma unroll
    for (int w = 1; w < NW; ++w) {
        pm = f4add(pm, *reinterpret_cast<const float4*>(ho + HO_DM + (w * 64 + lane) * 4));
        pl = f4add(pl, *reinterpret_cast<const float4*>(ho + HO_DL + (w * 64 + lane) * 4));
    }
    f32x4 dM, dL, GdM, dA;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int t = 4 * g + j;
        dM[j] = n <= t ? el(pm, j) : 0.0f;
        dL[j] = n < t ? -el(pl, j) : 0.0f;
        GdM[j] = G[j] * dM[j];
        dA[j] = dL[j] * el(bb, j) * G[j];
    }
    float4 gdmt, dat;  // (Gamma o dM)[n][4g ..], dA[n][4g ..]
    tile_t2(GdM, dA, gdmt, dat, scr, lane);
    float kb[4], qb[4];  // K, Q[4g + j][16hw + n]
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        kb[j] = sb[SB_K + (4 * g + j) * RP + 16 * hw + n];
        qb[j] = sb[SB_Q + (4 * g + j) * RP + 16 * hw + n];
    }
    const float4 qr = *reinterpret_cast<const float4*>(sb + SB_Q + n * RP + 16 * hw + 4 * g);
    const float4 kr = *reinterpret_cast<const float4*>(sb + SB_K + n * RP + 16 * hw + 4 * g);
    // dq^T = gamma o F^T + K^T (Gamma o dM)^T,
    // dk^T = Gamma[15] o D^T - beta gamma o Zt^T + Q^T (Gamma o dM) + K^T (dA + dA^T)
    f32x4 dq, dk;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        dq[j] = gam * F[j];
        dk[j] = gcn * D[j] - bt * gam * Zt[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        dq = mfma4(kb[j], el(gdmt, j), dq);
        dk = mfma4(qb[j], GdM[j], dk);
        dk = mfma4(kb[j], dA[j] + el(dat, j), dk);
    }
    // row sums over the helper's keys: in-register, then over the four lanes of
    // row n (lane bits 4 and 5)
    float rs[5];
    rs[EP_RQ] = el(qr, 0) * dq[0];
    rs[EP_RK] = el(kr, 0) * dk[0];
    rs[EP_QF] = el(qr, 0) * F[0];
    rs[EP_ZK] = el(kr, 0) * Zt[0];
    rs[EP_KD] = el(kr, 0) * D[0];
#pragma unroll
    for (int j = 1; j < 4; ++j) {
        rs[EP_RQ] += el(qr, j) * dq[j];
        rs[EP_RK] += el(kr, j) * dk[j];
        rs[EP_QF] += el(qr, j) * F[j];
        rs[EP_ZK] += el(kr, j) * Zt[j];
        rs[EP_KD] += el(kr, j) * D[j];
    }
#pragma unroll
    for (int e = 0; e < 5; ++e) rs[e] = add_xor32(add_xor16(rs[e]));
    float* gs = A.gsc + (unsigned)(c * GS_SZ);
    if (lane < 16) {
        ep[(hw * 2 + EP_RQ) * 16 + n] = rs[EP_RQ];
        ep[(hw * 2 + EP_RK) * 16 + n] = rs[EP_RK];
#pragma unroll
        for (int e = EP_QF; e <= EP_KD; ++e) gs[GS_ROW + (hw * 3 + e - EP_QF) * 16 + n] = rs[e];
    }
    dss = wave_sum(dss);
    if (lane == 0) gs[GS_DSS + hw] = dss;
    if (hw == 0) {
        if (lane < 16) {
            float yv = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; ++w) yv += ho[HO_YV + w * 16 + lane];
            gs[GS_YV + lane] = yv;
        }
        *reinterpret_cast<float4*>(gs + GS_DM + 4 * lane) = make_float4(dM[0], dM[1], dM[2], dM[3]);
        *reinterpret_cast<float4*>(gs + GS_DL + 4 * lane) = make_float4(dL[0], dL[1], dL[2], dL[3]);
    }
    cy.dq = dq;
    cy.dk = dk;
    cy.qr = qr;
    cy.kr = kr;
    cy.rq = __builtin_amdgcn_rcpf(hi.qn);
    cy.rk = __builtin_amdgcn_rcpf(hi.kn);
}

template <bool FUSED, bool AL>
ASCA_DEV void bhelp_epilogue(const BCarry& cy, const float* __restrict__ ep, float* __restrict__ scr, int c,
                             const BArgs& A, int hw, int lane) {
    const int n = lane & 15, g = lane >> 4;
    f32x4 dq = cy.dq, dk = cy.dk;
    if constexpr (FUSED) {
        float dotq = ep[EP_RQ * 16 + n], dotk = ep[EP_RK * 16 + n];
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            dotq += ep[(w * 2 + EP_RQ) * 16 + n];
            dotk += ep[(w * 2 + EP_RK) * 16 + n];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            dq[j] = (dq[j] - el(cy.qr, j) * dotq) * cy.rq;
            dk[j] = (dk[j] - el(cy.kr, j) * dotk) * cy.rk;
        }
    }
    if (c * C + n < A.T) {
        const unsigned o = (unsigned)((c * C + n) * A.ldxi + 16 * hw + 4 * g);
        store4<AL>(A.gq + o, make_float4(dq[0], dq[1], dq[2], dq[3]));
        store4<AL>(A.gk + o, make_float4(dk[0], dk[1], dk[2], dk[3]));
    }
}

// Gate gradients of block c (dalpha, dbeta and their sigmoid backward), run by
// one wave from the sums the helpers left in the scratch (loaded with the
// block's record, one block ahead); lane t of each row is step t.
struct BGateIn {
    float4 ar, bq, gr;  // K K^T, Q K^T, Gamma of the block (accumulator layout)
    float a, b;         // gates of step 16c + n (as loaded, for the sigmoid backward)
    float gam, bm;      // gamma, beta of step 16c + n (beta 0 past the sequence end)
    float4 bb;          // beta of steps 4g .. 4g + 3 (0 past the sequence end)
    float4 pm, pl;      // dM, dL (accumulator layout)
    float rw[3][NW];    // the helpers' row sums q.F, k.Zt, k.D of row n
    float ds[NW];       // the helpers' <X, S>
    float yv;           // row sum of Y o V of row n
};

ASCA_DEV void bgate_load(BGateIn& gi, int c, const BArgs& A, int lane) {
    const float4* rq = reinterpret_cast<const float4*>(A.rec + (unsigned)(c * R_SZ));
    gi.ar = rq[(R_A >> 2) + lane];
    gi.bq = rq[(R_BQ >> 2) + lane];
    gi.gr = rq[(R_G >> 2) + lane];
    const int t = min(c * C + (lane & 15), A.T - 1);
    gi.a = A.alpha[(unsigned)(t * A.H)];
    gi.b = A.beta[(unsigned)(t * A.H)];
    const int n = lane & 15;
    const float* rb = A.rec + (unsigned)(c * R_SZ);
    gi.gam = rb[RV_GAM + n];
    gi.bm = rb[RV_BET + n];
    gi.bb = rq[(RV_BET >> 2) + (lane >> 4)];
    const float* gs = A.gsc + (unsigned)(c * GS_SZ);
    gi.pm = *reinterpret_cast<const float4*>(gs + GS_DM + 4 * lane);
    gi.pl = *reinterpret_cast<const float4*>(gs + GS_DL + 4 * lane);
#pragma unroll
    for (int w = 0; w < NW; ++w) {
#pragma unroll
        for (int e = 0; e < 3; ++e) gi.rw[e][w] = gs[GS_ROW + (w * 3 + e) * 16 + n];
        gi.ds[w] = gs[GS_DSS + w];
    }
    gi.yv = gs[GS_YV + n];
}

// The gate gradients of NB blocks at once (block cs[i] from gin[i]): every
// phase runs over all NB blocks before the next, so their dependency chains
// interleave and the LDS transposes share their wave syncs.  scr holds NB
// areas of WSCR floats.  Blocks past the sequence end (clamped loads) store
// nothing: their rows lie outside the resources' range.
template <bool FUSED, int NB>
ASCA_DEV void bgate_batch(const BGateIn (&gin)[NB], const int (&cs)[NB], float* __restrict__ scr,
                          const BArgs& A, Rsrc rga, Rsrc rgb, int lane) {
    const int n = lane & 15, g = lane >> 4;
    float szk[NB], dgam[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const BGateIn& gi = gin[i];
        float sqf = 0.f, dss = 0.f;
        szk[i] = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            sqf += gi.rw[0][w];
            szk[i] += gi.rw[1][w];
            dss += gi.ds[w];
        }
        dgam[i] = -gi.bm * szk[i] + sqf + (n == C - 1 ? dss : 0.0f);
        scr[i * WSCR + SVO + 16 * g + n] = dgam[i];   // every lane: row n of copy g
    }
    wave_sync();
    float4 dg4[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) dg4[i] = *reinterpret_cast<const float4*>(scr + i * WSCR + SVO + 4 * g);
    wave_sync();
    // dGamma (strict lower part), row sums of dL o Gamma o A, the first term of dalpha
    f32x4 dgs[NB];
    float t1[NB], rb[NB][4];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const BGateIn& gi = gin[i];
        float skd = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) skd += gi.rw[2][w];
        t1[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = 4 * g + j;
            const float dL = el(gi.pl, j), G = el(gi.gr, j);
            rb[i][j] = rowsum16(dL * G * el(gi.ar, j));
            dgs[i][j] = n < t ? el(gi.pm, j) * el(gi.bq, j) + dL * el(gi.bb, j) * el(gi.ar, j) +
                                    (t == C - 1 ? skd : 0.0f)
                              : 0.0f;
            t1[i] += G * el(dg4[i], j);
        }
        t1[i] = add_xor32(add_xor16(t1[i]));
    }
    // R = dGs Gamma'^T with Gamma'[m][i] = Gamma[m-1][i] (the row above, zero for
    // m = 0) on the matrix cores, then sum_t Gamma[t][m] R[t][m]
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        float* st = scr + i * WSCR;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            st[(4 * g + j) * OTP + n] = dgs[i][j];
            st[C * OTP + (4 * g + j) * OTP + n] = el(gin[i].gr, j);
        }
        *reinterpret_cast<float4*>(st + SVO + 64 + 4 * g) = make_float4(rb[i][0], rb[i][1], rb[i][2], rb[i][3]);
    }
    wave_sync();
    float dal[NB], dbe[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const float* st = scr + i * WSCR;
        const float4 dgst = *reinterpret_cast<const float4*>(st + n * OTP + 4 * g);       // dGs[n][4g ..]
        const float4 gt = *reinterpret_cast<const float4*>(st + C * OTP + n * OTP + 4 * g);  // Gamma[n][4g ..]
        const float gp[4] = {dpp_or<0x111>(0.0f, gt.x), dpp_or<0x111>(0.0f, gt.y), dpp_or<0x111>(0.0f, gt.z),
                             dpp_or<0x111>(0.0f, gt.w)};   // Gamma[n-1][4g ..]
        f32x4 R = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) R = mfma4(el(dgst, j), gp[j], R);
        float t2 = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) t2 += el(gin[i].gr, j) * R[j];
        t2 = add_xor32(add_xor16(t2));
        const float gprev = dpp_or<0x111>(1.0f, gin[i].gam);   // gamma_{n-1}
        dal[i] = gprev * t1[i] + t2;
        // dbeta of step n: Y.V - gamma Z'.K + sum_l dL Gamma A (row n's sum from lane (n/4, .))
        const float rbn = st[SVO + 64 + n];
        dbe[i] = gin[i].yv - gin[i].gam * szk[i] + rbn;
    }
    wave_sync();
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        // every lane stores (the four lanes of row n hold the same values); rows
        // past the sequence end fall outside the resources and are dropped
        const unsigned r = 4u * (unsigned)((cs[i] * C + n) * A.ldgi);
        const float a = gin[i].a, b = gin[i].b;
        buf_store1(rga, r, FUSED ? dal[i] * a * (1.0f - a) : dal[i]);
        buf_store1(rgb, r, FUSED ? dbe[i] * b * (1.0f - b) : dbe[i]);
    }
}

// A helper's staging of block c: rows 4hw .. 4hw + 3 of k, q, dO and u, one
// 16-byte load per matrix and lane (row 4hw + lane/16, columns 4 (lane%16) ..);
// rows past the sequence end are zero.
struct BStage {
    float4 x[4];
};

template <bool AL>
ASCA_DEV void bstage_load(BStage& st, int c, const BArgs& A, const BRes& R, int hw, int lane) {
    const int j = lane & 15, r = 4 * hw + (lane >> 4);   // row c C + r of the block, columns 4 j ..
    if constexpr (AL) {
        // rows past the sequence end load as 0 (outside the row resources)
        const unsigned vo = 4u * (unsigned)(r * A.di + 4 * j), so = 4u * (unsigned)(c * C * A.di);
        st.x[0] = buf_load4(R.k, vo, so);
        st.x[1] = buf_load4(R.q, vo, so);
        st.x[2] = buf_load4(R.dO, vo, so);
        // u in the forward's tile layout: tile of columns 16 (j / 4), row r, columns 4 (j % 4) ..
        st.x[3] = buf_load4(R.u, 4u * (unsigned)((j >> 2) * 256 + r * 16 + 4 * (j & 3)), 4u * (unsigned)(c * U_BLK));
        return;
    }
    const int t = min(c * C + r, A.T - 1);
    const unsigned off = (unsigned)(t * A.di + 4 * (lane & 15));
    st.x[0] = ld4<AL>(A.k + off);
    st.x[1] = ld4<AL>(A.q + off);
    st.x[2] = ld4<AL>(A.d_o + off);
    // u (the workspace: aligned) as above, from row t % 16 of block t / 16
    st.x[3] = *reinterpret_cast<const float4*>(A.u + (unsigned)((t >> 4) * U_BLK + (j >> 2) * 256 + (t & 15) * 16 +
                                                                4 * (j & 3)));
}

// WHOLE: the caller knows block c is whole (every block but the last is).
template <bool WHOLE>
ASCA_DEV void bstage_store(const BStage& st, int c, float* __restrict__ sb, int T, int hw, int lane) {
    const int row = 4 * hw + (lane >> 4);
    float* dst = sb + row * RP + 4 * (lane & 15);
    if (WHOLE || (c + 1) * C <= T) {  // a whole block (uniform): the loaded registers go straight out
#pragma unroll
        for (int m = 0; m < 4; ++m) *reinterpret_cast<float4*>(dst + m * SB_MAT) = st.x[m];
    } else {
        const bool live = c * C + row < T;
#pragma unroll
        for (int m = 0; m < 4; ++m)
            *reinterpret_cast<float4*>(dst + m * SB_MAT) = live ? st.x[m] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// After the block loop: the gate gradients of every block, block c on wave
// c mod 8, four blocks of a wave at a time; the loop's LDS is free by then
// (the block's final barrier) and gives each wave four scratch areas.
template <bool FUSED>
ASCA_DEV void bgate_tail(const BArgs& A, float* __restrict__ lds, int w, int lane) {
    constexpr int NB = 4;
    __syncthreads();   // the scratch writes of every wave are visible, the loop's LDS is free
    float* scr = lds + w * NB * WSCR;
    // the unit's rows of dalpha, dbeta: row t at t * ldg
    const unsigned gbytes = 4u * (unsigned)((A.T - 1) * A.ldgi + 1);
    const Rsrc rga = make_rsrc(A.ga, gbytes), rgb = make_rsrc(A.gb, gbytes);
    for (int c0 = w; c0 < A.NC; c0 += 2 * NW * NB) {
        BGateIn gin[NB];
        int cs[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            cs[i] = c0 + 2 * NW * i;                 // past NC: rows beyond T, stores dropped
            bgate_load(gin[i], min(cs[i], A.NC - 1), A, lane);
        }
        bgate_batch<FUSED, NB>(gin, cs, scr, A, rga, rgb, lane);
    }
}

template <bool FUSED, bool AL>
__global__ __launch_bounds__(2 * NT) void ut_bwd64_k(BArgs A) {
    extern __shared__ float lds[];
    {
        A.unit = blockIdx.x;  // h*B + b
        A.h = A.unit / A.B;
        const int b = A.unit - A.h * A.B;
        const long ubase = (long)b * A.T * A.d + (long)A.h * DH;
        const long gbase = (long)b * A.T * A.H + A.h;
        const long rowbase = (long)b * A.T;
        // every pointer rebased on the unit: the per-block offsets are 32-bit
        A.q += ubase; A.k += ubase; A.v += ubase; A.d_o += ubase; A.u += (long)A.unit * A.NC * U_BLK;
        A.alpha += gbase; A.beta += gbase;
        if (A.qn) { A.qn += gbase; A.kn += gbase; }
        A.ckpt += (long)A.unit * A.nslots * DH2;
        A.rec += (long)A.unit * A.NC * R_SZ;
        A.gsc += (long)A.unit * A.NC * GS_SZ;
        A.gq += rowbase * A.ldx + (long)A.h * DH; A.gk += rowbase * A.ldx + (long)A.h * DH;
        A.gv += rowbase * A.ldx + (long)A.h * DH;
        A.ga += rowbase * A.ldg + A.h; A.gb += rowbase * A.ldg + A.h;
        A.ubase = 0; A.gbase = 0; A.rowbase = 0;
    }
    // the wave index, uniform in a scalar register (so are the block indices and
    // buffer offsets derived from it)
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int NC = A.NC;
    const BRes R = bres_make(A);
    float* scr = lds + B_SCR + w * WSCR;
    if (w >= NW) {
        // helper: step s runs the epilogue of block NC + 1 - s and the products
        // of block NC - s (the chain waves stage the rows).  Every global load is
        // made two steps ahead into buffer s & 1, unconditionally (clamped block
        // indices), and consumed at the start of its step, so no wait falls on a
        // recent memory operation.
        const int hw = w - NW;
        BHelpIn hin[2];
        BCarry cy;
        {
            BStage st0;
            bstage_load<AL>(st0, NC - 1, A, R, hw, lane);
            bstage_store<false>(st0, NC - 1, lds + B_STG + ((NC - 1) % NSB) * SB_BUF, A.T, hw, lane);
        }
        bhelp_load<FUSED>(hin[1], NC - 1, A, R, hw, lane);
        bhelp_load<FUSED>(hin[0], max(NC - 2, 0), A, R, hw, lane);
        lds_barrier();
        lds_barrier();  // step 0: the chain's first block
        // steps 1 .. NC: the products of block cp = NC - s on every path (the
        // carried dq, dk are then never copied), the epilogue of cp + 1 from
        // step 2 on; step NC + 1: the epilogue of block 0
        auto step = [&](int s, BHelpIn& hb) {
            const int cp = NC - s;
            if (s >= 2) bhelp_epilogue<FUSED, AL>(cy, lds + B_EP + ((cp + 1) & 1) * EP_SZ, scr, cp + 1, A, hw, lane);
            bhelp_products(cy, hb, lds + B_STG + (cp % NSB) * SB_BUF, lds + B_STG + ((cp + NSB - 1) % NSB) * SB_BUF,
                           lds + B_HO + (cp & 1) * HO_SZ, lds + B_EP + (cp & 1) * EP_SZ, scr, cp, A, hw, lane);
            bhelp_load<FUSED>(hb, max(cp - 2, 0), A, R, hw, lane);
            lds_barrier();
        };
        for (int s = 1; s <= NC; s += 2) {
            step(s, hin[1]);
            if (s + 1 <= NC) step(s + 1, hin[0]);
        }
        bhelp_epilogue<FUSED, AL>(cy, lds + B_EP, scr, 0, A, hw, lane);
        lds_barrier();
        bgate_tail<FUSED>(A, lds, w, lane);
        return;
    }
    // chain: step s runs block NC - 1 - s and stages rows 4w .. 4w + 3 of the
    // block after (NC - 2 - s) into its buffer, which no wave reads in step s
    f32x4 X[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) X[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    BChainIn cb[2];
    BStage sg[2];
    bchain_load<AL>(cb[0], NC - 1, A, R, w, lane);
    bchain_load<AL>(cb[1], max(NC - 2, 0), A, R, w, lane);
    bstage_load<AL>(sg[0], max(NC - 2, 0), A, R, w, lane);
    bstage_load<AL>(sg[1], max(NC - 3, 0), A, R, w, lane);
    lds_barrier();
    for (int s = 0; s < NC; ++s) {
        const int c = NC - 1 - s;
        // the chain's inputs are loaded two steps ahead into buffer s & 1
        // (static indices: no register copies; X is updated on every path)
        if ((s & 1) == 0) {
            // block c - 1 < NC - 1 is whole (only the last block can be partial)
            if (c >= 1) bstage_store<true>(sg[0], c - 1, lds + B_STG + ((c - 1) % NSB) * SB_BUF, A.T, w, lane);
            bchain_step<AL>(X, cb[0], lds + B_STG + (c % NSB) * SB_BUF, lds + B_HO + (c & 1) * HO_SZ, scr, c, A, w,
                            lane);
            bchain_load<AL>(cb[0], max(c - 2, 0), A, R, w, lane);
            bstage_load<AL>(sg[0], max(c - 3, 0), A, R, w, lane);
        } else {
            // block c - 1 < NC - 1 is whole (only the last block can be partial)
            if (c >= 1) bstage_store<true>(sg[1], c - 1, lds + B_STG + ((c - 1) % NSB) * SB_BUF, A.T, w, lane);
            bchain_step<AL>(X, cb[1], lds + B_STG + (c % NSB) * SB_BUF, lds + B_HO + (c & 1) * HO_SZ, scr, c, A, w,
                            lane);
            bchain_load<AL>(cb[1], max(c - 2, 0), A, R, w, lane);
            bstage_load<AL>(sg[1], max(c - 3, 0), A, R, w, lane);
        }
        lds_barrier();
    }
    // the helpers' last two steps (products of block 0, then its epilogue)
    lds_barrier();
    lds_barrier();
    bgate_tail<FUSED>(A, lds, w, lane);
}

}  // namespace ut64

static bool ut_aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <bool AL>
static int launch_ut_fwd64_t(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                             float* o, const DeltaWs& ws, int B, int T, int H, hipStream_t st) {
    const int units = B * H;
    const size_t lds = ut64::F_LDS;
    if (int arc = allow_lds(reinterpret_cast<const void*>(&ut64::ut_fwd64_k<AL>), ut64::F_LDS)) return arc;
    int rc = pre_launch("ut_fwd64");
    if (rc) return rc;
    hipLaunchKernelGGL(ut64::ut_fwd64_k<AL>, dim3(units), dim3(2 * ut64::NT), lds, st, q, k, v, alpha, beta, o, ws.sk,
                       ws.ckpt, ws.rec, B, T, H, ws.nslots);
    return post_launch("ut_fwd64");
}

// Floats of the backward's gate-sum scratch (ut64::BArgs::gsc).
inline size_t ut_bwd64_scratch_floats(int units, int NC) { return (size_t)units * NC * ut64::GS_SZ; }

template <bool FUSED, bool AL>
static int launch_ut_bwd64_t(const ut64::BArgs& a, int units, hipStream_t st) {
    if (int arc = allow_lds(reinterpret_cast<const void*>(&ut64::ut_bwd64_k<FUSED, AL>), ut64::B_LDS)) return arc;
    int rc = pre_launch("ut_bwd64");
    if (rc) return rc;
    hipLaunchKernelGGL((ut64::ut_bwd64_k<FUSED, AL>), dim3(units), dim3(2 * ut64::NT), ut64::B_LDS, st, a);
    return post_launch("ut_bwd64");
}

// The backward variants other than fused on aligned rows (delta_ut64_b.hip).
int launch_ut_bwd64_other(const ut64::BArgs& a, int units, bool fused, bool al, hipStream_t st);

}  // namespace asca
