// Gated delta rule, recurrent form, f32, for gfx950.
//
// Math (per sequence b, head h; S is dh x dh, S_0 = 0), as in
// rust/src/delta.rs:1-14 and DeltaBlock::scan_cpu (rust/src/delta.rs:244-334):
//   sk_t = S_{t-1}^T k_t,  u_t = beta_t (v_t - alpha_t sk_t),
//   S_t  = alpha_t S_{t-1} + k_t u_t^T,  o_t = S_t^T q_t.
//
// Design (MI355X-first, not a translation of rust/kernels/asca.cu):
//  * Column i of S only ever meets k, q, alpha, beta and its own v_i, sk_i, u_i,
//    so the forward splits each (sequence, head) unit into dh/16 independent
//    waves of 16 value columns.  Inside a wave, lane = 4*column + part; a lane
//    keeps dh/4 rows of its column in VGPRs and S^T k, S^T q are 4-lane DPP
//    butterflies.  No LDS, no barrier in the forward.  The step loop is
//    straight-line (unrolled per checkpoint chunk): inputs are prefetched PF
//    steps ahead into registers, the gates of a chunk arrive as one lane-
//    distributed load and are broadcast with v_readlane, and masked lanes store
//    into a trash buffer instead of branching, so every wait is exact.
//  * The forward stores S every C steps ("checkpoints", C = 8 at dh = 64, laid
//    out as S^T so each lane writes 16-byte vectors) and the per-step sk vector,
//    instead of the reference's full (T+1) dh^2 history (2.15 GB at B32 T512 H8
//    dh64).
//  * The backward walks C-step segments in reverse.  Each segment's inputs are
//    staged in LDS (loaded one segment ahead), the segment is recomputed from its
//    checkpoint into an LDS stash, then processed backwards.  A lane owns a
//    (dh/16) x 4 tile: du = dS^T k is a 16-lane DPP butterfly inside a row,
//    the column sums of dq and dk are transposed permlane32/permlane16 swaps
//    plus a per-segment cross-wave sum through LDS, where the L2-norm and
//    sigmoid backward of the drop-in variant also run.
#include "common.h"
#include "runtime.h"

namespace asca {

template <int DH>
struct DS {
    static constexpr int W = DH / 16;        // waves per unit, 16 value columns each
    static constexpr int THREADS = 64 * W;
    static constexpr int R = DH / 4;         // forward: rows per lane (4 lanes / column)
    static constexpr int M = DH / 16;        // backward: rows per lane (16 row groups)
    // Checkpoint interval: C states of the backward's LDS stash stay <= 128 KB.
    static constexpr int CK = (DH <= 32) ? 16 : (DH == 64) ? 8 : 2;
    static constexpr int PF = (DH == 128) ? 2 : 4;   // forward prefetch depth (steps)
    // backward LDS layout (floats unless noted)
    static constexpr int STASH_F4 = CK * W * M * 64;  // float4
    static constexpr int RED_F = CK * W * DH;         // dq / dk column sums per wave
    static constexpr int RAB_F = CK * W * 2;          // dalpha / dbeta per wave
    static constexpr int STQK_F = CK * DH;            // staged q (and k) rows
    static constexpr int STW_F = W * CK * 48;         // staged dO, v, sk per wave
    static constexpr int STAB_F = 2 * CK;             // staged alpha, beta
    static constexpr size_t LDS_BWD =
        (size_t)STASH_F4 * 16 + (size_t)(2 * RED_F + RAB_F + 2 * STQK_F + STW_F + STAB_F) * 4;
};

// Sink for the stores of masked-off lanes, so stores never need a branch.
__device__ float4 g_trash4[1024];

ASCA_DEV float* trash_f(int i) { return reinterpret_cast<float*>(g_trash4) + (i & 4095); }
ASCA_DEV float4* trash_f4(int i) { return g_trash4 + (i & 1023); }

ASCA_DEV float readlane_f(float x, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l)); }

// Masked vector helpers: invalid elements read 0 from a valid address.
template <bool EXACT>
ASCA_DEV float4 ld4m(const float* __restrict__ p, int col, int dh) {
    if constexpr (EXACT) {
        return *reinterpret_cast<const float4*>(p + col);
    } else {
        float4 r;
        float* rr = reinterpret_cast<float*>(&r);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const bool ok = col + e < dh;
            const float x = p[ok ? col + e : 0];
            rr[e] = ok ? x : 0.0f;
        }
        return r;
    }
}

// ------------------------------------------------------------------ forward

template <int DH, bool EXACT>
ASCA_DEV void fwd_load(float (&kk)[DH / 4], float (&qq)[DH / 4], float& vv, const float* __restrict__ kt,
                       const float* __restrict__ qt, const float* __restrict__ vt, int row0, int col, int dh) {
    constexpr int R = DH / 4;
    if constexpr (EXACT) {
#pragma unroll
        for (int j = 0; j < R; j += 4) {
            const float4 a = *reinterpret_cast<const float4*>(kt + row0 + j);
            const float4 c = *reinterpret_cast<const float4*>(qt + row0 + j);
            kk[j] = a.x; kk[j + 1] = a.y; kk[j + 2] = a.z; kk[j + 3] = a.w;
            qq[j] = c.x; qq[j + 1] = c.y; qq[j + 2] = c.z; qq[j + 3] = c.w;
        }
        vv = vt[col];
    } else {
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const bool ok = row0 + j < dh;
            const float a = kt[ok ? row0 + j : 0];
            const float c = qt[ok ? row0 + j : 0];
            kk[j] = ok ? a : 0.0f;
            qq[j] = ok ? c : 0.0f;
        }
        const bool okc = col < dh;
        const float x = vt[okc ? col : 0];
        vv = okc ? x : 0.0f;
    }
}

// One block per (sequence, head) unit, unit = h*B + b (the reference's s_pre
// order, rust/src/delta.rs:54-56).  ckpt: nslots = ceil(T/CK) states per unit,
// slot j = S^T before step j*CK (element (a, i) of S at [i*dh + a]).
template <int DH, bool EXACT>
__global__ __launch_bounds__(DS<DH>::THREADS) void delta_fwd_k(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ alpha, const float* __restrict__ beta, float* __restrict__ o,
    float* __restrict__ sk_out, float* __restrict__ ckpt, int B, int T, int H, int dh, int nslots) {
    using S = DS<DH>;
    constexpr int R = S::R, CK = S::CK, PF = S::PF;
    static_assert(CK % PF == 0 && 2 * CK <= 64, "chunk layout");
    const int unit = blockIdx.x;
    const int h = unit / B, b = unit - h * B;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int p = lane & 3, c = lane >> 2;
    const int col = w * 16 + c;
    const int row0 = p * R;
    const long d = (long)H * dh;
    const long dh2 = (long)dh * dh;
    const long ubase = (long)b * T * d + (long)h * dh;
    const float* qb = q + ubase;
    const float* kb = k + ubase;
    const float* vb = v + ubase;
    float* ob = o + ubase;
    float* skb = sk_out + ubase;
    const long gbase = (long)b * T * H + h;
    float* ckb = ckpt + (long)unit * nslots * dh2;
    const bool col_ok = EXACT || col < dh;
    float* const tr = trash_f(threadIdx.x);

    // gates of chunk t0: lane l < CK holds alpha of step t0+l, CK <= l < 2CK beta of t0+l-CK
    const int gl = lane & (2 * CK - 1);
    const float* gsrc = (gl < CK ? alpha : beta) + gbase;
    const int gstep = gl % CK;

    float s[R];
#pragma unroll
    for (int j = 0; j < R; ++j) s[j] = 0.0f;

    float kk[PF][R], qq[PF][R], vv[PF];
#pragma unroll
    for (int i = 0; i < PF - 1; ++i) {
        const long t = min(i, T - 1);
        fwd_load<DH, EXACT>(kk[i], qq[i], vv[i], kb + t * d, qb + t * d, vb + t * d, row0, col, dh);
    }
    float gnext = gsrc[(long)min(gstep, T - 1) * H];

    for (int t0 = 0; t0 < T; t0 += CK) {
        const float gcur = gnext;
        gnext = gsrc[(long)min(t0 + CK + gstep, T - 1) * H];
        {   // checkpoint: S before step t0, as S^T
            float* dst = ckb + (long)(t0 / CK) * dh2 + (long)col * dh + row0;
            if constexpr (EXACT) {
#pragma unroll
                for (int j = 0; j < R; j += 4)
                    *reinterpret_cast<float4*>(dst + j) = make_float4(s[j], s[j + 1], s[j + 2], s[j + 3]);
            } else {
#pragma unroll
                for (int j = 0; j < R; ++j) *((col_ok && row0 + j < dh) ? dst + j : tr) = s[j];
            }
        }
#pragma unroll
        for (int jj = 0; jj < CK; ++jj) {
            const int t = t0 + jj;
            {
                const int ls = (jj + PF - 1) % PF;
                const long tl = min(t + PF - 1, T - 1);
                fwd_load<DH, EXACT>(kk[ls], qq[ls], vv[ls], kb + tl * d, qb + tl * d, vb + tl * d, row0, col, dh);
            }
            const int cs = jj % PF;
            const float a = readlane_f(gcur, jj);
            const float bt = readlane_f(gcur, CK + jj);
            float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
            for (int j = 0; j < R; j += 2) {
                a0 = fmaf(s[j], kk[cs][j], a0);
                a1 = fmaf(s[j + 1], kk[cs][j + 1], a1);
            }
            const float sk = group_sum<4>(a0 + a1);
            const float u = bt * (vv[cs] - a * sk);
            float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
            for (int j = 0; j < R; j += 2) {
                s[j] = a * s[j] + kk[cs][j] * u;
                s[j + 1] = a * s[j + 1] + kk[cs][j + 1] * u;
                o0 = fmaf(s[j], qq[cs][j], o0);
                o1 = fmaf(s[j + 1], qq[cs][j + 1], o1);
            }
            const float oo = group_sum<4>(o0 + o1);
            const bool tv = t < T && col_ok;
            *((p == 0 && tv) ? ob + (long)t * d + col : tr) = oo;
            *((p == 1 && tv) ? skb + (long)t * d + col : tr) = sk;
        }
    }
}

// Full state history for download_states: S before every step then the final
// state, row-major S[a][i], unit h*B + b, (T+1) dh^2 floats per unit.  Same
// arithmetic as delta_fwd_k; a diagnostic path, not tuned.
template <int DH>
__global__ __launch_bounds__(DS<DH>::THREADS) void delta_states_k(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ alpha, const float* __restrict__ beta, float* __restrict__ states, int B, int T,
    int H, int dh) {
    constexpr int R = DS<DH>::R;
    const int unit = blockIdx.x;
    const int h = unit / B, b = unit - h * B;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int p = lane & 3, c = lane >> 2;
    const int col = w * 16 + c;
    const int row0 = p * R;
    const long d = (long)H * dh;
    const long dh2 = (long)dh * dh;
    const long ubase = (long)b * T * d + (long)h * dh;
    float* st = states + (long)unit * (T + 1) * dh2;
    float s[R];
#pragma unroll
    for (int j = 0; j < R; ++j) s[j] = 0.0f;
    for (int t = 0; t <= T; ++t) {
#pragma unroll
        for (int j = 0; j < R; ++j)
            if (col < dh && row0 + j < dh) st[(long)t * dh2 + (long)(row0 + j) * dh + col] = s[j];
        if (t == T) break;
        float kk[R], qq[R], vv;
        fwd_load<DH, false>(kk, qq, vv, k + ubase + (long)t * d, q + ubase + (long)t * d, v + ubase + (long)t * d,
                            row0, col, dh);
        const float a = alpha[(long)b * T * H + (long)t * H + h];
        const float bt = beta[(long)b * T * H + (long)t * H + h];
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int j = 0; j < R; j += 2) {
            a0 = fmaf(s[j], kk[j], a0);
            a1 = fmaf(s[j + 1], kk[j + 1], a1);
        }
        const float sk = group_sum<4>(a0 + a1);
        const float u = bt * (vv - a * sk);
#pragma unroll
        for (int j = 0; j < R; ++j) s[j] = a * s[j] + kk[j] * u;
    }
}

// ----------------------------------------------------------------- backward

// Per-step operands of the reverse walk, read from LDS: the stash tile of
// S_{t-1} (rows rowb..rowb+M-1, columns colb..colb+3), q and k rows, the dO, v
// and sk column quads and the two gates.
template <int M>
struct BOps {
    float4 s[M];
    float q[M], k[M];
    float4 dO, v, sk;
    float a, b;
};

template <int DH>
ASCA_DEV void lds_ops(BOps<DH / 16>& o, const float4* __restrict__ stash, const float* __restrict__ st_q,
                      const float* __restrict__ st_k, const float* __restrict__ st_w,
                      const float* __restrict__ st_ab, int j, int w, int lane, int rowb, int cg) {
    constexpr int M = DS<DH>::M, W = DS<DH>::W, CK = DS<DH>::CK;
#pragma unroll
    for (int m = 0; m < M; ++m) o.s[m] = stash[((j * W + w) * M + m) * 64 + lane];
    if constexpr (M % 4 == 0) {
#pragma unroll
        for (int m = 0; m < M; m += 4) {
            const float4 x = *reinterpret_cast<const float4*>(st_q + j * DH + rowb + m);
            const float4 y = *reinterpret_cast<const float4*>(st_k + j * DH + rowb + m);
            o.q[m] = x.x; o.q[m + 1] = x.y; o.q[m + 2] = x.z; o.q[m + 3] = x.w;
            o.k[m] = y.x; o.k[m + 1] = y.y; o.k[m + 2] = y.z; o.k[m + 3] = y.w;
        }
    } else {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            o.q[m] = st_q[j * DH + rowb + m];
            o.k[m] = st_k[j * DH + rowb + m];
        }
    }
    const float* sw = st_w + (w * CK + j) * 48 + cg * 4;
    o.dO = *reinterpret_cast<const float4*>(sw);
    o.v = *reinterpret_cast<const float4*>(sw + 16);
    o.sk = *reinterpret_cast<const float4*>(sw + 32);
    o.a = st_ab[j];
    o.b = st_ab[CK + j];
}

// One reverse step of the BPTT for this lane's tile (rust/src/delta.rs:485-572
// reorganised per value column; see the file header).  Updates ds in place,
// stores dv, and leaves the dq / dk row sums and the dalpha / dbeta totals of
// this wave in LDS for the epilogue.
template <int DH, bool EXACT>
ASCA_DEV void bwd_step(const BOps<DH / 16>& in, float (&ds)[DH / 16][4], float* __restrict__ red_q,
                       float* __restrict__ red_k, float* __restrict__ red_ab, float* __restrict__ dv_dst,
                       float* __restrict__ tr, int jj, int w, int lane, int rg, int cg, int rowb, int colb,
                       int dh) {
    constexpr int M = DS<DH>::M, W = DS<DH>::W;
    float sm[M][4];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        sm[m][0] = in.s[m].x; sm[m][1] = in.s[m].y; sm[m][2] = in.s[m].z; sm[m][3] = in.s[m].w;
    }
    const float a = in.a, bb = in.b;
    const float dO[4] = {in.dO.x, in.dO.y, in.dO.z, in.dO.w};
    const float vv[4] = {in.v.x, in.v.y, in.v.z, in.v.w};
    const float sk[4] = {in.sk.x, in.sk.y, in.sk.z, in.sk.w};

    // dS += q dO^T  (delta.rs:508-511)
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int n = 0; n < 4; ++n) ds[m][n] = fmaf(in.q[m], dO[n], ds[m][n]);
    // du = dS^T k  (delta.rs:536-542): 16-lane butterfly over row groups
    float du[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
        float acc = 0.0f;
#pragma unroll
        for (int m = 0; m < M; ++m) acc = fmaf(ds[m][n], in.k[m], acc);
        du[n] = group_sum<16>(acc);
    }
    float wv[4], u[4], dsk[4];
    const float c1 = -bb * a;
#pragma unroll
    for (int n = 0; n < 4; ++n) {
        wv[n] = vv[n] - a * sk[n];
        u[n] = bb * wv[n];
        dsk[n] = c1 * du[n];
    }
    // dv = beta du  (delta.rs:550), stored by the lanes of row group 0
    if constexpr (EXACT) {
        *(rg == 0 ? reinterpret_cast<float4*>(dv_dst) : reinterpret_cast<float4*>(tr)) =
            make_float4(bb * du[0], bb * du[1], bb * du[2], bb * du[3]);
    } else {
#pragma unroll
        for (int n = 0; n < 4; ++n) *((rg == 0 && colb + n < dh) ? dv_dst + n : tr + n) = bb * du[n];
    }

    // Off-critical-path partial sums over this lane's 4 columns.
    //   dq = S_t dO = alpha S_{t-1} dO + k (u.dO)          (delta.rs:504-507)
    //   dk = dS u + S_{t-1} dsk                           (delta.rs:532-534, 556-558)
    //   dalpha = <dS, S_{t-1}> - beta du.sk               (delta.rs:530, 552)
    //   dbeta = du.(v - alpha sk)                         (delta.rs:549)
    float y = 0.0f;
#pragma unroll
    for (int n = 0; n < 4; ++n) y = fmaf(dO[n], u[n], y);
    float adO[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) adO[n] = a * dO[n];
    float pq[M], pk[M];
    float pa0 = 0.0f, pa1 = 0.0f;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float xq = in.k[m] * y, xk = 0.0f;
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            xq = fmaf(sm[m][n], adO[n], xq);
            xk = fmaf(u[n], ds[m][n], xk);
            xk = fmaf(dsk[n], sm[m][n], xk);
        }
        pq[m] = xq;
        pk[m] = xk;
        pa0 = fmaf(ds[m][0], sm[m][0], pa0);
        pa1 = fmaf(ds[m][1], sm[m][1], pa1);
        pa0 = fmaf(ds[m][2], sm[m][2], pa0);
        pa1 = fmaf(ds[m][3], sm[m][3], pa1);
    }
    float ea = 0.0f, eb = 0.0f;
#pragma unroll
    for (int n = 0; n < 4; ++n) {
        ea = fmaf(-bb * du[n], sk[n], ea);
        eb = fmaf(du[n], wv[n], eb);
    }
    float pa = pa0 + pa1 + (rg == 0 ? ea : 0.0f);
    float pb = rg == 0 ? eb : 0.0f;

    // dS <- alpha dS + k dsk^T  (delta.rs:543-545, 559-563)
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int n = 0; n < 4; ++n) ds[m][n] = a * ds[m][n] + in.k[m] * dsk[n];

    // Column sums of pq, pk over the 4 column groups (lane bits 4,5),
    // transposed so each lane keeps whole-row sums.
    float* rq = red_q + (jj * W + w) * DH;
    float* rk = red_k + (jj * W + w) * DH;
    if constexpr (M == 1) {
        const float zq = add_xor16(add_xor32(pq[0]));
        const float zk = add_xor16(add_xor32(pk[0]));
        if (cg == 0) { rq[rowb] = zq; rk[rowb] = zk; }
    } else if constexpr (M == 2) {
        const float zq = add_xor16(tsum32(pq[0], pq[1]));
        const float zk = add_xor16(tsum32(pk[0], pk[1]));
        if ((cg & 1) == 0) { rq[rowb + (cg >> 1)] = zq; rk[rowb + (cg >> 1)] = zk; }
    } else if constexpr (M == 4) {
        rq[rowb + cg] = tsum16(tsum32(pq[0], pq[2]), tsum32(pq[1], pq[3]));
        rk[rowb + cg] = tsum16(tsum32(pk[0], pk[2]), tsum32(pk[1], pk[3]));
    } else {
        static_assert(M == 8, "unsupported tile");
        float yq[4], yk[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            yq[j] = tsum32(pq[j], pq[j + 4]);
            yk[j] = tsum32(pk[j], pk[j + 4]);
        }
        rq[rowb + 2 * cg] = tsum16(yq[0], yq[2]);
        rq[rowb + 2 * cg + 1] = tsum16(yq[1], yq[3]);
        rk[rowb + 2 * cg] = tsum16(yk[0], yk[2]);
        rk[rowb + 2 * cg + 1] = tsum16(yk[1], yk[3]);
    }
    pa = wave_sum(pa);
    pb = wave_sum(pb);
    if (lane == 0) {
        red_ab[(jj * W + w) * 2 + 0] = pa;
        red_ab[(jj * W + w) * 2 + 1] = pb;
    }
}

// Staged inputs of one segment, loaded one segment ahead into registers.
template <int DH>
struct Stage {
    static constexpr int CK = DS<DH>::CK, NT = DS<DH>::THREADS, M = DS<DH>::M;
    static constexpr int QK4 = CK * DH / 4;             // float4 per staged tensor (q or k)
    static constexpr int NQ = (2 * QK4 + NT - 1) / NT;  // staged q/k float4 per thread
    static constexpr int W4 = CK * 12;                  // per-wave float4 of dO, v, sk
    static constexpr int NW = (W4 + 63) / 64;
    float4 rq[NQ], rw[NW];
    float rab;
    float rck[4][M];  // checkpoint tile: column colb+n, rows rowb..rowb+M-1
};

template <int DH, bool EXACT>
ASCA_DEV void stage_load(Stage<DH>& st, int g, const float* __restrict__ q, const float* __restrict__ k,
                         const float* __restrict__ v, const float* __restrict__ d_o,
                         const float* __restrict__ skv, const float* __restrict__ alpha,
                         const float* __restrict__ beta, const float* __restrict__ ckb, long ubase, long gbase,
                         long d, long dh2, int T, int H, int dh, int w, int lane, int rowb, int colb) {
    using SG = Stage<DH>;
    constexpr int CK = SG::CK, M = SG::M;
    const int t0 = g * CK;
#pragma unroll
    for (int i = 0; i < SG::NQ; ++i) {
        const int f0 = (int)threadIdx.x + i * SG::NT;
        const int f = f0 < 2 * SG::QK4 ? f0 : 0;
        const int tsr = f >= SG::QK4;
        const int fl = f - tsr * SG::QK4;
        const int j = fl / (DH / 4), c4 = fl % (DH / 4);
        const long t = min(t0 + j, T - 1);
        st.rq[i] = ld4m<EXACT>((tsr ? k : q) + ubase + t * d, 4 * c4, dh);
    }
#pragma unroll
    for (int i = 0; i < SG::NW; ++i) {
        const int f0 = lane + 64 * i;
        const int f = f0 < SG::W4 ? f0 : 0;
        const int tsr = f / (CK * 4);
        const int rem = f % (CK * 4);
        const int j = rem / 4, part = rem % 4;
        const long t = min(t0 + j, T - 1);
        const float* src = tsr == 0 ? d_o : (tsr == 1 ? v : skv);
        st.rw[i] = ld4m<EXACT>(src + ubase + t * d, w * 16 + part * 4, dh);
    }
    {
        const int gl = lane & (2 * CK - 1);
        const long t = min(t0 + gl % CK, T - 1);
        st.rab = (gl < CK ? alpha : beta)[gbase + t * H];
    }
    const float* cks = ckb + (long)g * dh2;
#pragma unroll
    for (int n = 0; n < 4; ++n) {
        const int i = colb + n;
        if constexpr (EXACT && M % 4 == 0) {
#pragma unroll
            for (int m = 0; m < M; m += 4) {
                const float4 x = *reinterpret_cast<const float4*>(cks + (long)i * dh + rowb + m);
                st.rck[n][m] = x.x; st.rck[n][m + 1] = x.y; st.rck[n][m + 2] = x.z; st.rck[n][m + 3] = x.w;
            }
        } else {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const bool ok = i < dh && rowb + m < dh;
                const float x = cks[ok ? (long)i * dh + rowb + m : 0];
                st.rck[n][m] = ok ? x : 0.0f;
            }
        }
    }
}

template <int DH>
ASCA_DEV void stage_store(const Stage<DH>& st, float* __restrict__ st_q, float* __restrict__ st_k,
                          float* __restrict__ st_w, float* __restrict__ st_ab, int w, int lane) {
    using SG = Stage<DH>;
    constexpr int CK = SG::CK;
#pragma unroll
    for (int i = 0; i < SG::NQ; ++i) {
        const int f = (int)threadIdx.x + i * SG::NT;
        if (f < 2 * SG::QK4) {
            const int tsr = f >= SG::QK4;
            const int fl = f - tsr * SG::QK4;
            const int j = fl / (DH / 4), c4 = fl % (DH / 4);
            *reinterpret_cast<float4*>((tsr ? st_k : st_q) + j * DH + 4 * c4) = st.rq[i];
        }
    }
#pragma unroll
    for (int i = 0; i < SG::NW; ++i) {
        const int f = lane + 64 * i;
        if (f < SG::W4) {
            const int tsr = f / (CK * 4);
            const int rem = f % (CK * 4);
            const int j = rem / 4, part = rem % 4;
            *reinterpret_cast<float4*>(st_w + ((w * CK + j) * 3 + tsr) * 16 + part * 4) = st.rw[i];
        }
    }
    if (w == 0 && lane < 2 * CK) st_ab[lane] = st.rab;
}

// Backward of one unit per block.  Output pointers are already offset to the
// head-0 column of their quantity; element (r, h*dh + i) is at ptr[r*ldx + h*dh + i]
// and the per-head scalars at ga[r*ldg + h].  FUSED applies the L2-norm backward
// (rust/src/delta.rs:677-698) and the sigmoid backward (delta.rs:602-611).
template <int DH, bool EXACT, bool FUSED>
__global__ __launch_bounds__(DS<DH>::THREADS) void delta_bwd_k(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ alpha, const float* __restrict__ beta, const float* __restrict__ d_o,
    const float* __restrict__ skv, const float* __restrict__ ckpt, const float* __restrict__ qnorm,
    const float* __restrict__ knorm, float* __restrict__ gq, float* __restrict__ gk,
    float* __restrict__ gv, long ldx, float* __restrict__ ga, float* __restrict__ gb, long ldg, int B,
    int T, int H, int dh, int nslots) {
    using S = DS<DH>;
    constexpr int M = S::M, W = S::W, CK = S::CK;

    extern __shared__ float4 lds4[];
    float4* stash = lds4;                                            // [CK][W][M][64]
    float* red_q = reinterpret_cast<float*>(lds4 + S::STASH_F4);     // [CK][W][DH]
    float* red_k = red_q + S::RED_F;                                 // [CK][W][DH]
    float* red_ab = red_k + S::RED_F;                                // [CK][W][2]
    float* st_q = red_ab + S::RAB_F;                                 // [CK][DH]
    float* st_k = st_q + S::STQK_F;                                  // [CK][DH]
    float* st_w = st_k + S::STQK_F;                                  // [W][CK][3][16]
    float* st_ab = st_w + S::STW_F;                                  // [2][CK]

    const int unit = blockIdx.x;
    const int h = unit / B, b = unit - h * B;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int rg = lane & 15, cg = lane >> 4;
    const int colb = w * 16 + cg * 4;
    const int rowb = rg * M;
    const long d = (long)H * dh;
    const long dh2 = (long)dh * dh;
    const long ubase = (long)b * T * d + (long)h * dh;
    const long gbase = (long)b * T * H + h;
    const long hoff = (long)h * dh;
    const float* ckb = ckpt + (long)unit * nslots * dh2;
    const int nseg = (T + CK - 1) / CK;
    float* const tr = trash_f(threadIdx.x * 4);

    float ds[M][4];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int n = 0; n < 4; ++n) ds[m][n] = 0.0f;

    Stage<DH> stg;
    stage_load<DH, EXACT>(stg, nseg - 1, q, k, v, d_o, skv, alpha, beta, ckb, ubase, gbase, d, dh2, T, H, dh, w, lane,
                          rowb, colb);
    for (int g = nseg - 1; g >= 0; --g) {
        const int t0 = g * CK;
        const int len = min(CK, T - t0);
        float s[M][4];
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int n = 0; n < 4; ++n) s[m][n] = stg.rck[n][m];
        stage_store<DH>(stg, st_q, st_k, st_w, st_ab, w, lane);
        stage_load<DH, EXACT>(stg, g > 0 ? g - 1 : 0, q, k, v, d_o, skv, alpha, beta, ckb, ubase, gbase, d, dh2, T,
                              H, dh, w, lane, rowb, colb);
        __syncthreads();  // staging visible; every wave is past the previous epilogue

        // ---- phase A: stash S_{t0} .. S_{t0+len-1}
#pragma unroll
        for (int m = 0; m < M; ++m)
            stash[((0 * W + w) * M + m) * 64 + lane] = make_float4(s[m][0], s[m][1], s[m][2], s[m][3]);
        for (int j = 1; j < len; ++j) {
            const int jp = j - 1;
            float km[M];
#pragma unroll
            for (int m = 0; m < M; ++m) km[m] = st_k[jp * DH + rowb + m];
            const float* sw = st_w + (w * CK + jp) * 48 + cg * 4;
            const float4 vv = *reinterpret_cast<const float4*>(sw + 16);
            const float4 sk = *reinterpret_cast<const float4*>(sw + 32);
            const float a = st_ab[jp], bt = st_ab[CK + jp];
            const float u[4] = {bt * (vv.x - a * sk.x), bt * (vv.y - a * sk.y), bt * (vv.z - a * sk.z),
                                bt * (vv.w - a * sk.w)};
#pragma unroll
            for (int m = 0; m < M; ++m) {
#pragma unroll
                for (int n = 0; n < 4; ++n) s[m][n] = a * s[m][n] + km[m] * u[n];
                stash[((j * W + w) * M + m) * 64 + lane] = make_float4(s[m][0], s[m][1], s[m][2], s[m][3]);
            }
        }

        // ---- phase B: steps t0+len-1 .. t0 in reverse, operands prefetched one step ahead
        {
            BOps<M> opA, opB;
            lds_ops<DH>(opA, stash, st_q, st_k, st_w, st_ab, len - 1, w, lane, rowb, cg);
            for (int jj = len - 1; jj >= 0; jj -= 2) {
                lds_ops<DH>(opB, stash, st_q, st_k, st_w, st_ab, jj > 0 ? jj - 1 : 0, w, lane, rowb, cg);
                bwd_step<DH, EXACT>(opA, ds, red_q, red_k, red_ab, gv + ((long)b * T + t0 + jj) * ldx + hoff + colb,
                                    tr, jj, w, lane, rg, cg, rowb, colb, dh);
                if (jj == 0) break;
                lds_ops<DH>(opA, stash, st_q, st_k, st_w, st_ab, jj > 1 ? jj - 2 : 0, w, lane, rowb, cg);
                bwd_step<DH, EXACT>(opB, ds, red_q, red_k, red_ab,
                                    gv + ((long)b * T + t0 + jj - 1) * ldx + hoff + colb, tr, jj - 1, w, lane, rg,
                                    cg, rowb, colb, dh);
            }
        }
        __syncthreads();  // red_* of this segment complete

        // ---- phase C: cross-wave sums, optional norm/sigmoid backward, stores
        constexpr int NA = (DH + 63) / 64;
        for (int jj = w; jj < len; jj += W) {
            const long r = (long)b * T + t0 + jj;
            float dq[NA], dk[NA], qa[NA], ka[NA];
            float dotq = 0.0f, dotk = 0.0f;
#pragma unroll
            for (int ia = 0; ia < NA; ++ia) {
                const int a = lane + 64 * ia;
                dq[ia] = 0.0f;
                dk[ia] = 0.0f;
                qa[ia] = 0.0f;
                ka[ia] = 0.0f;
                if (a < DH) {
#pragma unroll
                    for (int w2 = 0; w2 < W; ++w2) {
                        dq[ia] += red_q[(jj * W + w2) * DH + a];
                        dk[ia] += red_k[(jj * W + w2) * DH + a];
                    }
                    if (FUSED) {
                        qa[ia] = st_q[jj * DH + a];
                        ka[ia] = st_k[jj * DH + a];
                    }
                }
                dotq = fmaf(qa[ia], dq[ia], dotq);
                dotk = fmaf(ka[ia], dk[ia], dotk);
            }
            float dA = 0.0f, dB = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < W; ++w2) {
                dA += red_ab[(jj * W + w2) * 2 + 0];
                dB += red_ab[(jj * W + w2) * 2 + 1];
            }
            if constexpr (FUSED) {
                dotq = wave_sum(dotq);
                dotk = wave_sum(dotk);
                const float qn = qnorm[r * H + h], kn = knorm[r * H + h];
#pragma unroll
                for (int ia = 0; ia < NA; ++ia) {
                    const int a = lane + 64 * ia;
                    if (a < dh) {
                        gq[r * ldx + hoff + a] = (dq[ia] - qa[ia] * dotq) / qn;
                        gk[r * ldx + hoff + a] = (dk[ia] - ka[ia] * dotk) / kn;
                    }
                }
                if (lane == 0) {
                    const float al = st_ab[jj], be = st_ab[CK + jj];
                    ga[r * ldg + h] = dA * al * (1.0f - al);
                    gb[r * ldg + h] = dB * be * (1.0f - be);
                }
            } else {
#pragma unroll
                for (int ia = 0; ia < NA; ++ia) {
                    const int a = lane + 64 * ia;
                    if (a < dh) {
                        gq[r * ldx + hoff + a] = dq[ia];
                        gk[r * ldx + hoff + a] = dk[ia];
                    }
                }
                if (lane == 0) {
                    ga[r * ldg + h] = dA;
                    gb[r * ldg + h] = dB;
                }
            }
        }
        __syncthreads();  // staging and red_* free for the next segment
    }
}

// ------------------------------------------------------------------- host

static int dh_class(int dh) {
    if (dh <= 0) return 0;
    if (dh <= 16) return 16;
    if (dh <= 32) return 32;
    if (dh <= 64) return 64;
    if (dh <= 128) return 128;
    return 0;
}

static int ck_for(int dhc) {
    switch (dhc) {
        case 16: return DS<16>::CK;
        case 32: return DS<32>::CK;
        case 64: return DS<64>::CK;
        default: return DS<128>::CK;
    }
}

struct DeltaWs {
    float* sk;
    float* ckpt;
    int ck;
    int nslots;
    size_t bytes;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static DeltaWs ws_layout(int B, int T, int H, int dh, void* base) {
    DeltaWs w;
    const int dhc = dh_class(dh);
    w.ck = ck_for(dhc);
    w.nslots = (T + w.ck - 1) / w.ck;
    const size_t sk_bytes = align256((size_t)B * T * H * dh * sizeof(float));
    const size_t ck_bytes = align256((size_t)B * H * w.nslots * dh * dh * sizeof(float));
    w.sk = reinterpret_cast<float*>(base);
    w.ckpt = base ? reinterpret_cast<float*>(reinterpret_cast<char*>(base) + sk_bytes) : nullptr;
    w.bytes = sk_bytes + ck_bytes;
    return w;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

static int check_shape(int B, int T, int H, int dh) {
    if (B < 0 || T < 0 || H < 0) return fail(ASCA_ERR_INVALID, "negative shape B=%d T=%d H=%d", B, T, H);
    if (!dh_class(dh)) return fail(ASCA_ERR_UNSUPPORTED, "dh=%d outside 1..128", dh);
    if ((long)B * H > 0x7fffffffL) return fail(ASCA_ERR_INVALID, "B*H too large");
    return ASCA_OK;
}

template <int DH, bool EXACT>
static int launch_fwd_t(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                        float* o, const DeltaWs& ws, int B, int T, int H, int dh, hipStream_t st) {
    int rc = pre_launch("delta_fwd");
    if (rc) return rc;
    hipLaunchKernelGGL((delta_fwd_k<DH, EXACT>), dim3(B * H), dim3(DS<DH>::THREADS), 0, st, q, k, v, alpha, beta, o,
                       ws.sk, ws.ckpt, B, T, H, dh, ws.nslots);
    return post_launch("delta_fwd");
}

static int launch_fwd(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                      float* o, const DeltaWs& ws, int B, int T, int H, int dh, hipStream_t st) {
    const int dhc = dh_class(dh);
    const bool exact = dh == dhc && aligned16(q) && aligned16(k);
#define ASCA_FWD(DHC)                                                                                    \
    if (dhc == DHC)                                                                                      \
        return exact ? launch_fwd_t<DHC, true>(q, k, v, alpha, beta, o, ws, B, T, H, dh, st)             \
                     : launch_fwd_t<DHC, false>(q, k, v, alpha, beta, o, ws, B, T, H, dh, st);
    ASCA_FWD(16)
    ASCA_FWD(32)
    ASCA_FWD(64)
    ASCA_FWD(128)
#undef ASCA_FWD
    return fail(ASCA_ERR_UNSUPPORTED, "dh=%d", dh);
}

template <int DH>
static int launch_states_t(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                           float* states, int B, int T, int H, int dh, hipStream_t st) {
    int rc = pre_launch("delta_states");
    if (rc) return rc;
    hipLaunchKernelGGL((delta_states_k<DH>), dim3(B * H), dim3(DS<DH>::THREADS), 0, st, q, k, v, alpha, beta,
                       states, B, T, H, dh);
    return post_launch("delta_states");
}

template <int DH, bool EXACT, bool FUSED>
static int launch_bwd_t(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                        const float* d_o, const DeltaWs& ws, const float* qn, const float* kn, float* gq, float* gk,
                        float* gv, long ldx, float* ga, float* gb, long ldg, int B, int T, int H, int dh,
                        hipStream_t st) {
    static bool attr = false;
    const size_t lds = DS<DH>::LDS_BWD;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&delta_bwd_k<DH, EXACT, FUSED>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipFuncSetAttribute(LDS %zu): %s", lds, hipGetErrorString(e));
        attr = true;
    }
    int rc = pre_launch("delta_bwd");
    if (rc) return rc;
    hipLaunchKernelGGL((delta_bwd_k<DH, EXACT, FUSED>), dim3(B * H), dim3(DS<DH>::THREADS), lds, st, q, k, v, alpha,
                       beta, d_o, ws.sk, ws.ckpt, qn, kn, gq, gk, gv, ldx, ga, gb, ldg, B, T, H, dh, ws.nslots);
    return post_launch("delta_bwd");
}

template <bool FUSED>
static int launch_bwd(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                      const float* d_o, const DeltaWs& ws, const float* qn, const float* kn, float* gq, float* gk,
                      float* gv, long ldx, float* ga, float* gb, long ldg, int B, int T, int H, int dh,
                      hipStream_t st) {
    const int dhc = dh_class(dh);
    const bool exact = dh == dhc && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(d_o) &&
                       aligned16(gv) && ((ldx * 4) % 16 == 0);
#define ASCA_BWD(DHC)                                                                                            \
    if (dhc == DHC)                                                                                              \
        return exact ? launch_bwd_t<DHC, true, FUSED>(q, k, v, alpha, beta, d_o, ws, qn, kn, gq, gk, gv, ldx, ga, \
                                                      gb, ldg, B, T, H, dh, st)                                  \
                     : launch_bwd_t<DHC, false, FUSED>(q, k, v, alpha, beta, d_o, ws, qn, kn, gq, gk, gv, ldx,   \
                                                       ga, gb, ldg, B, T, H, dh, st);
    ASCA_BWD(16)
    ASCA_BWD(32)
    ASCA_BWD(64)
    ASCA_BWD(128)
#undef ASCA_BWD
    return fail(ASCA_ERR_UNSUPPORTED, "dh=%d", dh);
}

}  // namespace asca

using namespace asca;

extern "C" {

int asca_delta_ws_bytes(int B, int T, int H, int dh, size_t* bytes) {
    if (!bytes) return fail(ASCA_ERR_INVALID, "null output pointer");
    int rc = check_shape(B, T, H, dh);
    if (rc) return rc;
    *bytes = ws_layout(B, T, H, dh, nullptr).bytes;
    return ASCA_OK;
}

int asca_delta_fwd(const float* q, const float* k, const float* v, const float* alpha, const float* beta, float* o,
                   void* ws, int B, int T, int H, int dh, void* stream) {
    int rc = check_shape(B, T, H, dh);
    if (rc) return rc;
    if ((long)B * T * H == 0) return ASCA_OK;
    if (!q || !k || !v || !alpha || !beta || !o || !ws) return fail(ASCA_ERR_INVALID, "null pointer in asca_delta_fwd");
    DeltaWs w = ws_layout(B, T, H, dh, ws);
    return launch_fwd(q, k, v, alpha, beta, o, w, B, T, H, dh, as_stream(stream));
}

int asca_delta_bwd_raw(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                       const float* d_o, const void* ws, float* dq, float* dk, float* dv, float* dalpha,
                       float* dbeta, int B, int T, int H, int dh, void* stream) {
    int rc = check_shape(B, T, H, dh);
    if (rc) return rc;
    if ((long)B * T * H == 0) return ASCA_OK;
    if (!q || !k || !v || !alpha || !beta || !d_o || !ws || !dq || !dk || !dv || !dalpha || !dbeta)
        return fail(ASCA_ERR_INVALID, "null pointer in asca_delta_bwd_raw");
    DeltaWs w = ws_layout(B, T, H, dh, const_cast<void*>(ws));
    const long d = (long)H * dh;
    return launch_bwd<false>(q, k, v, alpha, beta, d_o, w, nullptr, nullptr, dq, dk, dv, d, dalpha, dbeta, H, B, T,
                             H, dh, as_stream(stream));
}

int asca_delta_bwd_fused(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                         const float* qnorm, const float* knorm, const float* d_o, const void* ws, float* d_qkv,
                         float* d_gate, int B, int T, int H, int dh, void* stream) {
    int rc = check_shape(B, T, H, dh);
    if (rc) return rc;
    if ((long)B * T * H == 0) return ASCA_OK;
    if (!q || !k || !v || !alpha || !beta || !qnorm || !knorm || !d_o || !ws || !d_qkv || !d_gate)
        return fail(ASCA_ERR_INVALID, "null pointer in asca_delta_bwd_fused");
    DeltaWs w = ws_layout(B, T, H, dh, const_cast<void*>(ws));
    const long d = (long)H * dh;
    return launch_bwd<true>(q, k, v, alpha, beta, d_o, w, qnorm, knorm, d_qkv, d_qkv + d, d_qkv + 2 * d, 3 * d,
                            d_gate, d_gate + H, 2L * H, B, T, H, dh, as_stream(stream));
}

int asca_delta_states(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                      float* states, int B, int T, int H, int dh, void* stream) {
    int rc = check_shape(B, T, H, dh);
    if (rc) return rc;
    if ((long)B * H == 0) return ASCA_OK;
    if (!states) return fail(ASCA_ERR_INVALID, "null states pointer");
    if (T > 0 && (!q || !k || !v || !alpha || !beta))
        return fail(ASCA_ERR_INVALID, "null pointer in asca_delta_states");
    const hipStream_t st = as_stream(stream);
    switch (dh_class(dh)) {
        case 16: return launch_states_t<16>(q, k, v, alpha, beta, states, B, T, H, dh, st);
        case 32: return launch_states_t<32>(q, k, v, alpha, beta, states, B, T, H, dh, st);
        case 64: return launch_states_t<64>(q, k, v, alpha, beta, states, B, T, H, dh, st);
        default: return launch_states_t<128>(q, k, v, alpha, beta, states, B, T, H, dh, st);
    }
}

}  // extern "C"
