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
//    butterflies.  No LDS, no barrier in the forward.
//  * The forward stores S every C steps ("checkpoints", C = 8 at dh = 64) and
//    the per-step sk vector instead of the reference's full (T+1) dh^2 history
//    (2.15 GB at B32 T512 H8 dh64).
//  * The backward recomputes each C-step segment from its checkpoint into an
//    LDS stash, then walks it in reverse.  A lane there owns a (dh/16) x 4 tile:
//    row contractions (du = dS^T k) are 16-lane DPP butterflies inside a row,
//    column contractions (dq, dk) are transposed permlane32/permlane16 swaps
//    across rows plus a per-segment cross-wave sum through LDS.  The L2-norm
//    and sigmoid backward of the drop-in variant run in that epilogue.
#include "common.h"
#include "runtime.h"

namespace asca {

template <int DH>
struct DS {
    static constexpr int W = DH / 16;        // waves per unit, 16 value columns each
    static constexpr int THREADS = 64 * W;
    static constexpr int R = DH / 4;         // forward: rows per lane (4 lanes / column)
    static constexpr int M = DH / 16;        // backward: rows per lane (16 row groups)
    // Checkpoint interval: C states of the backward's LDS stash fill 128 KB.
    static constexpr int CK = (DH == 16) ? 64 : (DH == 32) ? 32 : (DH == 64) ? 8 : 2;
    static constexpr int PF = (DH == 128) ? 2 : 4;   // forward prefetch depth (steps)
    static constexpr size_t LDS_BWD =
        (size_t)CK * W * M * 64 * 16 + 2 * (size_t)CK * W * DH * 4 + (size_t)CK * W * 2 * 4;
};

// ------------------------------------------------------------------ forward

template <int DH>
struct FwdIn {
    float k[DH / 4];
    float q[DH / 4];
    float v, a, b;
};

template <int DH, bool EXACT>
ASCA_DEV void fwd_load(FwdIn<DH>& in, const float* __restrict__ q, const float* __restrict__ k,
                       const float* __restrict__ v, const float* __restrict__ alpha,
                       const float* __restrict__ beta, long base, long gi, int row0, int col, int dh) {
    constexpr int R = DH / 4;
    if constexpr (EXACT) {
#pragma unroll
        for (int j = 0; j < R; j += 4) {
            float4 kv = *reinterpret_cast<const float4*>(k + base + row0 + j);
            float4 qv = *reinterpret_cast<const float4*>(q + base + row0 + j);
            in.k[j] = kv.x; in.k[j + 1] = kv.y; in.k[j + 2] = kv.z; in.k[j + 3] = kv.w;
            in.q[j] = qv.x; in.q[j + 1] = qv.y; in.q[j + 2] = qv.z; in.q[j + 3] = qv.w;
        }
        in.v = v[base + col];
    } else {
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const int a = row0 + j;
            in.k[j] = a < dh ? k[base + a] : 0.0f;
            in.q[j] = a < dh ? q[base + a] : 0.0f;
        }
        in.v = col < dh ? v[base + col] : 0.0f;
    }
    in.a = alpha[gi];
    in.b = beta[gi];
}

// One block per (sequence, head) unit, unit = h*B + b (the reference's s_pre
// order, rust/src/delta.rs:54-56).  ckpt: nslots states of dh*dh per unit, slot
// j holding S before step j*ck; when T % ck == 0 and nslots > T/ck the final
// state goes to slot T/ck.  o / sk_out may be null.
template <int DH, bool EXACT>
__global__ __launch_bounds__(DS<DH>::THREADS) void delta_fwd_k(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ alpha, const float* __restrict__ beta, float* __restrict__ o,
    float* __restrict__ sk_out, float* __restrict__ ckpt, int B, int T, int H, int dh, int ck,
    int nslots) {
    constexpr int R = DS<DH>::R;
    constexpr int PF = DS<DH>::PF;
    const int unit = blockIdx.x;
    const int h = unit / B, b = unit - h * B;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int p = lane & 3, c = lane >> 2;
    const int col = w * 16 + c;
    const int row0 = p * R;
    const long d = (long)H * dh;
    const long dh2 = (long)dh * dh;
    const bool col_ok = EXACT || col < dh;
    float* ckb = ckpt ? ckpt + (long)unit * nslots * dh2 : nullptr;

    float s[R];
#pragma unroll
    for (int j = 0; j < R; ++j) s[j] = 0.0f;

    FwdIn<DH> buf[PF];
#pragma unroll
    for (int i = 0; i < PF - 1; ++i)
        if (i < T) {
            const long r = (long)b * T + i;
            fwd_load<DH, EXACT>(buf[i], q, k, v, alpha, beta, r * d + (long)h * dh, r * H + h, row0, col, dh);
        }

    int ckc = 0, slot = 0;
    for (int t0 = 0; t0 < T; t0 += PF) {
#pragma unroll
        for (int jj = 0; jj < PF; ++jj) {
            const int t = t0 + jj;
            if (t < T) {
                const int tl = t + PF - 1;
                if (tl < T) {
                    const long rl = (long)b * T + tl;
                    fwd_load<DH, EXACT>(buf[(jj + PF - 1) % PF], q, k, v, alpha, beta, rl * d + (long)h * dh,
                                        rl * H + h, row0, col, dh);
                }
                if (ckb && ckc == 0) {
                    float* dst = ckb + (long)slot * dh2;
#pragma unroll
                    for (int j = 0; j < R; ++j)
                        if (EXACT || (row0 + j < dh && col_ok)) dst[(long)(row0 + j) * dh + col] = s[j];
                    ++slot;
                }
                if (++ckc == ck) ckc = 0;

                const FwdIn<DH>& in = buf[jj];
                const long base = ((long)b * T + t) * d + (long)h * dh;
                float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
                for (int j = 0; j < R; j += 2) {
                    a0 = fmaf(s[j], in.k[j], a0);
                    a1 = fmaf(s[j + 1], in.k[j + 1], a1);
                }
                const float sk = group_sum<4>(a0 + a1);
                const float u = in.b * (in.v - in.a * sk);
                float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
                for (int j = 0; j < R; j += 2) {
                    s[j] = in.a * s[j] + in.k[j] * u;
                    s[j + 1] = in.a * s[j + 1] + in.k[j + 1] * u;
                    o0 = fmaf(s[j], in.q[j], o0);
                    o1 = fmaf(s[j + 1], in.q[j + 1], o1);
                }
                const float oo = group_sum<4>(o0 + o1);
                if (p == 0 && col_ok) {
                    if (o) o[base + col] = oo;
                    if (sk_out) sk_out[base + col] = sk;
                }
            }
        }
    }
    if (ckb && T % ck == 0 && slot < nslots) {
        float* dst = ckb + (long)slot * dh2;
#pragma unroll
        for (int j = 0; j < R; ++j)
            if (EXACT || (row0 + j < dh && col_ok)) dst[(long)(row0 + j) * dh + col] = s[j];
    }
}

// ----------------------------------------------------------------- backward

template <bool EXACT>
ASCA_DEV float4 ld4(const float* __restrict__ p, long off, int col, int dh) {
    if constexpr (EXACT) {
        return *reinterpret_cast<const float4*>(p + off + col);
    } else {
        float4 r;
        r.x = col < dh ? p[off + col] : 0.0f;
        r.y = col + 1 < dh ? p[off + col + 1] : 0.0f;
        r.z = col + 2 < dh ? p[off + col + 2] : 0.0f;
        r.w = col + 3 < dh ? p[off + col + 3] : 0.0f;
        return r;
    }
}

template <int M, bool EXACT>
ASCA_DEV void ldrows(float (&x)[M], const float* __restrict__ p, long off, int row, int dh) {
    if constexpr (EXACT && M % 4 == 0) {
#pragma unroll
        for (int m = 0; m < M; m += 4) {
            float4 t = *reinterpret_cast<const float4*>(p + off + row + m);
            x[m] = t.x; x[m + 1] = t.y; x[m + 2] = t.z; x[m + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int m = 0; m < M; ++m) x[m] = (EXACT || row + m < dh) ? p[off + row + m] : 0.0f;
    }
}

template <bool EXACT>
ASCA_DEV void st4(float* __restrict__ p, long off, int col, int dh, float4 v) {
    if constexpr (EXACT) {
        *reinterpret_cast<float4*>(p + off + col) = v;
    } else {
        if (col < dh) p[off + col] = v.x;
        if (col + 1 < dh) p[off + col + 1] = v.y;
        if (col + 2 < dh) p[off + col + 2] = v.z;
        if (col + 3 < dh) p[off + col + 3] = v.w;
    }
}

template <int M>
struct BwdIn {
    float q[M], k[M];
    float4 dO, v, sk;
    float a, b;
};

template <int DH, bool EXACT>
ASCA_DEV void bwd_load(BwdIn<DH / 16>& in, const float* __restrict__ q, const float* __restrict__ k,
                       const float* __restrict__ v, const float* __restrict__ alpha,
                       const float* __restrict__ beta, const float* __restrict__ d_o,
                       const float* __restrict__ skv, long base, long gi, int rowb, int colb, int dh) {
    constexpr int M = DH / 16;
    ldrows<M, EXACT>(in.q, q, base, rowb, dh);
    ldrows<M, EXACT>(in.k, k, base, rowb, dh);
    in.dO = ld4<EXACT>(d_o, base, colb, dh);
    in.v = ld4<EXACT>(v, base, colb, dh);
    in.sk = ld4<EXACT>(skv, base, colb, dh);
    in.a = alpha[gi];
    in.b = beta[gi];
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
    float4* stash = lds4;                                                 // [CK][W][M][64]
    float* red_q = reinterpret_cast<float*>(lds4 + (size_t)CK * W * M * 64);  // [CK][W][DH]
    float* red_k = red_q + CK * W * DH;                                   // [CK][W][DH]
    float* red_ab = red_k + CK * W * DH;                                  // [CK][W][2]

    const int unit = blockIdx.x;
    const int h = unit / B, b = unit - h * B;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int rg = lane & 15, cg = lane >> 4;
    const int colb = w * 16 + cg * 4;
    const int rowb = rg * M;
    const long d = (long)H * dh;
    const long dh2 = (long)dh * dh;
    const float* ckb = ckpt + (long)unit * nslots * dh2;
    const int nseg = (T + CK - 1) / CK;
    const long hoff = (long)h * dh;

    float ds[M][4];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int n = 0; n < 4; ++n) ds[m][n] = 0.0f;

    for (int g = nseg - 1; g >= 0; --g) {
        const int t0 = g * CK;
        const int len = min(CK, T - t0);

        // ---- phase A: S_{t0} from its checkpoint, then S_{t0+1..t0+len-1}
        {
            float s[M][4];
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const int a = rowb + m;
                float4 t4 = (EXACT || a < dh) ? ld4<EXACT>(ckb, (long)g * dh2 + (long)a * dh, colb, dh)
                                              : make_float4(0.f, 0.f, 0.f, 0.f);
                s[m][0] = t4.x; s[m][1] = t4.y; s[m][2] = t4.z; s[m][3] = t4.w;
                stash[((0 * W + w) * M + m) * 64 + lane] = t4;
            }
            float kc[M], kn[M];
            float4 vc, skc, vn4, skn4;
            float ac = 0.f, bc = 0.f, an = 0.f, bn = 0.f;
            if (len > 1) {
                const long r = (long)b * T + t0;
                ldrows<M, EXACT>(kc, k, r * d + hoff, rowb, dh);
                vc = ld4<EXACT>(v, r * d + hoff, colb, dh);
                skc = ld4<EXACT>(skv, r * d + hoff, colb, dh);
                ac = alpha[r * H + h];
                bc = beta[r * H + h];
            }
            for (int j = 1; j < len; ++j) {
                if (j + 1 < len) {
                    const long r = (long)b * T + t0 + j;
                    ldrows<M, EXACT>(kn, k, r * d + hoff, rowb, dh);
                    vn4 = ld4<EXACT>(v, r * d + hoff, colb, dh);
                    skn4 = ld4<EXACT>(skv, r * d + hoff, colb, dh);
                    an = alpha[r * H + h];
                    bn = beta[r * H + h];
                }
                float u[4];
                u[0] = bc * (vc.x - ac * skc.x);
                u[1] = bc * (vc.y - ac * skc.y);
                u[2] = bc * (vc.z - ac * skc.z);
                u[3] = bc * (vc.w - ac * skc.w);
#pragma unroll
                for (int m = 0; m < M; ++m) {
#pragma unroll
                    for (int n = 0; n < 4; ++n) s[m][n] = ac * s[m][n] + kc[m] * u[n];
                    stash[((j * W + w) * M + m) * 64 + lane] = make_float4(s[m][0], s[m][1], s[m][2], s[m][3]);
                }
#pragma unroll
                for (int m = 0; m < M; ++m) kc[m] = kn[m];
                vc = vn4; skc = skn4; ac = an; bc = bn;
            }
        }
        __syncthreads();  // every wave is past the previous epilogue: red_* is free

        // ---- phase B: steps t0+len-1 .. t0 in reverse
        {
            BwdIn<M> cur, nxt;
            {
                const long r = (long)b * T + t0 + len - 1;
                bwd_load<DH, EXACT>(cur, q, k, v, alpha, beta, d_o, skv, r * d + hoff, r * H + h, rowb, colb, dh);
            }
            for (int jj = len - 1; jj >= 0; --jj) {
                if (jj > 0) {
                    const long r = (long)b * T + t0 + jj - 1;
                    bwd_load<DH, EXACT>(nxt, q, k, v, alpha, beta, d_o, skv, r * d + hoff, r * H + h, rowb, colb,
                                        dh);
                }
                const long r = (long)b * T + t0 + jj;
                float s[M][4];
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    float4 t4 = stash[((jj * W + w) * M + m) * 64 + lane];
                    s[m][0] = t4.x; s[m][1] = t4.y; s[m][2] = t4.z; s[m][3] = t4.w;
                }
                const float a = cur.a, bb = cur.b;
                const float dO[4] = {cur.dO.x, cur.dO.y, cur.dO.z, cur.dO.w};
                const float vv[4] = {cur.v.x, cur.v.y, cur.v.z, cur.v.w};
                const float sk[4] = {cur.sk.x, cur.sk.y, cur.sk.z, cur.sk.w};

                // dS += q dO^T  (delta.rs:508-511)
#pragma unroll
                for (int m = 0; m < M; ++m)
#pragma unroll
                    for (int n = 0; n < 4; ++n) ds[m][n] = fmaf(cur.q[m], dO[n], ds[m][n]);
                // du = dS^T k  (delta.rs:536-542): 16-lane butterfly over row groups
                float du[4];
#pragma unroll
                for (int n = 0; n < 4; ++n) {
                    float acc = 0.0f;
#pragma unroll
                    for (int m = 0; m < M; ++m) acc = fmaf(ds[m][n], cur.k[m], acc);
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
                // dv = beta du  (delta.rs:550)
                if (rg == 0)
                    st4<EXACT>(gv, r * ldx + hoff, colb, dh,
                               make_float4(bb * du[0], bb * du[1], bb * du[2], bb * du[3]));

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
                    float xq = cur.k[m] * y, xk = 0.0f;
#pragma unroll
                    for (int n = 0; n < 4; ++n) {
                        xq = fmaf(s[m][n], adO[n], xq);
                        xk = fmaf(u[n], ds[m][n], xk);
                        xk = fmaf(dsk[n], s[m][n], xk);
                    }
                    pq[m] = xq;
                    pk[m] = xk;
                    pa0 = fmaf(ds[m][0], s[m][0], pa0);
                    pa1 = fmaf(ds[m][1], s[m][1], pa1);
                    pa0 = fmaf(ds[m][2], s[m][2], pa0);
                    pa1 = fmaf(ds[m][3], s[m][3], pa1);
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
                    for (int n = 0; n < 4; ++n) ds[m][n] = a * ds[m][n] + cur.k[m] * dsk[n];

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
                    const float zq = tsum16(tsum32(pq[0], pq[2]), tsum32(pq[1], pq[3]));
                    const float zk = tsum16(tsum32(pk[0], pk[2]), tsum32(pk[1], pk[3]));
                    rq[rowb + cg] = zq;
                    rk[rowb + cg] = zk;
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
                if (jj > 0) cur = nxt;
            }
        }
        __syncthreads();  // red_* of this segment complete

        // ---- phase C: cross-wave sums, optional norm/sigmoid backward, stores
        constexpr int NA = (DH + 63) / 64;
        for (int jj = w; jj < len; jj += W) {
            const long r = (long)b * T + t0 + jj;
            const long base = r * d + hoff;
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
                    if (FUSED && (EXACT || a < dh)) {
                        qa[ia] = q[base + a];
                        ka[ia] = k[base + a];
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
                    const float al = alpha[r * H + h], be = beta[r * H + h];
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
                        float* o, float* sk, float* ckpt, int B, int T, int H, int dh, int ck, int nslots,
                        hipStream_t st) {
    int rc = pre_launch("delta_fwd");
    if (rc) return rc;
    hipLaunchKernelGGL((delta_fwd_k<DH, EXACT>), dim3(B * H), dim3(DS<DH>::THREADS), 0, st, q, k, v, alpha, beta, o,
                       sk, ckpt, B, T, H, dh, ck, nslots);
    return post_launch("delta_fwd");
}

static int launch_fwd(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                      float* o, float* sk, float* ckpt, int B, int T, int H, int dh, int ck, int nslots,
                      hipStream_t st) {
    const int dhc = dh_class(dh);
    const bool exact = dh == dhc && aligned16(q) && aligned16(k);
#define ASCA_FWD(DHC)                                                                                         \
    if (dhc == DHC)                                                                                           \
        return exact ? launch_fwd_t<DHC, true>(q, k, v, alpha, beta, o, sk, ckpt, B, T, H, dh, ck, nslots, st) \
                     : launch_fwd_t<DHC, false>(q, k, v, alpha, beta, o, sk, ckpt, B, T, H, dh, ck, nslots, st);
    ASCA_FWD(16)
    ASCA_FWD(32)
    ASCA_FWD(64)
    ASCA_FWD(128)
#undef ASCA_FWD
    return fail(ASCA_ERR_UNSUPPORTED, "dh=%d", dh);
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
    return launch_fwd(q, k, v, alpha, beta, o, w.sk, w.ckpt, B, T, H, dh, w.ck, w.nslots, as_stream(stream));
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
    if (T == 0) {
        return asca_memset32(states, 0u, (size_t)B * H * dh * dh, stream);
    }
    if (!q || !k || !v || !alpha || !beta) return fail(ASCA_ERR_INVALID, "null pointer in asca_delta_states");
    return launch_fwd(q, k, v, alpha, beta, nullptr, nullptr, states, B, T, H, dh, 1, T + 1, as_stream(stream));
}

}  // extern "C"
